// Host/device interface of the flash-attention kernels (flash_attn.hip) and the RoPE pass (rope.hip).
#pragma once
#include "common.hpp"

namespace samhip {

// Arguments of one flash-attention launch. Strides are in elements: [0] batch, [1] row (token),
// [2] head; the head dimension is contiguous.
struct FlashParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  long sq[3], sk[3], sv[3], so[3];
  int b, h, lq, lk, d;
  float sc;                    // scale * log2(e)
  float fscale;                // scale itself (the f32 kernel works in natural units, as the reference)
  int qblocks, nsplit, tps;    // query blocks, key splits, key tiles (of 64) per split
  float* opart;                // nsplit > 1: partial O [nsplit][b*h][lq][padded d]: f16 O / sum, or f32 O (bf16)
  float* ml;                   // nsplit > 1: running (max, sum) [nsplit][b*h][lq][2]
  const float* rcos;           // RoPE tables [rrows][d] (f32) for the first nrq queries, or null
  const float* rsin;
  int rrows, nrq;
  void* vt;                    // head dim 256: V as transposed key tiles (flash_vt.hpp), flash256_vt_bytes
  int vt_ready;                // the tiles are already written (by the rotation launch)
  const void* mask;            // additive mask (element type), or null; strides sm: batch, head, query, key
  long sm[4];
};

// V of a head-dim-256 call, to be written as transposed key tiles at vt (flash_vt.hpp).
struct VtJob {
  const void* v;
  long sv[3];
  int b, h, lk;
  void* vt;
};
long flash256_vt_blocks(const VtJob& j);                                // workgroups of its pass (256 threads)
hipError_t flash256_vt(const VtJob& j, hipStream_t stream);             // the pass as a launch of its own

int flash_padded_dim(int d);
int flash_queries_per_block(int dtype, int d, int lk);
void flash_plan(int dtype, int b, int h, int lq, int lk, int d, int cus, int* qblocks, int* nsplit, int* tps);
size_t flash_partial_bytes(int b, int h, int lq, int d, int nsplit);
hipError_t flash_attn_half(int dtype, FlashParams p, bool ropeq, hipStream_t stream);
// f32 (flash_attn_f32.hip): the attention kernel and, with key splits, the combine.
hipError_t flash_attn_f32(FlashParams p, bool ropeq, hipStream_t stream);
hipError_t flash_combine_f32(FlashParams p, int dp, hipStream_t stream);
// The head-dim-256 kernel (flash_attn_d256.hip): the bytes of its transposed V tiles, whether it takes
// p, and its launch (the V tile pass and the main kernel; not the combine).
size_t flash256_vt_bytes(int b, int h, int lk, int d);
bool flash256_eligible(const FlashParams& p, int elem_bytes);
hipError_t flash256_launch(int dtype, FlashParams p, bool ropeq, hipStream_t stream);

// x [b, l, h, d] (strides sx) -> out (strides so): row r < nrot rotated with table row r % trows,
// the other rows copied.
hipError_t rope_rows(int dtype, const void* x, const long* sx, void* out, const long* so, int b, int l, int h, int d,
                     const float* cos_t, const float* sin_t, int trows, int nrot, hipStream_t stream);
// One f16 / bf16 row set of a rope_rows2 launch (total = b * l * h * d / 8 threads).
struct RopeJob {
  const void* x;
  void* out;
  long sx[3], so[3];
  int b, l, h, nrot;
  long total;
};
RopeJob rope_job(const void* x, const long* sx, void* out, const long* so, int b, int l, int h, int d, int nrot);
// rope_rows over job a and, if b is not null, job b in one launch (f16 / bf16; both with head dim d);
// if vt is not null, the same launch also writes that V as transposed key tiles.
hipError_t rope_rows2(int dtype, const RopeJob& a, const RopeJob* b, int d, const float* cos_t, const float* sin_t,
                      int trows, hipStream_t stream, const VtJob* vt = nullptr);

}  // namespace samhip
