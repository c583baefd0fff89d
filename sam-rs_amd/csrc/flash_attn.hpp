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
  int qblocks, nsplit, tps;    // query blocks, key splits, key tiles (of 64) per split
  float* opart;                // nsplit > 1: unnormalised partial O [nsplit][b*h][lq][padded d]
  float* ml;                   // nsplit > 1: running (max, sum) [nsplit][b*h][lq][2]
  const float* rcos;           // RoPE tables [rrows][d] (f32) for the first nrq queries, or null
  const float* rsin;
  int rrows, nrq;
};

int flash_padded_dim(int d);
int flash_queries_per_block(int d);
void flash_plan(int b, int h, int lq, int lk, int d, int cus, int* qblocks, int* nsplit, int* tps);
size_t flash_partial_bytes(int b, int h, int lq, int d, int nsplit);
hipError_t flash_attn_half(int dtype, FlashParams p, bool ropeq, hipStream_t stream);

// x [b, l, h, d] (strides sx) -> out (strides so): row r < nrot rotated with table row r % trows,
// the other rows copied.
hipError_t rope_rows(int dtype, const void* x, const long* sx, void* out, const long* so, int b, int l, int h, int d,
                     const float* cos_t, const float* sin_t, int trows, int nrot, hipStream_t stream);

}  // namespace samhip
