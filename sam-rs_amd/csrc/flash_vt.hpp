// V of a head-dim-256 flash-attention call as transposed key tiles: the byte image in which
// flash256_kernel (flash_attn_d256.hip) reads each 64-key tile of V from LDS, written once per call so
// that the kernel can move a tile by plain 1 KB DMAs and read it with 16-byte LDS reads.
//
// Tile t of batch*head bh is 256 rows (head-dim columns) of 64 keys, 128 bytes a row, 32 KB in all, at
// vt + (bh * tiles + t) * 32 KB. The 16-byte chunk q (0..7) of row r sits at position vt_pos(q, r) and
// holds keys vt_key(q, 0..7) of the tile; keys past lk are 0.
#pragma once
#include "flash_attn.hpp"

namespace samhip {

namespace vtl {
constexpr int kTileBytes = 64 * 256 * 2;
// Key of element j (0..7) of chunk q = 4 u + g: the P^T operand u of the 16x16x32 MFMA (the tile's
// keys 32 u .. 32 u + 31), taken straight from the S^T accumulators of key blocks 2u and 2u + 1,
// gives a lane of row group g (lanes 16 g ..) the keys 32 u + 4 g + (j & 3) + 16 (j >> 2).
__host__ __device__ constexpr int vt_key(int q, int j) { return 32 * (q >> 2) + 4 * (q & 3) + (j & 3) + 16 * (j >> 2); }
// Stored position of chunk q of row r; its own inverse. The 16 rows r..r+15 that a quarter wave reads
// at one chunk then fall on 16 distinct 16-byte bank groups.
__host__ __device__ constexpr int vt_pos(int q, int r) { return q ^ ((r >> 1) & 7); }
}  // namespace vtl

// Workgroup blk (256 threads) of the pass: a quarter of a tile, 64 keys x 64 head-dim columns. It reads
// the 64 key rows' 128-byte pieces (two 16-byte loads per thread), transposes them through LDS, and
// writes the 64 rows' 128-byte V^T pieces (two 16-byte stores per thread).
__device__ __forceinline__ void flash256_vt_quarter(const VtJob& j, long blk) {
  using namespace vtl;
  __shared__ __attribute__((aligned(16))) unsigned short tile[64][72];  // 144-byte rows
  const int ntiles = (j.lk + 63) >> 6;
  const int quarter = (int)(blk & 3);
  const long tb = blk >> 2;
  const int t = (int)(tb % ntiles);
  const long bhi = tb / ntiles;
  const int bi = (int)(bhi / j.h), head = (int)(bhi % j.h);
  const unsigned short* vb = reinterpret_cast<const unsigned short*>(j.v) + bi * j.sv[0] + head * j.sv[2] + 64 * quarter;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i, row = c >> 3, col = 8 * (c & 7);
    const int key = 64 * t + row;
    u32x4 val = u32x4{0u, 0u, 0u, 0u};
    if (key < j.lk) val = *reinterpret_cast<const u32x4*>(vb + (long)key * j.sv[1] + col);
    *reinterpret_cast<u32x4*>(&tile[row][col]) = val;
  }
  __syncthreads();
  unsigned short* out = reinterpret_cast<unsigned short*>(j.vt) + ((size_t)bhi * ntiles + t) * (64 * 256) + 64 * 64 * quarter;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = threadIdx.x + 256 * i, rr = c >> 3, pos = c & 7;
    const int q = vt_pos(pos, rr);  // rows 64 quarter + rr: the same low bits as rr
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 8; e += 2) w[e >> 1] = (unsigned)tile[vt_key(q, e)][rr] | ((unsigned)tile[vt_key(q, e + 1)][rr] << 16);
    *reinterpret_cast<u32x4*>(out + rr * 64 + pos * 8) = w;
  }
}

}  // namespace samhip
