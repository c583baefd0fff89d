// qkv projection output -> q, kT, v with the bias added, for gfx950 (the producer of the fused
// attention's input layout):
//
//   y [T, 3*C] (T = windows * n tokens, C = nh * hd; columns ordered (qkv, head, d)) + bias [3*C]
//   -> out [3, BH*n*hd]: q [BH, n, hd], kT [BH, hd, n], v [BH, n, hd], BH = windows * nh
//
// as the reference's qkv_split (kernels.rs:872-894; sam.cu:111-128; CPU twin kernels.rs:228-264). Every
// output element is from_T(to_f32(y) + to_f32(bias)), the reference's arithmetic, so results are
// bit-identical to it.
//
// One workgroup per (window, token tile, head), the tiles of a window balanced (196 tokens: 4 x 49).
// A thread owns one token of the tile and every fourth 16-byte vector of its head's row, so the index
// arithmetic has no division: q and v rows are copied with 16-byte accesses on both sides; the k part
// goes through an LDS tile so that kT is written as rows of consecutive tokens (up to 128 bytes in
// f16) rather than 2-byte scatters. Bound by HBM: y is read once, out written once.
#include "common.hpp"

namespace samhip {

constexpr int kQkvTok = 64;     // tokens per tile at most
constexpr int kQkvLanes = 4;    // threads per token row
constexpr int kQkvThreads = kQkvTok * kQkvLanes;

template <typename T, int VE>  // VE elements per vector access (16 bytes, or 1 when hd is odd-sized)
__global__ __launch_bounds__(kQkvThreads) void qkv_split_kernel(const T* __restrict__ y, const T* __restrict__ bias,
                                                               T* __restrict__ out, int n, int nh, int hd, int tiles,
                                                               int tt, long plane) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* kt_tile = reinterpret_cast<float*>(smem);  // [hd][kQkvTok + 1]
  typedef typename Vec<T>::x8 V8;
  const int C = nh * hd;
  // workgroup i runs on XCD i % 8: give each XCD a contiguous range of (window, tile, head), so the heads
  // of a token tile, whose row slices share cache lines at their edges, meet in one L2
  const int nblk = gridDim.x, xcd = blockIdx.x & 7, per = nblk >> 3, rem = nblk & 7;
  const long lin = (long)xcd * per + (xcd < rem ? xcd : rem) + (blockIdx.x >> 3);
  const int head = (int)(lin % nh);
  const int tile = (int)((lin / nh) % tiles);
  const long win = lin / ((long)nh * tiles);
  const int n0 = tile * tt;
  const int ntok = min(tt, n - n0);
  const long bh = win * nh + head;
  const int vpr = hd / VE;  // vectors per token row of one head
  const int tok = threadIdx.x / kQkvLanes, lane = threadIdx.x % kQkvLanes;
  if (tok < ntok) {
    const long t = win * n + n0 + tok;
    const T* yrow = y + t * 3L * C + head * hd;
#pragma unroll
    for (int which = 0; which < 3; ++which) {
      const T* src = yrow + which * C;
      const T* bsrc = bias + which * C + head * hd;
      T* dst = out + which * plane + (bh * n + n0 + tok) * hd;
      for (int v = lane; v < vpr; v += kQkvLanes) {
        const int d0 = v * VE;
        float vals[VE];
        if constexpr (VE == 8) {
          const V8 a = *reinterpret_cast<const V8*>(src + d0);
          const V8 bb = *reinterpret_cast<const V8*>(bsrc + d0);
#pragma unroll
          for (int e = 0; e < 8; ++e) vals[e] = to_f32(a[e]) + to_f32(bb[e]);
        } else {
          vals[0] = to_f32(src[d0]) + to_f32(bsrc[d0]);
        }
        if (which == 1) {
#pragma unroll
          for (int e = 0; e < VE; ++e) kt_tile[(d0 + e) * (kQkvTok + 1) + tok] = vals[e];
        } else if constexpr (VE == 8) {
          V8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = from_f32<T>(vals[e]);
          *reinterpret_cast<V8*>(dst + d0) = o;
        } else {
          dst[d0] = from_f32<T>(vals[0]);
        }
      }
    }
  }
  __syncthreads();
  // kT rows: kt[bh][d][n0 .. n0 + ntok), a wave writing one row of up to 64 consecutive tokens
  T* kdst = out + plane + bh * (long)hd * n + n0;
  const int wtok = threadIdx.x % kQkvTok, wrow = threadIdx.x / kQkvTok;
  if (wtok < ntok)
    for (int d = wrow; d < hd; d += kQkvThreads / kQkvTok)
      kdst[(long)d * n + wtok] = from_f32<T>(kt_tile[d * (kQkvTok + 1) + wtok]);
}

template <typename T>
static hipError_t launch_qkv(const void* y, const void* bias, void* out, long tokens, int n, int nh, int hd,
                             hipStream_t stream) {
  const long windows = tokens / n;
  const int tiles = (n + kQkvTok - 1) / kQkvTok;
  const int tt = (n + tiles - 1) / tiles;  // balanced tiles of at most kQkvTok tokens
  const long blocks = windows * tiles * nh;
  const long plane = tokens * nh * (long)hd;
  const size_t lds = (size_t)hd * (kQkvTok + 1) * sizeof(float);
  if (hd % 8 == 0)
    hipLaunchKernelGGL((qkv_split_kernel<T, 8>), dim3((unsigned)blocks), dim3(kQkvThreads), lds, stream,
                       (const T*)y, (const T*)bias, (T*)out, n, nh, hd, tiles, tt, plane);
  else
    hipLaunchKernelGGL((qkv_split_kernel<T, 1>), dim3((unsigned)blocks), dim3(kQkvThreads), lds, stream,
                       (const T*)y, (const T*)bias, (T*)out, n, nh, hd, tiles, tt, plane);
  return hipGetLastError();
}

// Checked by the caller: tokens % n == 0, hd <= 256, 3*nh*hd*tokens < 2^40, blocks < 2^31.
hipError_t qkv_split(int dtype, const void* y, const void* bias, void* out, long tokens, int n, int nh, int hd,
                     hipStream_t stream) {
  if (dtype == kF32) return launch_qkv<float>(y, bias, out, tokens, n, nh, hd, stream);
  if (dtype == kF16) return launch_qkv<f16>(y, bias, out, tokens, n, nh, hd, stream);
  return launch_qkv<bf16>(y, bias, out, tokens, n, nh, hd, stream);
}

}  // namespace samhip
