// SAM 3 ViT's qkv step, for gfx950: the fused qkv projection's output with the bias added, 2-D RoPE on
// q and k, split into the packed layout that the attention reads:
//
//   y [T, 3*C] (C = nh * hd; columns ordered (qkv, head, d)) + bias [3*C]
//   -> out [3, T, nh, hd], with for the pair (x0, x1) = (y + bias)[2i, 2i+1] of a q or k row of token t
//        out[2i]   = x0 * cos[t % n, 2i] - x1 * sin[t % n, 2i]
//        out[2i+1] = x1 * cos[t % n, 2i] + x0 * sin[t % n, 2i]
//      and v rows biased only,
//
// the reference's qkv_rope (kernels.rs:1013-1037; GPU op sam.cu:210-235, launcher kernels.rs:1330-1343;
// CPU twin kernels.rs:321-362). Both elements of a pair use the table's even column, as the reference
// reads it. The arithmetic is f32: y and the bias are added in f32 (not rounded to the element type first),
// each product and the difference (sum) are rounded as the CPU twin rounds them (no FMA contraction),
// and the result is converted to the element type once.
//
// Bound by HBM: y is read once and out written once; the bias (6 KB for SAM 3) and the cos/sin rows come
// from the caches. When hd % 8 == 0, a thread owns one token, one 8-column piece k of a head row, and a
// group of G consecutive head rows of the token's 3*nh (q heads, k heads, v heads): it reads the token's
// table piece once for the whole group (a thread per vector would read it once per vector, the table
// bytes through L1 then outnumbering y's) and requests the group's y vectors before it stores the first.
// The 8 lanes of one (token, group) read and write a head row's 8-column pieces side by side, so every
// access of a wave covers whole rows. f16/bf16 move y and out with non-temporal loads and stores (G = 8);
// f32 with ordinary ones (G = 4), each the faster form measured for its type. Head dims that are not a
// multiple of 8 take a per-pair kernel with the same arithmetic.
#include "common.hpp"

namespace samhip {

constexpr int kRopeThreads = 256;

// One rotated or biased pair, in the reference's order of operations.
__device__ __forceinline__ void qkv_rope_pair(float& x0, float& x1, float c, float s, bool rot) {
#pragma clang fp contract(off)
  if (rot) {
    const float r0 = x0 * c - x1 * s;
    const float r1 = x1 * c + x0 * s;
    x0 = r0;
    x1 = r1;
  }
}

// Head rows per thread, and whether y and out move by non-temporal accesses, for element type T.
template <typename T> struct RopeGroup {
  static constexpr int G = 8;
  static constexpr bool kNT = true;
};
template <> struct RopeGroup<float> {
  static constexpr int G = 4;
  static constexpr bool kNT = false;
};

// hd % 8 == 0: thread i is piece k = i % cv (cv = hd / 8) of head rows G g .. G g + G - 1 (g = (i / cv) %
// ng, ng = ceil(3 nh / G)) of token i / (cv ng). nthr = T * cv * ng < 2^32 (the caller bounds T * 3 C / 8,
// which is larger).
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void qkv_rope_kernel(const T* __restrict__ y, const T* __restrict__ bias,
                                                                 const float* __restrict__ cos_t,
                                                                 const float* __restrict__ sin_t,
                                                                 T* __restrict__ out, unsigned nthr, unsigned cv,
                                                                 int c, int hd, int n, long plane) {
  typedef typename Vec<T>::x8 X8;
  typedef float F8 __attribute__((ext_vector_type(8)));
  constexpr int G = RopeGroup<T>::G;
  constexpr bool kNT = RopeGroup<T>::kNT;
  const unsigned i = blockIdx.x * kRopeThreads + threadIdx.x;
  if (i >= nthr) return;
  const int nrows = 3 * c / hd;
  const unsigned ng = (unsigned)(nrows + G - 1) / G;
  const unsigned k = i % cv, rest = i / cv, grp = rest % ng, tok = rest / ng;
  const int r0 = G * (int)grp;
  const long tr = (long)(tok % (unsigned)n) * hd + 8 * k;
  const F8 cs = *reinterpret_cast<const F8*>(cos_t + tr);
  const F8 sn = *reinterpret_cast<const F8*>(sin_t + tr);
  const T* yr = y + (long)tok * (3L * c) + 8 * k;
  X8 a[G], b[G];
#pragma unroll
  for (int u = 0; u < G; ++u)
    if (r0 + u < nrows) {
      const X8* src = reinterpret_cast<const X8*>(yr + (r0 + u) * hd);
      a[u] = kNT ? __builtin_nontemporal_load(src) : *src;
      b[u] = *reinterpret_cast<const X8*>(bias + (r0 + u) * hd + 8 * k);
    }
#pragma unroll
  for (int u = 0; u < G; ++u)
    if (r0 + u < nrows) {
      const int col = (r0 + u) * hd;
      const int which = col >= c ? (col >= 2 * c ? 2 : 1) : 0;
      float r[8];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        float x0 = to_f32(a[u][j]) + to_f32(b[u][j]);
        float x1 = to_f32(a[u][j + 1]) + to_f32(b[u][j + 1]);
        qkv_rope_pair(x0, x1, cs[j], sn[j], which < 2);
        r[j] = x0;
        r[j + 1] = x1;
      }
      X8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = from_f32<T>(r[j]);
      X8* dst = reinterpret_cast<X8*>(out + which * plane + (long)tok * c + (col - which * c) + 8 * k);
      if (kNT)
        __builtin_nontemporal_store(o, dst);
      else
        *dst = o;
    }
}

// Any even hd: one thread per pair of the flattened rows (npair = T * 3*C / 2).
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void qkv_rope_pair_kernel(const T* __restrict__ y,
                                                                      const T* __restrict__ bias,
                                                                      const float* __restrict__ cos_t,
                                                                      const float* __restrict__ sin_t,
                                                                      T* __restrict__ out, long npair, int c, int hd,
                                                                      int n, long plane) {
  const long p = (long)blockIdx.x * kRopeThreads + threadIdx.x;
  if (p >= npair) return;
  const long ppr = 3L * c / 2;  // pairs per token row
  const long t = p / ppr;
  const int col = (int)(p - t * ppr) * 2;
  const int which = col / c, within = col - which * c;
  float x0 = to_f32(y[t * 3L * c + col]) + to_f32(bias[col]);
  float x1 = to_f32(y[t * 3L * c + col + 1]) + to_f32(bias[col + 1]);
  if (which < 2) {
    const long tr = (t % n) * hd + within % hd;
    qkv_rope_pair(x0, x1, cos_t[tr], sin_t[tr], true);
  }
  T* o = out + which * plane + t * c + within;
  o[0] = from_f32<T>(x0);
  o[1] = from_f32<T>(x1);
}

template <typename T>
static hipError_t launch_qkv_rope(const void* y, const void* bias, const float* cos_t, const float* sin_t, void* out,
                                  long tokens, int n, int nh, int hd, hipStream_t stream) {
  const int c = nh * hd;
  const long plane = tokens * (long)c;
  if (hd % 8 == 0) {
    constexpr int G = RopeGroup<T>::G;
    const long cv = hd / 8, nthr = tokens * cv * ((3L * c / hd + G - 1) / G);
    const long blocks = (nthr + kRopeThreads - 1) / kRopeThreads;
    hipLaunchKernelGGL(qkv_rope_kernel<T>, dim3((unsigned)blocks), dim3(kRopeThreads), 0, stream, (const T*)y,
                       (const T*)bias, cos_t, sin_t, (T*)out, (unsigned)nthr, (unsigned)cv, c, hd, n, plane);
  } else {
    const long npair = tokens * 3L * c / 2;
    const long blocks = (npair + kRopeThreads - 1) / kRopeThreads;
    hipLaunchKernelGGL(qkv_rope_pair_kernel<T>, dim3((unsigned)blocks), dim3(kRopeThreads), 0, stream, (const T*)y,
                       (const T*)bias, cos_t, sin_t, (T*)out, npair, c, hd, n, plane);
  }
  return hipGetLastError();
}

hipError_t qkv_rope(int dtype, const void* y, const void* bias, const float* cos_t, const float* sin_t, void* out,
                    long tokens, int n, int nh, int hd, hipStream_t stream) {
  switch (dtype) {
    case kF16: return launch_qkv_rope<f16>(y, bias, cos_t, sin_t, out, tokens, n, nh, hd, stream);
    case kBF16: return launch_qkv_rope<bf16>(y, bias, cos_t, sin_t, out, tokens, n, nh, hd, stream);
    default: return launch_qkv_rope<float>(y, bias, cos_t, sin_t, out, tokens, n, nh, hd, stream);
  }
}

}  // namespace samhip
