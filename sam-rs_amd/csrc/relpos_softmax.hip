// Softmax over materialised scores with the decomposed relative-position bias, for gfx950:
//
//   out[bh, r, k] = softmax_k( scale * s[bh, r, k] + q[bh, r] . Th[i - kh + H-1] + q[bh, r] . Tw[j - kw + W-1] )
//
// with r = i*W + j, k = kh*W + kw. This is the reference's relpos_softmax (kernels.rs:12-43, GPU kernel
// sam.cu:44-96, CPU twin kernels.rs:62-105), kept for callers that already hold the score matrix; the
// fused attention (attn_relpos.hip) never materialises it.
//
// One workgroup of 256 threads per score row (as the reference), the row held in registers (ITEMS
// values per thread, N <= 256 * ITEMS). The H + W bias dot products are spread over the threads
// (one each), with q staged in LDS; max and sum are reduced across each wave with DPP row shifts and
// permlane32_swap, then across the 4 waves through LDS. The row is read and written once: the kernel
// is bound by HBM (2 * N elements per row).
#include "common.hpp"

namespace samhip {

constexpr int kSmThreads = 256;

__device__ __forceinline__ float wave_max(float v) {
  // within rows of 16 lanes, then across the 4 rows of a wave
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return max_with_partner32(v);
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
  v += __shfl_xor(v, 16, 64);
  return sum_with_partner32(v);
}

template <typename T, int ITEMS, bool VEC8>
__global__ __launch_bounds__(kSmThreads) void relpos_softmax_kernel(const T* __restrict__ s, const T* __restrict__ q,
                                                                   const T* __restrict__ tab, T* __restrict__ out,
                                                                   int H, int W, int HD, float scale) {
  __shared__ float qs[256];  // hd <= 256
  __shared__ float rh[128], rw[128];
  __shared__ float red[2][4];
  const int N = H * W;
  const long row = blockIdx.x;
  const int rem = (int)(row % N), i = rem / W, j = rem % W;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int c = tid; c < HD; c += kSmThreads) qs[c] = to_f32(q[row * HD + c]);
  __syncthreads();
  if (tid < H + W) {
    const bool is_h = tid < H;
    const int kk = is_h ? tid : tid - H;
    const T* tr = tab + (is_h ? (long)(i - kk + H - 1) : (long)(2 * H - 1) + (j - kk + W - 1)) * HD;
    float a = 0.f;
    for (int c = 0; c < HD; ++c) a += qs[c] * to_f32(tr[c]);
    (is_h ? rh : rw)[kk] = a;
  }
  __syncthreads();

  // element k of this thread's t-th chunk: k = (t * 256 + tid) * CH + e, CH = 8 (vector) or 1
  constexpr int CH = VEC8 ? 8 : 1;
  constexpr int NCH = ITEMS / CH;
  const T* sr = s + row * N;
  float x[ITEMS];
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < NCH; ++t) {
    const int k0 = (t * kSmThreads + tid) * CH;
    if (VEC8) {
      typename Vec<T>::x8 v8 = {};
      if (k0 < N) v8 = *reinterpret_cast<const typename Vec<T>::x8*>(sr + k0);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = k0 + e;
        float val = -INFINITY;
        if (k < N) {
          const int kh = k / W, kw = k - kh * W;
          val = to_f32(v8[e]) * scale + rh[kh] + rw[kw];
        }
        x[t * 8 + e] = val;
        m = fmaxf(m, val);
      }
    } else {
      float val = -INFINITY;
      if (k0 < N) {
        const int kh = k0 / W, kw = k0 - kh * W;
        val = to_f32(sr[k0]) * scale + rh[kh] + rw[kw];
      }
      x[t] = val;
      m = fmaxf(m, val);
    }
  }
  m = wave_max(m);
  if (lane == 0) red[0][wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < ITEMS; ++t) {
    const float e = __expf(x[t] - m);
    x[t] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) red[1][wave] = sum;
  __syncthreads();
  const float inv = 1.f / (red[1][0] + red[1][1] + red[1][2] + red[1][3]);
  T* orow = out + row * N;
#pragma unroll
  for (int t = 0; t < NCH; ++t) {
    const int k0 = (t * kSmThreads + tid) * CH;
    if (VEC8) {
      if (k0 < N) {
        typename Vec<T>::x8 v8;
#pragma unroll
        for (int e = 0; e < 8; ++e) v8[e] = from_f32<T>(x[t * 8 + e] * inv);
        *reinterpret_cast<typename Vec<T>::x8*>(orow + k0) = v8;
      }
    } else if (k0 < N) {
      orow[k0] = from_f32<T>(x[t] * inv);
    }
  }
}

template <typename T, int ITEMS>
static hipError_t launch_sm(const void* s, const void* q, const void* tab, void* out, long rows, int h, int w, int hd,
                            float scale, hipStream_t stream) {
  const int n = h * w;
  if (n % 8 == 0 && ITEMS >= 8)
    hipLaunchKernelGGL((relpos_softmax_kernel<T, ITEMS, true>), dim3((unsigned)rows), dim3(kSmThreads), 0, stream,
                       (const T*)s, (const T*)q, (const T*)tab, (T*)out, h, w, hd, scale);
  else
    hipLaunchKernelGGL((relpos_softmax_kernel<T, ITEMS, false>), dim3((unsigned)rows), dim3(kSmThreads), 0, stream,
                       (const T*)s, (const T*)q, (const T*)tab, (T*)out, h, w, hd, scale);
  return hipGetLastError();
}

template <typename T>
static hipError_t pick_items(const void* s, const void* q, const void* tab, void* out, long rows, int h, int w, int hd,
                             float scale, hipStream_t stream) {
  const int n = h * w;
  // the vector path needs ITEMS a multiple of 8; the scalar path takes any ITEMS
  if (n <= 256) return launch_sm<T, 1>(s, q, tab, out, rows, h, w, hd, scale, stream);
  if (n <= 2048) return launch_sm<T, 8>(s, q, tab, out, rows, h, w, hd, scale, stream);
  if (n <= 4096) return launch_sm<T, 16>(s, q, tab, out, rows, h, w, hd, scale, stream);
  return launch_sm<T, 32>(s, q, tab, out, rows, h, w, hd, scale, stream);
}

// Checked by the caller: n = h*w <= 8192, h, w <= 128, hd <= 256.
hipError_t relpos_softmax(int dtype, const void* s, const void* q, const void* tab, void* out, long rows, int h, int w,
                          int hd, float scale, hipStream_t stream) {
  if (dtype == kF32) return pick_items<float>(s, q, tab, out, rows, h, w, hd, scale, stream);
  if (dtype == kF16) return pick_items<f16>(s, q, tab, out, rows, h, w, hd, scale, stream);
  return pick_items<bf16>(s, q, tab, out, rows, h, w, hd, scale, stream);
}

}  // namespace samhip
