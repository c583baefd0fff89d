// The elementwise steps around the encoder's attention and MLP, for gfx950 (f32, f16, bf16):
//   bias_residual: out = res + y + bias[col]                       (kernels.rs:618-640, sam.cu:129-134)
//   bias_gelu:     out = gelu_erf(y + bias[col])                   (kernels.rs:642-663, sam.cu:136-141)
// with col = index % c, the arithmetic in f32 in the reference's order ((res + y) + bias; x = y + bias,
// then 0.5 * x * (1 + erf(x / sqrt(2))), the erf term through an erfc fit, see gelu_erf) and one
// rounding to the output type.
//
//   bias_residual_ln: the same out, and also ln = LayerNorm(out) over each row of c (weight w, bias b,
//   epsilon eps), from out as rounded to the output type: the two steps the encoder block runs one
//   after the other (sam1/encoder.rs:118-124, a residual then the next norm), fused so that out is not
//   read back. Mean and variance are two passes in f32 over the row held in registers, ln =
//   ((x - mean) * rstd) * w + b in f32 with one rounding.
//
// out may be res or y (in place): each element is read and then written by the same thread.
// Both are bound by HBM: each thread moves 16-byte vectors of every operand (4 f32 or 8 f16/bf16
// elements; c a multiple of the vector width keeps a vector inside one bias period), in a grid-stride
// loop over enough workgroups to fill the chip. Other c take a scalar loop.
#include <algorithm>

#include "common.hpp"

namespace samhip {

namespace bias {
constexpr int kThreads = 256;
}

template <typename T> struct Vec16;
template <> struct Vec16<float> { typedef f32x4 type; static constexpr int n = 4; };
template <> struct Vec16<f16> { typedef f16x8 type; static constexpr int n = 8; };
template <> struct Vec16<bf16> { typedef bf16x8 type; static constexpr int n = 8; };

// 0.5 x (1 + erf(x / sqrt 2)), with 1 + erf(x / sqrt 2) taken as erfc(|x| / sqrt 2) for x < 0 and
// 2 - erfc(|x| / sqrt 2) otherwise, so that negative x loses nothing to cancellation. erfc is the
// Chebyshev fit of Press et al., Numerical Recipes in C (2nd ed., section 6.2, erfcc): fractional
// error below 1.2e-7 for every argument (1.04e-7 measured in float64 against the exact erfc; the f32
// evaluation here stays within 7e-8 of the exact gelu in absolute terms). About 18 instructions
// against some 45 for the device erff, which made this kernel arithmetic-bound.
__device__ __forceinline__ float gelu_erf(float x) {
#pragma clang fp contract(off)
  const float z = fabsf(x) * 0.70710678118654752f;
  const float t = __builtin_amdgcn_rcpf(1.f + 0.5f * z);
  float p = 0.17087277f;
  p = fmaf(t, p, -0.82215223f);
  p = fmaf(t, p, 1.48851587f);
  p = fmaf(t, p, -1.13520398f);
  p = fmaf(t, p, 0.27886807f);
  p = fmaf(t, p, -0.18628806f);
  p = fmaf(t, p, 0.09678418f);
  p = fmaf(t, p, 0.37409196f);
  p = fmaf(t, p, 1.00002368f);
  p = fmaf(t, p, -1.26551223f);
  const float e = t * __builtin_amdgcn_exp2f(fmaf(-z, z, p) * 1.4426950408889634f);
  return 0.5f * x * (x >= 0.f ? 2.f - e : e);
}

// MODE 0: bias_residual (res used), MODE 1: bias_gelu (res unused)
template <typename T, int MODE, bool VEC>
__global__ __launch_bounds__(bias::kThreads) void bias_ops_kernel(const T* res, const T* y, const T* __restrict__ b,
                                                                  T* out, long total, int c) {
#pragma clang fp contract(off)
  const long stride = (long)gridDim.x * bias::kThreads;
  if constexpr (VEC) {
    typedef typename Vec16<T>::type V;
    constexpr int n = Vec16<T>::n;
    const long nv = total / n;
    // the bias column moves by the same amount every iteration: one 64-bit remainder per thread
    long i = (long)blockIdx.x * bias::kThreads + threadIdx.x;
    int col = (int)((i * n) % c);
    const int step = (int)((stride * n) % c);
    for (; i < nv; i += stride) {
      const long e = i * n;
      const V yv = *reinterpret_cast<const V*>(y + e);
      const V bv = *reinterpret_cast<const V*>(b + col);
      col += step;
      if (col >= c) col -= c;
      V o;
      if constexpr (MODE == 0) {
        const V rv = *reinterpret_cast<const V*>(res + e);
#pragma unroll
        for (int k = 0; k < n; ++k) o[k] = from_f32<T>(to_f32(rv[k]) + to_f32(yv[k]) + to_f32(bv[k]));
      } else {
#pragma unroll
        for (int k = 0; k < n; ++k) o[k] = from_f32<T>(f32_result(gelu_erf(to_f32(yv[k]) + to_f32(bv[k]))));
      }
      *reinterpret_cast<V*>(out + e) = o;
    }
  } else {
    long i = (long)blockIdx.x * bias::kThreads + threadIdx.x;
    int col = (int)(i % c);
    const int step = (int)(stride % c);
    for (; i < total; i += stride) {
      const float bb = to_f32(b[col]);
      col += step;
      if (col >= c) col -= c;
      if constexpr (MODE == 0)
        out[i] = from_f32<T>(to_f32(res[i]) + to_f32(y[i]) + bb);
      else
        out[i] = from_f32<T>(f32_result(gelu_erf(to_f32(y[i]) + bb)));
    }
  }
}

// One wave per row of c elements, NV 16-byte vectors per lane at most (c <= 64 * NV * vector width).
template <typename T, int NV>
__global__ __launch_bounds__(bias::kThreads) void bias_residual_ln_kernel(
    const T* res, const T* y, const T* __restrict__ b, const T* __restrict__ lw, const T* __restrict__ lb, T* out,
    T* __restrict__ ln, long rows, int c, float eps) {
#pragma clang fp contract(off)
  typedef typename Vec16<T>::type V;
  constexpr int n = Vec16<T>::n;
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * (bias::kThreads / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nv = c / n;
  const long base = row * c;
  float x[NV][n];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int v = lane + 64 * j;
    if (v < nv) {
      const V rv = *reinterpret_cast<const V*>(res + base + v * n);
      const V yv = *reinterpret_cast<const V*>(y + base + v * n);
      const V bv = *reinterpret_cast<const V*>(b + v * n);
      V o;
#pragma unroll
      for (int k = 0; k < n; ++k) {
        o[k] = from_f32<T>(to_f32(rv[k]) + to_f32(yv[k]) + to_f32(bv[k]));
        x[j][k] = to_f32(o[k]);
        sum += x[j][k];
      }
      *reinterpret_cast<V*>(out + base + v * n) = o;
    } else {
#pragma unroll
      for (int k = 0; k < n; ++k) x[j][k] = 0.f;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m);
  const float mean = sum / (float)c;
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (lane + 64 * j < nv) {
#pragma unroll
      for (int k = 0; k < n; ++k) {
        const float d = x[j][k] - mean;
        sq += d * d;
      }
    }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) sq += __shfl_xor(sq, m);
  const float rstd = 1.f / sqrtf(sq / (float)c + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int v = lane + 64 * j;
    if (v < nv) {
      const V wv = *reinterpret_cast<const V*>(lw + v * n);
      const V bv = *reinterpret_cast<const V*>(lb + v * n);
      V o;
#pragma unroll
      for (int k = 0; k < n; ++k) o[k] = from_f32<T>(((x[j][k] - mean) * rstd) * to_f32(wv[k]) + to_f32(bv[k]));
      *reinterpret_cast<V*>(ln + base + v * n) = o;
    }
  }
}

template <typename T, int MODE>
static hipError_t launch_bias(const void* res, const void* y, const void* b, void* out, long total, int c,
                              hipStream_t stream) {
  constexpr int n = Vec16<T>::n;
  const auto aligned = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; };
  const bool vec = c % n == 0 && aligned(res) && aligned(y) && aligned(b) && aligned(out);
  const long items = vec ? total / n : total;
  // about 8 workgroups of 256 threads per CU (256 CUs), fewer for small tensors
  const long blocks = std::min<long>((items + bias::kThreads - 1) / bias::kThreads, 2048);
  if (blocks <= 0) return hipSuccess;
  if (vec)
    hipLaunchKernelGGL((bias_ops_kernel<T, MODE, true>), dim3((unsigned)blocks), dim3(bias::kThreads), 0, stream,
                       (const T*)res, (const T*)y, (const T*)b, (T*)out, total, c);
  else
    hipLaunchKernelGGL((bias_ops_kernel<T, MODE, false>), dim3((unsigned)blocks), dim3(bias::kThreads), 0, stream,
                       (const T*)res, (const T*)y, (const T*)b, (T*)out, total, c);
  return hipGetLastError();
}

// Checked by the caller: total >= 0, c >= 1, total % c == 0.
hipError_t bias_residual(int dtype, const void* res, const void* y, const void* b, void* out, long total, int c,
                         hipStream_t stream) {
  if (dtype == kF32) return launch_bias<float, 0>(res, y, b, out, total, c, stream);
  if (dtype == kF16) return launch_bias<f16, 0>(res, y, b, out, total, c, stream);
  return launch_bias<bf16, 0>(res, y, b, out, total, c, stream);
}

template <typename T>
static hipError_t launch_residual_ln(const void* res, const void* y, const void* b, const void* lw, const void* lb,
                                     void* out, void* ln, long rows, int c, float eps, hipStream_t stream) {
  const int nv = (c / Vec16<T>::n + 63) / 64;
  const unsigned blocks = (unsigned)((rows + bias::kThreads / 64 - 1) / (bias::kThreads / 64));
  if (rows <= 0) return hipSuccess;
#define SAMHIP_RLN(NV)                                                                                          \
  hipLaunchKernelGGL((bias_residual_ln_kernel<T, NV>), dim3(blocks), dim3(bias::kThreads), 0, stream,            \
                     (const T*)res, (const T*)y, (const T*)b, (const T*)lw, (const T*)lb, (T*)out, (T*)ln, rows, c, \
                     eps)
  if (nv <= 1)
    SAMHIP_RLN(1);
  else if (nv <= 2)
    SAMHIP_RLN(2);
  else if (nv <= 3)
    SAMHIP_RLN(3);
  else if (nv <= 4)
    SAMHIP_RLN(4);
  else
    SAMHIP_RLN(8);
#undef SAMHIP_RLN
  return hipGetLastError();
}

// Checked by the caller: rows >= 0, 1 <= c <= kResidualLnMax(dtype), c a multiple of the 16-byte vector
// width, 16-byte aligned pointers.
hipError_t bias_residual_ln(int dtype, const void* res, const void* y, const void* b, const void* lw, const void* lb,
                            void* out, void* ln, long rows, int c, float eps, hipStream_t stream) {
  if (dtype == kF32) return launch_residual_ln<float>(res, y, b, lw, lb, out, ln, rows, c, eps, stream);
  if (dtype == kF16) return launch_residual_ln<f16>(res, y, b, lw, lb, out, ln, rows, c, eps, stream);
  return launch_residual_ln<bf16>(res, y, b, lw, lb, out, ln, rows, c, eps, stream);
}

hipError_t bias_gelu(int dtype, const void* y, const void* b, void* out, long total, int c, hipStream_t stream) {
  if (dtype == kF32) return launch_bias<float, 1>(nullptr, y, b, out, total, c, stream);
  if (dtype == kF16) return launch_bias<f16, 1>(nullptr, y, b, out, total, c, stream);
  return launch_bias<bf16, 1>(nullptr, y, b, out, total, c, stream);
}

}  // namespace samhip
