// The elementwise steps around the encoder's attention and MLP, for gfx950 (f32, f16, bf16):
//   bias_residual: out = res + y + bias[col]                       (kernels.rs:618-640, sam.cu:129-134)
//   bias_gelu:     out = gelu_erf(y + bias[col])                   (kernels.rs:642-663, sam.cu:136-141)
// with col = index % c, the arithmetic in f32 in the reference's order ((res + y) + bias; x = y + bias,
// then 0.5 * x * (1 + erf(x / sqrt(2))), the erf term through an erfc fit, see gelu_erf) and one
// rounding to the output type.
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
        for (int k = 0; k < n; ++k) o[k] = from_f32<T>(gelu_erf(to_f32(yv[k]) + to_f32(bv[k])));
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
        out[i] = from_f32<T>(gelu_erf(to_f32(y[i]) + bb));
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

hipError_t bias_gelu(int dtype, const void* y, const void* b, void* out, long total, int c, hipStream_t stream) {
  if (dtype == kF32) return launch_bias<float, 1>(nullptr, y, b, out, total, c, stream);
  if (dtype == kF16) return launch_bias<f16, 1>(nullptr, y, b, out, total, c, stream);
  return launch_bias<bf16, 1>(nullptr, y, b, out, total, c, stream);
}

}  // namespace samhip
