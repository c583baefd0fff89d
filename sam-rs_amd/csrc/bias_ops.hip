// The elementwise steps around the encoder's attention and MLP, for gfx950 (f32, f16, bf16):
//   bias_residual: out = res + y + bias[col]                       (kernels.rs:618-640, sam.cu:129-134)
//   bias_gelu:     out = gelu_erf(y + bias[col])                   (kernels.rs:642-663, sam.cu:136-141)
// with col = index % c, the arithmetic in f32 in the reference's order ((res + y) + bias; x = y + bias,
// then 0.5 * x * (1 + erf(x / sqrt(2)))) and one rounding to the output type.
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

__device__ __forceinline__ float gelu_erf(float x) {
#pragma clang fp contract(off)
  return 0.5f * x * (1.f + erff(x * 0.70710678118654752f));
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
    for (long i = (long)blockIdx.x * bias::kThreads + threadIdx.x; i < nv; i += stride) {
      const long e = i * n;
      const V yv = *reinterpret_cast<const V*>(y + e);
      const V bv = *reinterpret_cast<const V*>(b + (int)(e % c));
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
    for (long i = (long)blockIdx.x * bias::kThreads + threadIdx.x; i < total; i += stride) {
      const float bb = to_f32(b[(int)(i % c)]);
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
