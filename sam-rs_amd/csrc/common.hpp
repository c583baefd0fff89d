// Device helpers shared by the gfx950 (CDNA4) kernels: element types, MFMA wrappers, LDS transpose
// reads and wave64 cross-lane exchanges. Written for gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace samhip {

// Opts kernel fn in to `bytes` of dynamic LDS on the current device, once per device (devices 0..63)
// and process. `done` is the kernel's own flag word, one bit per device. Callers on several threads
// may both make the call; repeating it is harmless, and the flag word is atomic.
inline hipError_t lds_opt_in(std::atomic<unsigned long long>& done, const void* fn, int bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const unsigned long long bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

// Compute units of the current device, read once per device (at most 64 devices cached; 256 if the
// query fails).
inline int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 256;
  if (dev >= 0 && dev < 64) cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

typedef _Float16 f16;
typedef __bf16 bf16;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Dtype codes of the C ABI; the same order as the reference's dtype dispatch (F16, BF16, F32 there).
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

template <typename T> struct Vec;
template <> struct Vec<f16> {
  typedef f16x8 x8;
  typedef f16x4 x4;
};
template <> struct Vec<bf16> {
  typedef bf16x8 x8;
  typedef bf16x4 x4;
};
template <> struct Vec<float> {
  typedef float x8 __attribute__((ext_vector_type(8)));
  typedef f32x4 x4;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) { return (f16)v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }

// v as a finished f32 result. Without it the compiler may fold the multiply that produced v into the
// conversion that follows (v_fma_mixlo_f16), rounding the exact product to f16 once, where the f32
// multiply and then the conversion round twice, as the reference's f32 arithmetic does: the two differ
// by one f16 ulp when the f32 product lands on an f16 rounding midpoint.
__device__ __forceinline__ float f32_result(float v) {
  asm("" : "+v"(v));
  return v;
}

// D(32x32, f32) += A(32x16) * B(16x32). Lane l supplies A[l%32][8*(l/32)+j] and B[8*(l/32)+j][l%32],
// j = 0..7; it receives D[8*(i/4) + 4*(l/32) + i%4][l%32] in element i (layout checked on gfx950).
__device__ __forceinline__ f32x16 mma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// D(16x16, f32) += A(16x32) * B(32x16). Lane l supplies A[l%16][8*(l/16)+j] and B[8*(l/16)+j][l%16],
// j = 0..7; it receives D[4*(l/16) + i][l%16] in element i.
__device__ __forceinline__ f32x4 mma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// LDS transpose read (ds_read_b64_tr_b16). Within each group of 16 lanes, lane i receives element
// (i % 4) of the 4 x 16-bit values addressed by lanes 4*s + i/4 of its group, in element s (s = 0..3).
// So if lane 4*s + c of the group points at row (k0 + s) of a row-major tile, at column n0 + 4*c,
// lane i gets the column n0 + i for rows k0..k0+3: the MFMA operand layout, from a tile whose
// reduction dimension is the strided one.
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

template <typename T>
__device__ __forceinline__ typename Vec<T>::x8 join8(i16x4 lo, i16x4 hi) {
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  i16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Vec<T>::x8, v);
}

// max(a, b) as v_maximum_f32 / v_maximum3_f32: unlike fmaxf it needs no quieting of its operands
// first (a NaN operand gives NaN; +0 is above -0), which the max reductions over MFMA results would
// otherwise pay for with one extra instruction per operand not known to be canonical.
__device__ __forceinline__ float max_nc(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Value of `x` held by lane (l ^ 32): v_permlane32_swap exchanges the upper half of its first operand
// with the lower half of its second, so with both operands = x the pair holds x[l] and x[l ^ 32].
__device__ __forceinline__ float max_with_partner32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_with_partner32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Max and sum over the four lanes l % 16 + 16 g (g = 0..3) of a 16-lane column: v_permlane16_swap
// exchanges the odd 16-lane rows of its first operand with the even rows of its second, so with both
// operands = x the pair holds x[l] and x[l ^ 16]; permlane32_swap then pairs l and l ^ 32.
__device__ __forceinline__ float max_over_rows16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_with_partner32(max_nc(__uint_as_float(r[0]), __uint_as_float(r[1])));
}
__device__ __forceinline__ float sum_over_rows16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return sum_with_partner32(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Packs 8 f32 values into the 8 x 16-bit MFMA operand (round to nearest even).
__device__ __forceinline__ f16x8 pack8(const float* v, f16x8*) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (f16)v[i];
  return r;
}
__device__ __forceinline__ bf16x8 pack8(const float* v, bf16x8*) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16)v[i];
  return r;
}

__device__ __forceinline__ int wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

}  // namespace samhip
