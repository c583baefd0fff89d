// Measurement kernel for bench.py (not part of the sam-rs path): the rate at which a CU can return
// 16-byte gathers of random 128-byte rows to registers, the access pattern of the deformable-attention
// gather (deform_attn.hip: a corner row of D = 32 f32 is 8 lanes x 16 bytes, loaded through one buffer
// descriptor, 16 independent loads in flight per lane). The rows come from a region small enough to
// stay in an XCD's L2 (one DINO-tiny head's value rows are 2.85 MB), so HBM does not enter: what is
// measured is the L2 -> L1 -> texture-data -> VGPR path that the gather's counters show saturated.
//
// Lane group g (8 lanes) of wave w reads, in step i, row hash(w, g, i) of the region; lane k of the
// group reads bytes [16 k, 16 k + 16) of it. Each lane folds what it loads into one sum, written once,
// so no load is dead.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 16;  // independent loads in flight per lane, as in the deform gather

__device__ __forceinline__ unsigned mix(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

__global__ __launch_bounds__(kThreads) void gather_probe_kernel(const float* __restrict__ base, unsigned rows,
                                                                 int steps, float* __restrict__ out) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(rows * 128u), 0x00020000);
  const unsigned gid = blockIdx.x * kThreads + threadIdx.x;
  const unsigned group = gid >> 3, k = gid & 7;
  float acc = 0.f;
  for (int i0 = 0; i0 < steps; i0 += kUnroll) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    f32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const unsigned row = mix(group * 0x9E3779B9U + (unsigned)(i0 + u)) % rows;
      v[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(row * 128u + 16u * k), 0, 0));
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
  }
  out[gid] = acc;
}

}  // namespace

extern "C" {

// Gathers `steps` 16-byte pieces per lane (a multiple of 16) from random 128-byte rows of the first
// `rows` rows at `base` (rows * 128 bytes of device memory, rows <= 2^23), with `blocks`
// workgroups of 256 lanes; out holds blocks * 256 floats. Returns the launch's hipError_t. The bytes
// delivered to registers are blocks * 256 * steps * 16.
int sam_probe_gather(const void* base, unsigned rows, int steps, int blocks, float* out, void* stream) {
  if (!base || !out || rows == 0 || rows > (1u << 23) || steps <= 0 || steps % kUnroll != 0 || blocks <= 0)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(gather_probe_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), (const float*)base, rows, steps, out);
  return (int)hipGetLastError();
}

}  // extern "C"
