// 2-D axial RoPE applied to rows of a [B, L, H, D] tensor, for gfx950:
//
//   out[b, r, h, 2i]   = x[2i] * cos[t, 2i]   + (-x[2i+1]) * sin[t, 2i]
//   out[b, r, h, 2i+1] = x[2i+1] * cos[t, 2i+1] + x[2i] * sin[t, 2i+1]      for r < nrot, t = r % trows
//   out[b, r, h, :]    = x[b, r, h, :]                                       for r >= nrot
//
// the reference's rope (sam3/video.rs:106-113: f32 arithmetic, each product and the sum rounded, then
// converted back to the element type) together with RopeAttn's key handling (sam3/video.rs:133-141:
// the tables tiled over the first M - n_exclude keys, the object-pointer keys left as they are).
// One thread per 8 contiguous elements; bound by HBM (x read once, out written once, the f32 tables
// read from L2). For f16 / bf16 one launch can rotate two row sets (an attention call's keys and queries).
#include "flash_attn.hpp"

namespace samhip {

template <typename T>
__device__ __forceinline__ void rope_rows_one(const RopeJob& jb, int d, const float* __restrict__ cos_t,
                                              const float* __restrict__ sin_t, int trows, long c) {
  typedef typename Vec<T>::x8 X8;
  if (c >= jb.total) return;
  const int cpr = d / 8;
  const int c8 = (int)(c % cpr) * 8;
  const long rowi = c / cpr;  // (b, r, h)
  const int hi = (int)(rowi % jb.h);
  const long br = rowi / jb.h;
  const int r = (int)(br % jb.l);
  const long bi = br / jb.l;
  const T* x = reinterpret_cast<const T*>(jb.x);
  T* out = reinterpret_cast<T*>(jb.out);
  const X8 xv = *reinterpret_cast<const X8*>(x + bi * jb.sx[0] + r * jb.sx[1] + hi * jb.sx[2] + c8);
  X8 yv = xv;
  if (r < jb.nrot) {
#pragma clang fp contract(off)  // the reference rounds each product and the sum: no FMA
    const long tr = (long)(r % trows) * d + c8;
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float x0 = to_f32(xv[j]), x1 = to_f32(xv[j + 1]);
      y[j] = x0 * cos_t[tr + j] + -x1 * sin_t[tr + j];
      y[j + 1] = x1 * cos_t[tr + j + 1] + x0 * sin_t[tr + j + 1];
    }
    yv = pack8(y, (X8*)nullptr);
  }
  *reinterpret_cast<X8*>(out + bi * jb.so[0] + r * jb.so[1] + hi * jb.so[2] + c8) = yv;
}

// Up to two row sets in one launch (the keys and the queries of one attention call): blocks below
// blocks_a work on job a, the rest on job b.
template <typename T>
__global__ __launch_bounds__(256) void rope_rows_kernel(RopeJob a, RopeJob b, long blocks_a, int d,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, int trows) {
  const long blk = blockIdx.x;
  if (blk < blocks_a) rope_rows_one<T>(a, d, cos_t, sin_t, trows, blk * 256 + threadIdx.x);
  else rope_rows_one<T>(b, d, cos_t, sin_t, trows, (blk - blocks_a) * 256 + threadIdx.x);
}

// f32 rows: one thread per 4 contiguous elements.
__global__ __launch_bounds__(256) void rope_rows_f32_kernel(const float* __restrict__ x, long sx0, long sx1,
                                                            long sx2, float* __restrict__ out, long so0, long so1,
                                                            long so2, int l, int h, int d,
                                                            const float* __restrict__ cos_t,
                                                            const float* __restrict__ sin_t, int trows, int nrot,
                                                            long total) {
  const long c = (long)blockIdx.x * 256 + threadIdx.x;
  if (c >= total) return;
  const int cpr = d / 4;
  const int c4 = (int)(c % cpr) * 4;
  const long rowi = c / cpr;
  const int hi = (int)(rowi % h);
  const long br = rowi / h;
  const int r = (int)(br % l);
  const long bi = br / l;
  const f32x4 xv = *reinterpret_cast<const f32x4*>(x + bi * sx0 + r * sx1 + hi * sx2 + c4);
  f32x4 yv = xv;
  if (r < nrot) {
#pragma clang fp contract(off)  // the reference rounds each product and the sum: no FMA
    const long tr = (long)(r % trows) * d + c4;
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
      yv[j] = xv[j] * cos_t[tr + j] + -xv[j + 1] * sin_t[tr + j];
      yv[j + 1] = xv[j + 1] * cos_t[tr + j + 1] + xv[j] * sin_t[tr + j + 1];
    }
  }
  *reinterpret_cast<f32x4*>(out + bi * so0 + r * so1 + hi * so2 + c4) = yv;
}

RopeJob rope_job(const void* x, const long* sx, void* out, const long* so, int b, int l, int h, int d, int nrot) {
  RopeJob j;
  j.x = x;
  j.out = out;
  for (int i = 0; i < 3; ++i) {
    j.sx[i] = sx[i];
    j.so[i] = so[i];
  }
  j.b = b;
  j.l = l;
  j.h = h;
  j.nrot = nrot;
  j.total = (long)b * l * h * (d / 8);
  return j;
}

hipError_t rope_rows2(int dtype, const RopeJob& a, const RopeJob* b, int d, const float* cos_t, const float* sin_t,
                      int trows, hipStream_t stream) {
  RopeJob none{};
  const RopeJob& jb = b ? *b : none;
  const long ba = (a.total + 255) / 256, bb = (jb.total + 255) / 256;
  const unsigned blocks = (unsigned)(ba + bb);
  if (dtype == kF16)
    hipLaunchKernelGGL(rope_rows_kernel<f16>, dim3(blocks), dim3(256), 0, stream, a, jb, ba, d, cos_t, sin_t, trows);
  else
    hipLaunchKernelGGL(rope_rows_kernel<bf16>, dim3(blocks), dim3(256), 0, stream, a, jb, ba, d, cos_t, sin_t, trows);
  return hipGetLastError();
}

hipError_t rope_rows(int dtype, const void* x, const long* sx, void* out, const long* so, int b, int l, int h, int d,
                     const float* cos_t, const float* sin_t, int trows, int nrot, hipStream_t stream) {
  if (dtype == kF32) {
    const long total = (long)b * l * h * (d / 4);
    const unsigned blocks = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(rope_rows_f32_kernel, dim3(blocks), dim3(256), 0, stream, (const float*)x, sx[0], sx[1], sx[2],
                       (float*)out, so[0], so[1], so[2], l, h, d, cos_t, sin_t, trows, nrot, total);
    return hipGetLastError();
  }
  return rope_rows2(dtype, rope_job(x, sx, out, so, b, l, h, d, nrot), nullptr, d, cos_t, sin_t, trows, stream);
}

}  // namespace samhip
