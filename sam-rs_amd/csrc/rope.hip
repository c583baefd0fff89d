// 2-D axial RoPE applied to rows of a [B, L, H, D] tensor, for gfx950:
//
//   out[b, r, h, 2i]   = x[2i] * cos[t, 2i]   + (-x[2i+1]) * sin[t, 2i]
//   out[b, r, h, 2i+1] = x[2i+1] * cos[t, 2i+1] + x[2i] * sin[t, 2i+1]      for r < nrot, t = r % trows
//   out[b, r, h, :]    = x[b, r, h, :]                                       for r >= nrot
//
// the reference's rope (sam3/video.rs:106-113: f32 arithmetic, each product and the sum rounded, then
// converted back to the element type) together with RopeAttn's key handling (sam3/video.rs:133-141:
// the tables tiled over the first M - n_exclude keys, the object-pointer keys left as they are).
// f16 / bf16: rope_shared_kernel, which reads each piece of the tables once for every row that uses it;
// one launch can rotate two row sets (an attention call's keys and queries). f32: one thread per 4
// contiguous elements. Bound by HBM (x read once, out written once).
#include <algorithm>

#include "flash_attn.hpp"
#include "flash_vt.hpp"

namespace samhip {

// Rotation with shared table reads: a thread owns (batch*head, table row t, 8 columns), reads that
// piece of the cos and sin tables once, and rotates every row r = t (mod trows), r < nrot, of both row
// sets (the cross-attention keys use each table row 7 times, and the queries once more). The threads
// past the rotation part copy the rows r >= nrot. Workgroups past those of the rows (vt_blocks of
// them) write a head-dim-256 attention call's V as transposed key tiles (flash_vt.hpp), so that the
// call's preparation is one launch.
template <typename T>
__device__ __forceinline__ void rope_rotate_rows(const RopeJob& jb, long bhx, int t, int c8, int trows,
                                                 const float* cs, const float* sn) {
  typedef typename Vec<T>::x8 X8;
  if (bhx >= (long)jb.b * jb.h || t >= jb.nrot) return;
  const int hi = (int)(bhx % jb.h);
  const long bi = bhx / jb.h;
  const T* x = reinterpret_cast<const T*>(jb.x) + bi * jb.sx[0] + hi * jb.sx[2] + c8;
  T* out = reinterpret_cast<T*>(jb.out) + bi * jb.so[0] + hi * jb.so[2] + c8;
  for (int r0 = t; r0 < jb.nrot; r0 += 4 * trows) {
    X8 xv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = r0 + u * trows;
      if (r < jb.nrot) xv[u] = *reinterpret_cast<const X8*>(x + (long)r * jb.sx[1]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int r = r0 + u * trows;
      if (r < jb.nrot) {
#pragma clang fp contract(off)  // the reference rounds each product and the sum: no FMA
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const float x0 = to_f32(xv[u][j]), x1 = to_f32(xv[u][j + 1]);
          y[j] = x0 * cs[j] + -x1 * sn[j];
          y[j + 1] = x1 * cs[j + 1] + x0 * sn[j + 1];
        }
        *reinterpret_cast<X8*>(out + (long)r * jb.so[1]) = pack8(y, (X8*)nullptr);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void rope_shared_kernel(RopeJob a, RopeJob b, int d, const float* __restrict__ cos_t,
                                                          const float* __restrict__ sin_t, int trows, int tused,
                                                          long nrt, long ncopy_a, long ncopy_b, VtJob vt,
                                                          unsigned row_blocks) {
  typedef typename Vec<T>::x8 X8;
  if (blockIdx.x >= row_blocks) {  // uniform per workgroup
    flash256_vt_quarter(vt, (long)(blockIdx.x - row_blocks));
    return;
  }
  const long c = (long)blockIdx.x * 256 + threadIdx.x;
  const int cpr = d / 8;
  if (c < nrt) {
    const int c8 = (int)(c % cpr) * 8;
    const long rest = c / cpr;
    const int t = (int)(rest % tused);
    const long bhx = rest / tused;
    const long tr = (long)t * d + c8;
    float cs[8], sn[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      cs[j] = cos_t[tr + j];
      sn[j] = sin_t[tr + j];
    }
    rope_rotate_rows<T>(a, bhx, t, c8, trows, cs, sn);
    rope_rotate_rows<T>(b, bhx, t, c8, trows, cs, sn);
    return;
  }
  long k = c - nrt;
  if (k >= ncopy_a + ncopy_b) return;
  const bool in_a = k < ncopy_a;
  const RopeJob& jb = in_a ? a : b;
  if (!in_a) k -= ncopy_a;
  const int c8 = (int)(k % cpr) * 8;
  const long rest = k / cpr;
  const int nl = jb.l - jb.nrot;
  const int r = jb.nrot + (int)(rest % nl);
  const long bhx = rest / nl;
  const int hi = (int)(bhx % jb.h);
  const long bi = bhx / jb.h;
  *reinterpret_cast<X8*>(reinterpret_cast<T*>(jb.out) + bi * jb.so[0] + (long)r * jb.so[1] + hi * jb.so[2] + c8) =
      *reinterpret_cast<const X8*>(reinterpret_cast<const T*>(jb.x) + bi * jb.sx[0] + (long)r * jb.sx[1] +
                                   hi * jb.sx[2] + c8);
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
                      int trows, hipStream_t stream, const VtJob* vt) {
  RopeJob none{};
  const RopeJob& jb = b ? *b : none;
  // the shared-table kernel: one thread per (batch*head, used table row, 8 columns), then one per 8
  // columns of every row past nrot
  const int cpr = d / 8;
  const long bh = std::max((long)a.b * a.h, (long)jb.b * jb.h);
  const int tused = std::min(trows, std::max(a.nrot, jb.nrot));
  const long nrt = bh * tused * cpr;
  const long ncopy_a = (long)a.b * a.h * (a.l - a.nrot) * cpr, ncopy_b = (long)jb.b * jb.h * (jb.l - jb.nrot) * cpr;
  const long threads = nrt + ncopy_a + ncopy_b;
  const unsigned row_blocks = (unsigned)((threads + 255) / 256);
  const VtJob vj = vt ? *vt : VtJob{};
  const unsigned blocks = row_blocks + (vt ? (unsigned)flash256_vt_blocks(*vt) : 0u);
  if (blocks == 0) return hipSuccess;
  if (dtype == kF16)
    hipLaunchKernelGGL(rope_shared_kernel<f16>, dim3(blocks), dim3(256), 0, stream, a, jb, d, cos_t, sin_t, trows,
                       tused, nrt, ncopy_a, ncopy_b, vj, row_blocks);
  else
    hipLaunchKernelGGL(rope_shared_kernel<bf16>, dim3(blocks), dim3(256), 0, stream, a, jb, d, cos_t, sin_t, trows,
                       tused, nrt, ncopy_a, ncopy_b, vj, row_blocks);
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
