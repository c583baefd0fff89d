// Multi-scale deformable attention (Grounding DINO / Deformable DETR), forward, for gfx950.
//
//   out[b, q, h*D + d] = sum_{l, p} attn[b,q,h,l,p] * bilinear(value_l[b, :, h, d], loc * (W_l, H_l) - 0.5)
//
// value [B, S, H, D] (the levels' pixels concatenated, level l starting at sum_{m<l} H_m*W_m),
// loc [B, Q, H, L, P, 2] as (x, y) in [0, 1], attn [B, Q, H, L, P]; bilinear sampling with zero
// padding, corners outside the level contribute nothing (kernels.rs:776-818, sam.cu:305-350).
//
// The reference GPU kernel gives every output element its own thread, which recomputes the 16 point
// weights 32 times per (q, h). Here a group of LP lanes owns one (b, q, h) pair and each lane a vector
// of VEC consecutive d (16 bytes: 4 f32 or 8 f16/bf16), so one load per corner is a 16-byte gather and
// a pair's corner row (D elements, contiguous in `value`) is read by its lanes in one coalesced access.
// The L*P points of a pair are turned once into 4 (element offset, weight) corners in LDS by the
// pair's own lanes, then every lane walks them, accumulating in f32 in the reference's (l, p, corner)
// order. Work is bound by the gathers (64 corner rows per pair), which hit L2 / the Infinity cache:
// `value` is read once from HBM.
#include "common.hpp"

namespace samhip {

constexpr int kDeformMaxLevels = 4;  // the reference's GPU limit (kernels.rs:1175-1177)
constexpr int kDeformThreads = 256;

struct Levels {
  int h[kDeformMaxLevels];
  int w[kDeformMaxLevels];
  int start[kDeformMaxLevels];
};

template <typename T, int VEC> struct VecLoad;
template <> struct VecLoad<float, 4> { typedef f32x4 type; };
template <> struct VecLoad<f16, 8> { typedef f16x8 type; };
template <> struct VecLoad<bf16, 8> { typedef bf16x8 type; };
template <typename T> struct VecLoad<T, 1> { typedef T type; };

template <typename T, int VEC>
__global__ __launch_bounds__(kDeformThreads) void deform_attn_kernel(const T* __restrict__ value,
                                                                    const T* __restrict__ loc,
                                                                    const T* __restrict__ attn,
                                                                    T* __restrict__ out, int B, int S, int Q,
                                                                    int H, int D, int L, int P, int lp_shift,
                                                                    Levels lv) {
  typedef typename VecLoad<T, VEC>::type VT;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int LP = 1 << lp_shift;            // lanes per (b, q, h) pair
  const int ppw = 64 >> lp_shift;          // pairs per wave
  const int npt = L * P;                   // points per pair
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> lp_shift, li = lane & (LP - 1);
  const long pair = ((long)blockIdx.x * (kDeformThreads / 64) + wave) * ppw + sub;
  const long npairs = (long)B * Q * H;
  const bool valid = pair < npairs;
  // corner table of this pair: npt * 4 entries of (element offset into value, weight); offset -1 = skip
  int2* corners = reinterpret_cast<int2*>(smem) + ((long)wave * ppw + sub) * npt * 4;

  const int h = valid ? (int)(pair % H) : 0;
  const long bq = valid ? pair / H : 0;  // b * Q + q
  const long b = bq / Q;
  for (int j = li; j < npt; j += LP) {
    const int l = j / P;
    int2 c4[4];
    if (valid) {
      const long base = pair * npt + j;  // ((b*Q + q)*H + h)*L*P + l*P + p
      const float wgt = to_f32(attn[base]);
      const int Hl = lv.h[l], Wl = lv.w[l];
      const float x = to_f32(loc[base * 2]) * (float)Wl - 0.5f;
      const float y = to_f32(loc[base * 2 + 1]) * (float)Hl - 0.5f;
      const float xf = floorf(x), yf = floorf(y);
      const int x0 = (int)xf, y0 = (int)yf;
      const float fx = x - xf, fy = y - yf;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int xx = x0 + (c & 1), yy = y0 + (c >> 1);
        const bool in = xx >= 0 && xx < Wl && yy >= 0 && yy < Hl;
        const float wt = wgt * ((c & 1) ? fx : 1.f - fx) * ((c >> 1) ? fy : 1.f - fy);
        const long off = ((b * S + lv.start[l] + (long)yy * Wl + xx) * H + h) * (long)D;
        c4[c] = make_int2(in ? (int)off : -1, __float_as_int(wt));
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) c4[c] = make_int2(-1, 0);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) corners[j * 4 + c] = c4[c];
  }
  __syncthreads();
  if (!valid) return;

  T* orow = out + bq * (long)H * D + (long)h * D;
  for (int d0 = li * VEC; d0 < D; d0 += LP * VEC) {
    float acc[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
    for (int j = 0; j < npt * 4; ++j) {
      const int2 cw = corners[j];
      if (cw.x >= 0) {
        const float wt = __int_as_float(cw.y);
        const VT vv = *reinterpret_cast<const VT*>(value + cw.x + d0);
        if constexpr (VEC == 1) {
          acc[0] += wt * to_f32(vv);
        } else {
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] += wt * to_f32(vv[i]);
        }
      }
    }
    if constexpr (VEC == 1) {
      orow[d0] = from_f32<T>(acc[0]);
    } else {
      VT o;
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = from_f32<T>(acc[i]);
      *reinterpret_cast<VT*>(orow + d0) = o;
    }
  }
}

template <typename T, int VEC>
static hipError_t launch_deform(const void* value, const void* loc, const void* attn, void* out, int b, int s, int q,
                                int h, int d, int l, int p, const Levels& lv, hipStream_t stream) {
  // at least 8 lanes per pair keeps the corner tables within 64 KB of LDS (8 pairs x 64 points per wave)
  const int lanes = (d + VEC - 1) / VEC;
  int shift = 3;
  while ((1 << shift) < lanes && shift < 6) ++shift;
  const int ppw = 64 >> shift;
  const long pairs = (long)b * q * h;
  const long waves = (pairs + ppw - 1) / ppw;
  const long blocks = (waves + kDeformThreads / 64 - 1) / (kDeformThreads / 64);
  const size_t lds = (size_t)(kDeformThreads / 64) * ppw * l * p * 4 * sizeof(int2);
  hipLaunchKernelGGL((deform_attn_kernel<T, VEC>), dim3((unsigned)blocks), dim3(kDeformThreads), lds, stream,
                     (const T*)value, (const T*)loc, (const T*)attn, (T*)out, b, s, q, h, d, l, p, shift, lv);
  return hipGetLastError();
}

template <typename T, int VEC>
static hipError_t pick_deform(const void* value, const void* loc, const void* attn, void* out, int b, int s, int q,
                              int h, int d, int l, int p, const Levels& lv, hipStream_t stream) {
  if (d % VEC == 0) return launch_deform<T, VEC>(value, loc, attn, out, b, s, q, h, d, l, p, lv, stream);
  return launch_deform<T, 1>(value, loc, attn, out, b, s, q, h, d, l, p, lv, stream);
}

// Checked by the caller: 1 <= l <= 4, l * p <= 64, sum of level sizes == s, offsets fit in int32.
hipError_t deform_attn(int dtype, const void* value, const void* loc, const void* attn, void* out, int b, int s,
                       int q, int h, int d, int l, int p, const int* shapes, hipStream_t stream) {
  Levels lv{};
  int start = 0;
  for (int i = 0; i < l; ++i) {
    lv.h[i] = shapes[2 * i];
    lv.w[i] = shapes[2 * i + 1];
    lv.start[i] = start;
    start += lv.h[i] * lv.w[i];
  }
  if (dtype == kF32) return pick_deform<float, 4>(value, loc, attn, out, b, s, q, h, d, l, p, lv, stream);
  if (dtype == kF16) return pick_deform<f16, 8>(value, loc, attn, out, b, s, q, h, d, l, p, lv, stream);
  return pick_deform<bf16, 8>(value, loc, attn, out, b, s, q, h, d, l, p, lv, stream);
}

}  // namespace samhip
