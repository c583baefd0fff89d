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
// The L*P points of a pair are turned once into 4 (offset, weight) corners in LDS by the pair's own
// lanes, then every lane walks them, accumulating in f32 in the reference's (l, p, corner) order.
//
// Work is bound by the gathers (64 corner rows per pair for DINO), so two choices decide the speed:
// - deform_attn_gather_kernel (D a multiple of VEC): branch-free corner walk through a buffer
//   descriptor, so each wave keeps many gathers in flight, and a head-major work order in contiguous
//   ranges per XCD, so that each XCD's 4 MB L2 holds the value rows of one or two heads (value is
//   [B, S, H, D]: a head's row of a pixel is its own D-element run, shared with no other head).
// - deform_attn_kernel (other D, or more than 3.75 GB of value): the same contract with scalar lanes
//   and a branch per corner.
//
// Both kernels also take the inputs of Deform::forward between its projections (dino/mod.rs:166-178)
// in place of loc and attn (template parameter NC = 2 or 4): the sampling offsets [B,Q,H,L,P,2], the
// attention logits [B,Q,H,L,P] and the reference points [B,Q,L,NC]. The pair's lanes then softmax its
// L*P logits and form each point's location while they build its corner table, so the locations and
// weights never go through memory (the reference writes and reads both as tensors).
#include "common.hpp"

namespace samhip {

constexpr int kDeformMaxLevels = 4;  // the reference's GPU limit (kernels.rs:1175-1177)
constexpr int kDeformThreads = 256;

struct Levels {
  int h[kDeformMaxLevels];
  int w[kDeformMaxLevels];
  int start[kDeformMaxLevels];
};

// floor(x) as an index, as the reference's `x.floor() as i64` takes it (kernels.rs:799-800): NaN gives 0,
// large values saturate; the clamp to +-2^30 keeps the conversion defined and the corner x0 + 1 from
// overflowing, and any index that far out lies outside every level
__device__ __forceinline__ int floor_index(float xf) {
  return xf != xf ? 0 : (int)fminf(fmaxf(xf, -1073741824.f), 1073741824.f);
}

template <typename T, int VEC> struct VecLoad;
template <> struct VecLoad<float, 4> { typedef f32x4 type; };
template <> struct VecLoad<f16, 8> { typedef f16x8 type; };
template <> struct VecLoad<bf16, 8> { typedef bf16x8 type; };
template <typename T> struct VecLoad<T, 1> { typedef T type; };

// Where a pair's points come from. NC = 0: loc and attn as the reference's deform_attn takes them.
// NC = 2 or 4: loc holds the sampling offsets, attn the attention logits, refs the reference points.
template <typename T> struct PointSrc {
  const T* loc;
  const T* attn;
  const T* refs;
  float inv_p;  // (float)(1 / P): candle's `off / p` is affine(1/p, 0)
};

// Softmax statistics of a pair's L*P logits (NC != 0): their max and the sum of exp(x - max), reduced
// over the LP lanes li = 0..LP-1 of the pair's lane group. Every lane of the wave takes part.
template <typename T>
__device__ __forceinline__ void pair_softmax(const T* logits, long base0, int npt, int li, int LP, bool valid,
                                             float& mx, float& sum) {
  float m = -INFINITY;
  if (valid)
    for (int j = li; j < npt; j += LP) m = fmaxf(m, to_f32(logits[base0 + j]));
  for (int o = LP >> 1; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  float s = 0.f;
  if (valid)
    for (int j = li; j < npt; j += LP) s += expf(to_f32(logits[base0 + j]) - m);
  for (int o = LP >> 1; o > 0; o >>= 1) s += __shfl_xor(s, o);
  mx = m;
  sum = s;
}

// Point j (level l) of pair `pair` (bq = b * Q + q): normalised location (x, y) and weight w.
// NC = 2 (encoder, dino/mod.rs:169-173): loc = ref + off / (W_l, H_l).
// NC = 4 (decoder, dino/mod.rs:174-178): loc = xy + ((off * (1/P)) * wh) * 0.5.
// Each step is one f32 rounding, as the reference's tensor ops are (no contraction). Those ops run in
// the query's dtype, so for f16 / bf16 each step's result, the softmax output and the level sizes (the
// `norm` tensor, converted to the dtype at :170) are rounded to T as well.
template <typename T>
__device__ __forceinline__ float round_t(float x) {
  if constexpr (__is_same(T, float))
    return x;
  else
    return to_f32(from_f32<T>(f32_result(x)));
}

template <typename T, int NC>
__device__ __forceinline__ void point_xyw(const PointSrc<T>& src, long pair, long bq, int npt, int j, int l, int L,
                                          int Wl, int Hl, float mx, float sum, float& x, float& y, float& w) {
#pragma clang fp contract(off)
  const long base = pair * npt + j;
  const float ax = to_f32(src.loc[base * 2]), ay = to_f32(src.loc[base * 2 + 1]);
  if constexpr (NC == 0) {
    w = to_f32(src.attn[base]);
    x = ax;
    y = ay;
  } else {
    w = round_t<T>(expf(to_f32(src.attn[base]) - mx) / sum);
    const T* r = src.refs + (bq * L + l) * NC;
    if constexpr (NC == 2) {
      x = round_t<T>(to_f32(r[0]) + round_t<T>(ax / round_t<T>((float)Wl)));
      y = round_t<T>(to_f32(r[1]) + round_t<T>(ay / round_t<T>((float)Hl)));
    } else {
      const float ux = round_t<T>(round_t<T>(ax * src.inv_p) * to_f32(r[2]));
      const float uy = round_t<T>(round_t<T>(ay * src.inv_p) * to_f32(r[3]));
      x = round_t<T>(to_f32(r[0]) + round_t<T>(ux * 0.5f));
      y = round_t<T>(to_f32(r[1]) + round_t<T>(uy * 0.5f));
    }
  }
}

template <typename T, int VEC, int NC>
__global__ __launch_bounds__(kDeformThreads) void deform_attn_kernel(const T* __restrict__ value, PointSrc<T> src,
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
  float mx = 0.f, sum = 1.f;
  if constexpr (NC != 0) pair_softmax(src.attn, pair * npt, npt, li, LP, valid, mx, sum);
  for (int j = li; j < npt; j += LP) {
    const int l = j / P;
    int2 c4[4];
    if (valid) {
      // point ((b*Q + q)*H + h)*L*P + l*P + p
      const int Hl = lv.h[l], Wl = lv.w[l];
      float lx, ly, wgt;
      point_xyw<T, NC>(src, pair, bq, npt, j, l, L, Wl, Hl, mx, sum, lx, ly, wgt);
      const float x = lx * (float)Wl - 0.5f;
      const float y = ly * (float)Hl - 0.5f;
      const float xf = floorf(x), yf = floorf(y);
      const int x0 = floor_index(xf), y0 = floor_index(yf);
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

// The same contract through buffer-descriptor loads, for VEC-wide lanes: a skipped corner (outside
// its level) points past the end of the descriptor, where the load returns 0, so the corner walk has
// no branches and a wave keeps kDeformUnroll independent gathers in flight. The corner table of a pair
// is padded to a multiple of kDeformUnroll entries with skipped corners of weight 0. One descriptor
// covers all of `value` (wave-uniform), whose size in bytes must stay below kDeformSkip (checked by the
// launcher).
constexpr int kDeformUnroll = 16;
constexpr unsigned kDeformSkip = 0xF0000000u;

// Location and weight of a point from its staged inputs (the arithmetic of point_xyw, NC = 2 or 4):
// lg = the point's exp(logit - max) (the softmax numerator), r = its reference point.
template <typename T, int NC>
__device__ __forceinline__ void staged_xyw(const float* st, float inv_p, float sum, int Wl, int Hl, float& x,
                                           float& y, float& w) {
#pragma clang fp contract(off)
  const float e = st[0], ax = st[1], ay = st[2];
  w = round_t<T>(e / sum);
  if constexpr (NC == 2) {
    x = round_t<T>(st[3] + round_t<T>(ax / round_t<T>((float)Wl)));
    y = round_t<T>(st[4] + round_t<T>(ay / round_t<T>((float)Hl)));
  } else {
    const float ux = round_t<T>(round_t<T>(ax * inv_p) * st[5]);
    const float uy = round_t<T>(round_t<T>(ay * inv_p) * st[6]);
    x = round_t<T>(st[3] + round_t<T>(ux * 0.5f));
    y = round_t<T>(st[4] + round_t<T>(uy * 0.5f));
  }
}

template <typename T, int VEC, int NC>
__global__ __launch_bounds__(kDeformThreads) void deform_attn_gather_kernel(const T* __restrict__ value,
                                                                           PointSrc<T> src,
                                                                           T* __restrict__ out, int B, int S,
                                                                           int Q, int H, int D, int L, int P,
                                                                           int lp_shift, int ntab, Levels lv) {
  typedef typename VecLoad<T, VEC>::type VT;
  static_assert(sizeof(VT) == 16, "16-byte lanes");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int LP = 1 << lp_shift;            // lanes per (b, q, h) pair
  const int ppw = 64 >> lp_shift;          // pairs per wave
  const int npt = L * P;                   // points per pair
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> lp_shift, li = lane & (LP - 1);
  // Work items in head-major order (h, b, q), in contiguous ranges per XCD: workgroup i runs on XCD
  // i % 8, so an XCD's L2 holds the value rows of one or two heads instead of all of them.
  const int nblk = gridDim.x, xcd = blockIdx.x & 7, per = nblk >> 3, rem = nblk & 7;
  const long lin = (long)xcd * per + (xcd < rem ? xcd : rem) + (blockIdx.x >> 3);
  const long item = (lin * (kDeformThreads / 64) + wave) * ppw + sub;
  const long BQ = (long)B * Q;
  const bool valid = item < BQ * H;
  const int h = valid ? (int)(item / BQ) : 0;
  const long bq = valid ? item % BQ : 0;  // b * Q + q
  const long b = bq / Q;
  const long pair = bq * H + h;  // index of the (b, q, h) pair in loc and attn
  // corner table of this pair: ntab entries of (byte offset into value, weight)
  int2* corners = reinterpret_cast<int2*>(smem) + ((long)wave * ppw + sub) * ntab;
  float mx = 0.f, sum = 1.f;
  if constexpr (NC != 0) {
    // Deform::forward's inputs: every global load of the pair's points (logit, offsets, reference point)
    // is issued in one pass and staged in the point's own 32 bytes of the corner table (this lane alone
    // reads them back), then the softmax statistics, each exponential computed once.
    float m = -INFINITY;
#pragma unroll 2
    for (int j = li; j < npt; j += LP) {
      if (valid) {
        const long base = pair * npt + j;
        const T* r = src.refs + (bq * L + j / P) * NC;
        float* st = reinterpret_cast<float*>(corners + j * 4);
        const float lg = to_f32(src.attn[base]);
        st[0] = lg;
        st[1] = to_f32(src.loc[base * 2]);
        st[2] = to_f32(src.loc[base * 2 + 1]);
#pragma unroll
        for (int c = 0; c < NC; ++c) st[3 + c] = to_f32(r[c]);
        m = fmaxf(m, lg);
      }
    }
    for (int o = LP >> 1; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float ssum = 0.f;
    for (int j = li; j < npt; j += LP) {
      if (valid) {
        float* st = reinterpret_cast<float*>(corners + j * 4);
        const float e = expf(st[0] - m);
        st[0] = e;
        ssum += e;
      }
    }
    for (int o = LP >> 1; o > 0; o >>= 1) ssum += __shfl_xor(ssum, o);
    mx = m;
    sum = ssum;
  }
  for (int j = li; j < (ntab >> 2); j += LP) {
    int2 c4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) c4[c] = make_int2((int)kDeformSkip, 0);
    if (valid && j < npt) {
      const int l = j / P;
      // point ((b*Q + q)*H + h)*L*P + l*P + p
      const int Hl = lv.h[l], Wl = lv.w[l];
      float lx, ly, wgt;
      if constexpr (NC != 0) {
        float st[3 + NC];
#pragma unroll
        for (int c = 0; c < 3 + NC; ++c) st[c] = reinterpret_cast<const float*>(corners + j * 4)[c];
        staged_xyw<T, NC>(st, src.inv_p, sum, Wl, Hl, lx, ly, wgt);
      } else {
        point_xyw<T, NC>(src, pair, bq, npt, j, l, L, Wl, Hl, mx, sum, lx, ly, wgt);
      }
      const float x = lx * (float)Wl - 0.5f;
      const float y = ly * (float)Hl - 0.5f;
      const float xf = floorf(x), yf = floorf(y);
      const int x0 = floor_index(xf), y0 = floor_index(yf);
      const float fx = x - xf, fy = y - yf;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int xx = x0 + (c & 1), yy = y0 + (c >> 1);
        const bool in = xx >= 0 && xx < Wl && yy >= 0 && yy < Hl;
        const float wt = wgt * ((c & 1) ? fx : 1.f - fx) * ((c >> 1) ? fy : 1.f - fy);
        const unsigned off = (unsigned)(((b * S + lv.start[l] + (long)yy * Wl + xx) * H + h) * D * (long)sizeof(T));
        if (in) c4[c] = make_int2((int)off, __float_as_int(wt));
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) corners[j * 4 + c] = c4[c];
  }
  __syncthreads();
  if (!valid) return;

  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)value, (short)0, (int)(unsigned)((long)B * S * H * D * (long)sizeof(T)), 0x00020000);
  T* orow = out + bq * (long)H * D + (long)h * D;
  for (int d0 = li * VEC; d0 < D; d0 += LP * VEC) {
    float acc[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
    const unsigned dbytes = (unsigned)(d0 * sizeof(T));
    for (int j0 = 0; j0 < ntab; j0 += kDeformUnroll) {
      int2 cw[kDeformUnroll];
      VT vv[kDeformUnroll];
#pragma unroll
      for (int u = 0; u < kDeformUnroll; ++u) cw[u] = corners[j0 + u];
#pragma unroll
      for (int u = 0; u < kDeformUnroll; ++u)
        vv[u] = __builtin_bit_cast(VT, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)((unsigned)cw[u].x + dbytes), 0, 0));
#pragma unroll
      for (int u = 0; u < kDeformUnroll; ++u) {
        const float wt = __int_as_float(cw[u].y);
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[i] = fmaf(wt, to_f32(vv[u][i]), acc[i]);
      }
    }
    VT o;
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = from_f32<T>(acc[i]);
    *reinterpret_cast<VT*>(orow + d0) = o;
  }
}

template <typename T, int VEC, int NC>
static hipError_t launch_deform(const void* value, PointSrc<T> src, void* out, int b, int s, int q, int h, int d, int l,
                                int p, const Levels& lv, hipStream_t stream) {
  // at least 8 lanes per pair keeps the corner tables within 64 KB of LDS (8 pairs x 64 points per wave)
  const int lanes = (d + VEC - 1) / VEC;
  int shift = 3;
  while ((1 << shift) < lanes && shift < 6) ++shift;
  const int ppw = 64 >> shift;
  const long pairs = (long)b * q * h;
  const long waves = (pairs + ppw - 1) / ppw;
  const long blocks = (waves + kDeformThreads / 64 - 1) / (kDeformThreads / 64);
  const size_t lds = (size_t)(kDeformThreads / 64) * ppw * l * p * 4 * sizeof(int2);
  hipLaunchKernelGGL((deform_attn_kernel<T, VEC, NC>), dim3((unsigned)blocks), dim3(kDeformThreads), lds, stream,
                     (const T*)value, src, (T*)out, b, s, q, h, d, l, p, shift, lv);
  return hipGetLastError();
}

template <typename T, int VEC, int NC>
static hipError_t launch_gather(const void* value, PointSrc<T> src, void* out, int b, int s, int q, int h, int d, int l,
                                int p, const Levels& lv, hipStream_t stream) {
  const int lanes = d / VEC;
  const int ntab = (l * p * 4 + kDeformUnroll - 1) / kDeformUnroll * kDeformUnroll;
  // as few lanes per pair as cover a corner row (4 for 16-bit D = 32: every lane of a gather busy),
  // but at least 8 when the corner tables of 16 pairs per wave would pass 64 KB of LDS
  int shift = 2;
  if ((size_t)(kDeformThreads / 64) * 16 * ntab * sizeof(int2) > 65536) shift = 3;
  while ((1 << shift) < lanes && shift < 6) ++shift;
  const int ppw = 64 >> shift;
  const long pairs = (long)b * q * h;
  const long waves = (pairs + ppw - 1) / ppw;
  const long blocks = (waves + kDeformThreads / 64 - 1) / (kDeformThreads / 64);
  const size_t lds = (size_t)(kDeformThreads / 64) * ppw * ntab * sizeof(int2);
  hipLaunchKernelGGL((deform_attn_gather_kernel<T, VEC, NC>), dim3((unsigned)blocks), dim3(kDeformThreads), lds,
                     stream, (const T*)value, src, (T*)out, b, s, q, h, d, l, p, shift, ntab, lv);
  return hipGetLastError();
}

template <typename T, int VEC, int NC>
static hipError_t pick_deform(const void* value, PointSrc<T> src, void* out, int b, int s, int q, int h, int d, int l,
                              int p, const Levels& lv, hipStream_t stream) {
  // byte offsets into value, plus a row, stay below the skip marker
  const long block_bytes = ((long)b * s * h * d + d) * (long)sizeof(T);
  if (d % VEC == 0 && block_bytes < (long)kDeformSkip)
    return launch_gather<T, VEC, NC>(value, src, out, b, s, q, h, d, l, p, lv, stream);
  if (d % VEC == 0) return launch_deform<T, VEC, NC>(value, src, out, b, s, q, h, d, l, p, lv, stream);
  return launch_deform<T, 1, NC>(value, src, out, b, s, q, h, d, l, p, lv, stream);
}

static Levels make_levels(int l, const int* shapes) {
  Levels lv{};
  int start = 0;
  for (int i = 0; i < l; ++i) {
    lv.h[i] = shapes[2 * i];
    lv.w[i] = shapes[2 * i + 1];
    lv.start[i] = start;
    start += lv.h[i] * lv.w[i];
  }
  return lv;
}

template <typename T>
static hipError_t pick_nc(const void* value, const void* a, const void* w, const void* refs, int nc, void* out, int b,
                          int s, int q, int h, int d, int l, int p, const Levels& lv, hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(T);
  const PointSrc<T> src{(const T*)a, (const T*)w, (const T*)refs, (float)(1.0 / (double)p)};
  if (nc == 2) return pick_deform<T, VEC, 2>(value, src, out, b, s, q, h, d, l, p, lv, stream);
  if (nc == 4) return pick_deform<T, VEC, 4>(value, src, out, b, s, q, h, d, l, p, lv, stream);
  return pick_deform<T, VEC, 0>(value, src, out, b, s, q, h, d, l, p, lv, stream);
}

static hipError_t deform_dispatch(int dtype, const void* value, const void* a, const void* w, const void* refs, int nc,
                                  void* out, int b, int s, int q, int h, int d, int l, int p, const int* shapes,
                                  hipStream_t stream) {
  const Levels lv = make_levels(l, shapes);
  if (dtype == kF32) return pick_nc<float>(value, a, w, refs, nc, out, b, s, q, h, d, l, p, lv, stream);
  if (dtype == kF16) return pick_nc<f16>(value, a, w, refs, nc, out, b, s, q, h, d, l, p, lv, stream);
  return pick_nc<bf16>(value, a, w, refs, nc, out, b, s, q, h, d, l, p, lv, stream);
}

// Checked by the caller: 1 <= l <= 4, l * p <= 64, sum of level sizes == s, offsets fit in int32.
hipError_t deform_attn(int dtype, const void* value, const void* loc, const void* attn, void* out, int b, int s,
                       int q, int h, int d, int l, int p, const int* shapes, hipStream_t stream) {
  return deform_dispatch(dtype, value, loc, attn, nullptr, 0, out, b, s, q, h, d, l, p, shapes, stream);
}

// Deform::forward between its projections: offsets, logits and reference points (ncoord 2 or 4) in
// place of loc and attn. Same checks as deform_attn, plus ncoord in {2, 4}.
hipError_t deform_core(int dtype, const void* value, const void* offsets, const void* logits, const void* refs,
                       int ncoord, void* out, int b, int s, int q, int h, int d, int l, int p, const int* shapes,
                       hipStream_t stream) {
  return deform_dispatch(dtype, value, offsets, logits, refs, ncoord, out, b, s, q, h, d, l, p, shapes, stream);
}

}  // namespace samhip
