// Fused SAM ViT attention with the decomposed relative-position bias, f16 / bf16, for gfx950.
//
//   out[bh, r, :] = softmax_k( scale * q[r] . k[k] + q[r] . Th[i - kh + H-1] + q[r] . Tw[j - kw + W-1] ) . v
//   r = i*W + j (query), k = kh*W + kw (key), Th = table rows [0, 2H-1), Tw = rows [2H-1, 2H-1 + 2W-1)
//
// This is the whole of the reference's GPU sequence bmm(q, kT) -> relpos_softmax -> bmm(P, v)
// (sam1/encoder.rs:79-82, kernels.rs:12-43 and 899-924) in one kernel, without the N x N score matrix.
// Inputs use the reference layouts: q [BH, N, hd], kT [BH, hd, N] (as qkv_split writes it), v [BH, N, hd].
//
// Work decomposition (one workgroup = NW waves of 64 lanes, one (bh, 32*NW-query block)):
//   * every wave owns 32 queries; scores are computed transposed, S^T = K . Q^T, on
//     v_mfma_f32_32x32x16 so that each lane holds one query (lane % 32) and 16 keys per 32-key block;
//     the row softmax then needs one cross-lane exchange (lane ^ 32) per tile, done with v_permlane32_swap;
//   * O^T = V^T . P^T reuses the S^T accumulators as the B operand directly (a fixed key permutation
//     that the V^T fragment addresses follow), so P never moves between lanes;
//   * key tiles of 64 "slots" are staged in LDS in the reference layouts; ds_read_b64_tr_b16 turns
//     both the kT tile ([hd][keys]) and the V tile ([keys][hd]) into MFMA operands with the reduction
//     dimension packed per lane, so no transpose pass is needed anywhere;
//   * a tile covers whole key rows of the H x W grid: 4 rows padded to 16 columns (W <= 16), 2 rows
//     padded to 32 (W <= 32) or 1 row padded to 64 (W <= 64). Each lane's keys then always sit at the
//     same columns, so the Rw part of the bias lives in registers for the whole loop and the Rh part is
//     one LDS read per 32-key block; both are computed once in a prologue as Q . Tw^T and Q . Th^T on the
//     MFMA, then scattered along the diagonal band;
//   * online softmax in the exp2 domain; the running max is only raised when a tile exceeds it by more
//     than 8 (log2 units), so the O rescale is skipped on almost every tile (p <= 2^8 stays exact enough
//     in f16/bf16 and far from overflow).
#include "relpos_geom.hpp"

namespace samhip {

template <int VK> struct KChunk;
template <> struct KChunk<8> { typedef u32x4 type; };
template <> struct KChunk<2> { typedef unsigned int type; };
template <> struct KChunk<1> { typedef unsigned short type; };

constexpr float kRescaleSlack = 8.0f;

// LDS strides in elements: padded so the transpose reads of consecutive rows start in different banks.
constexpr int kKStride = 64 + 8;
template <int HDP> struct VGeom {
  static constexpr int MBO = (HDP + 31) / 32;  // 32-row blocks of O^T
  static constexpr int STRIDE = MBO * 32 + 8;
};

template <typename T, int HDP, int MODE, int VK, int NW>
__global__ __launch_bounds__(NW * 64) void attn_relpos_kernel(const T* __restrict__ q, const T* __restrict__ kt,
                                                             const T* __restrict__ v, const T* __restrict__ table,
                                                             T* __restrict__ out, int hd, int H, int W, float scale) {
  typedef KeyGeom<MODE> G;
  typedef typename Vec<T>::x8 X8;
  constexpr bool kSplitP = __is_same(T, bf16);
  constexpr int KS = HDP / 16;
  constexpr int MBO = VGeom<HDP>::MBO;
  constexpr int VSTR = VGeom<HDP>::STRIDE;
  constexpr int NT = NW * 64;
  constexpr int KBUF = HDP * kKStride;  // elements per K buffer
  constexpr int VBUF = 64 * VSTR;       // elements per V buffer

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* ks_base = reinterpret_cast<T*>(smem);
  T* vs_base = ks_base + 2 * KBUF;
  float* rhs_base = reinterpret_cast<float*>(vs_base + 2 * VBUF);

  const int N = H * W;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;
  const long bh = blockIdx.y;
  const int qidx = (blockIdx.x * NW + wave) * 32 + n;
  const bool qvalid = qidx < N;
  const int qi = qvalid ? qidx / W : 0, qj = qvalid ? qidx % W : 0;
  float* rhs = rhs_base + wave * 64 * 32;  // [row][query lane], up to 64 rows

  // ---- Q fragments (B operand of S^T = K Q^T): lane supplies Q[query n][16*ks + 8*hh + j]
  X8 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int c = 16 * s + 8 * hh;
    if (qvalid && c < hd)
      qf[s] = __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(q + (bh * N + qidx) * hd + c));
    else
      qf[s] = X8{};
  }

  // ---- prologue: G = T . Q^T on the MFMA, scattered along the diagonal band (log2 units).
  // Rw first (into the rhs scratch), copied to registers; then Rh into rhs, which stays for the loop.
  const T* th = table;
  const T* tw = table + (long)(2 * H - 1) * hd;
  auto band = [&](const T* tab, int rows, int base, int len) {
    for (int r0 = 0; r0 < rows; r0 += 32) {
      f32x16 acc = {};
      const int r = r0 + n;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int c = 16 * s + 8 * hh;
        X8 a = X8{};
        if (r < rows && c < hd) a = __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(tab + (long)r * hd + c));
        acc = mma32(a, qf[s], acc);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = r0 + 8 * (e >> 2) + 4 * hh + (e & 3);
        const int k = base + len - 1 - rr;  // kh = i + H-1 - rr, kw = j + W-1 - rr
        if (rr < rows && k >= 0 && k < len) rhs[k * 32 + n] = acc[e] * kLog2e;
      }
    }
  };
  band(tw, 2 * W - 1, qj, W);
  __syncthreads();
  float rw[G::RWN];
#pragma unroll
  for (int mb = 0; mb < (MODE == kRow64 ? 2 : 1); ++mb)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int c = G::col(mb, e, hh);
      rw[G::rw_index(mb, e)] = c < W ? rhs[c * 32 + n] : -INFINITY;
    }
  __syncthreads();
  band(th, 2 * H - 1, qi, H);

  // zero the V padding columns (read by the last O^T block when HDP is not a multiple of 32)
  for (int i = tid; i < 2 * 64; i += NT) {
    T* rowp = vs_base + (i >> 6) * VBUF + (i & 63) * VSTR;
    for (int c = HDP; c < VSTR; ++c) rowp[c] = from_f32<T>(0.f);
  }

  // ---- key tiles
  typedef typename KChunk<VK>::type KV;
  constexpr int KCPR = 64 / VK;           // K chunks per hd row
  constexpr int KCH = HDP * KCPR;         // K chunks per tile
  constexpr int KPT = (KCH + NT - 1) / NT;
  constexpr int VCPR = HDP / 8;           // V chunks per key slot
  constexpr int VCH = 64 * VCPR;
  constexpr int VPT = (VCH + NT - 1) / NT;
  KV kreg[KPT];
  u32x4 vreg[VPT];
  const T* ktb = kt + bh * hd * (long)N;
  const T* vb = v + bh * (long)N * hd;

  auto load_tile = [&](int t) {
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * NT;
      const int d = c / KCPR, s0 = (c % KCPR) * VK;
      const int rho = s0 / G::WP, kap = s0 % G::WP, row = t * G::RPT + rho;
      KV val = KV{};
      if (c < KCH && d < hd && kap < W && row < H)
        val = *reinterpret_cast<const KV*>(ktb + (long)d * N + row * W + kap);
      kreg[u] = val;
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * NT;
      const int sl = c / VCPR, d0 = (c % VCPR) * 8;
      const int rho = sl / G::WP, kap = sl % G::WP, row = t * G::RPT + rho;
      u32x4 val = u32x4{};
      if (c < VCH && d0 < hd && kap < W && row < H)
        val = *reinterpret_cast<const u32x4*>(vb + (long)(row * W + kap) * hd + d0);
      vreg[u] = val;
    }
  };
  auto store_tile = [&](int buf) {
    T* kbuf = ks_base + buf * KBUF;
    T* vbuf = vs_base + buf * VBUF;
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * NT;
      if (c < KCH) {
        const int d = c / KCPR, s0 = (c % KCPR) * VK;
        *reinterpret_cast<KV*>(kbuf + d * kKStride + s0) = kreg[u];
      }
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * NT;
      if (c < VCH) {
        const int sl = c / VCPR, d0 = (c % VCPR) * 8;
        *reinterpret_cast<u32x4*>(vbuf + sl * VSTR + d0) = vreg[u];
      }
    }
  };

  // per-lane constant parts of the transpose-read addresses
  // K (A operand of S^T): source lane (4*s + c) of group g reads hd row 8*(g>>1) + s (+16*ks + 4*r),
  // slots slot(mb, 16*(g&1) + 4*c) .. +3
  int koff[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) koff[mb] = (8 * (g >> 1) + (gi >> 2)) * kKStride + G::slot(mb, 16 * (g & 1) + 4 * (gi & 3));
  // V^T (A operand of O^T): source lane (4*s + c) reads slot of logical key 8*(g>>1) + 4*r + s of k-step u,
  // hd columns 32*ob + 16*(g&1) + 4*c .. +3
  int voff[4][2];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int ms = 16 * (u & 1) + 8 * r + 4 * (g >> 1) + (gi >> 2);
      voff[u][r] = G::slot(u >> 1, ms) * VSTR + 16 * (g & 1) + 4 * (gi & 3);
    }

  const float sc = scale * kLog2e;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[MBO];
#pragma unroll
  for (int ob = 0; ob < MBO; ++ob) o[ob] = f32x16{};

  const int ntiles = (H + G::RPT - 1) / G::RPT;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load_tile(t + 1);
    const T* kbuf = ks_base + buf * KBUF;
    const T* vbuf = vs_base + buf * VBUF;

    // S^T = K . Q^T for the two 32-key blocks
    f32x16 s[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      s[mb] = f32x16{};
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const T* p = kbuf + koff[mb] + 16 * k * kKStride;
        const X8 a = join8<T>(lds_read_tr16(p), lds_read_tr16(p + 4 * kKStride));
        s[mb] = mma32(a, qf[k], s[mb]);
      }
    }

    // bias and online softmax (exp2 domain)
    float rh[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int row = t * G::RPT + G::row(mb, hh);
      rh[mb] = row < H ? rhs[row * 32 + n] : -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      float mm = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float x = fmaf(s[mb][e], sc, rw[G::rw_index(mb, e)]);
        s[mb][e] = x;
        mm = fmaxf(mm, x);
      }
      mt = fmaxf(mt, mm + rh[mb]);
    }
    mt = max_with_partner32(mt);
    if (wave_any(mt > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = exp2_fast(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int ob = 0; ob < MBO; ++ob) o[ob] *= alpha;
      m_run = m_new;
    }
    float lsum = 0.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const float c = rh[mb] - m_run;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = exp2_fast(s[mb][e] + c);
        s[mb][e] = p;
        lsum += p;
      }
    }
    l_run += lsum;

    // O^T += V^T . P^T. In bf16, P (8 significant bits) is split into two bf16 terms, hi + lo, so the
    // product keeps ~16 bits of P: one bf16 rounding of P alone would cost ~2^-9 of every output.
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = s[u >> 1][8 * (u & 1) + j];
      const X8 b = pack8(pv, (X8*)nullptr);
      X8 blo;
      if (kSplitP) {
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] -= to_f32(b[j]);
        blo = pack8(pv, (X8*)nullptr);
      }
#pragma unroll
      for (int ob = 0; ob < MBO; ++ob) {
        const T* p0 = vbuf + voff[u][0] + 32 * ob;
        const T* p1 = vbuf + voff[u][1] + 32 * ob;
        const X8 a = join8<T>(lds_read_tr16(p0), lds_read_tr16(p1));
        o[ob] = mma32(a, b, o[ob]);
        if (kSplitP) o[ob] = mma32(a, blo, o[ob]);
      }
    }

    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane holds O^T[32*ob + 8*a + 4*hh + b][query n]
  const float inv = 1.f / sum_with_partner32(l_run);
  if (qvalid) {
    T* orow = out + (bh * N + qidx) * hd;
#pragma unroll
    for (int ob = 0; ob < MBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * ob + 8 * a + 4 * hh;
        if (d0 < hd) {
          typename Vec<T>::x4 w4;
#pragma unroll
          for (int b = 0; b < 4; ++b) w4[b] = from_f32<T>(o[ob][4 * a + b] * inv);
          *reinterpret_cast<typename Vec<T>::x4*>(orow + d0) = w4;
        }
      }
  }
}

// ---------------------------------------------------------------------------------------------- launch

template <typename T, int HDP, int MODE, int VK, int NW>
static hipError_t launch_attn(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                              int hd, int h, int w, float scale, hipStream_t stream) {
  constexpr int VSTR = VGeom<HDP>::STRIDE;
  const size_t lds = (size_t)(2 * HDP * kKStride + 2 * 64 * VSTR) * sizeof(T) + (size_t)NW * 64 * 32 * sizeof(float);
  auto kern = attn_relpos_kernel<T, HDP, MODE, VK, NW>;
  static bool attr_set = false;  // one-time opt-in to more than 64 KB of dynamic LDS
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int n = h * w;
  dim3 grid((n + 32 * NW - 1) / (32 * NW), bh);
  hipLaunchKernelGGL(kern, grid, dim3(NW * 64), lds, stream, (const T*)q, (const T*)kt, (const T*)v,
                     (const T*)table, (T*)out, hd, h, w, scale);
  return hipGetLastError();
}

template <typename T, int HDP, int MODE, int VK>
static hipError_t pick_nw(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                          int h, int w, float scale, hipStream_t stream) {
  if (h * w > 1024) return launch_attn<T, HDP, MODE, VK, 8>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return launch_attn<T, HDP, MODE, VK, 4>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

template <typename T, int HDP, int MODE>
static hipError_t pick_vk(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                          int h, int w, float scale, hipStream_t stream) {
  const int n = h * w;
  if (w % 8 == 0 && n % 8 == 0) return pick_nw<T, HDP, MODE, 8>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (w % 2 == 0 && n % 2 == 0) return pick_nw<T, HDP, MODE, 2>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return pick_nw<T, HDP, MODE, 1>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

template <typename T, int HDP>
static hipError_t pick_mode(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                            int h, int w, float scale, hipStream_t stream) {
  if (w <= 16) return pick_vk<T, HDP, kPair>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (w <= 32) return pick_vk<T, HDP, kRow32>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return pick_vk<T, HDP, kRow64>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

template <typename T>
static hipError_t pick_hd(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                          int h, int w, float scale, hipStream_t stream) {
  if (hd <= 16) return pick_mode<T, 16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 32) return pick_mode<T, 32>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 64) return pick_mode<T, 64>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 80) return pick_mode<T, 80>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return pick_mode<T, 128>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

// Shape limits are checked by the caller (sam_hip_abi.cpp): 1 <= h, w <= 64, hd % 8 == 0, hd <= 128.
hipError_t attn_relpos_half(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out,
                            int bh, int hd, int h, int w, float scale, hipStream_t stream) {
  if (dtype == kF16) return pick_hd<f16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return pick_hd<bf16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

}  // namespace samhip
