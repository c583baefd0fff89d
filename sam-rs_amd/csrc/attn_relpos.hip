// Fused SAM ViT attention with the decomposed relative-position bias, f16 / bf16, for gfx950.
//
//   out[bh, r, :] = softmax_k( scale * q[r] . k[k] + q[r] . Th[i - kh + H-1] + q[r] . Tw[j - kw + W-1] ) . v
//   r = i*W + j (query), k = kh*W + kw (key), Th = table rows [0, 2H-1), Tw = rows [2H-1, 2H-1 + 2W-1)
//
// This is the whole of the reference's GPU sequence bmm(q, kT) -> relpos_softmax -> bmm(P, v)
// (sam1/encoder.rs:79-82, kernels.rs:12-43 and 899-924) in one kernel, without the N x N score matrix.
// Inputs use the reference layouts: q [BH, N, hd], kT [BH, hd, N] (as qkv_split writes it), v [BH, N, hd].
//
// Work decomposition (one workgroup = 8 waves of 64 lanes = one (bh, 256-query block)):
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
//     same columns, so the Rw part of the bias is constant per lane for the whole loop: it is the
//     initial accumulator (C operand, pre-divided by the scale) of every S^T MFMA, which adds it for
//     free. The Rh part is one LDS read per 32-key block. Both come from a prologue that computes
//     Q . Tw^T and Q . Th^T on the MFMA (the table staged once in LDS) and scatters them along the
//     diagonal band;
//   * online softmax in the exp2 domain: per score one max3 share, one FMA (scale and the Rh term),
//     one exp2 and half a pack; the running max is only raised when a tile exceeds it by more than 8
//     (log2 units), so the O rescale is skipped on almost every tile (p <= 2^8 stays exact enough in
//     f16/bf16 and far from overflow);
//   * when hd is not a multiple of 32 (hd 80 -> 96 rows of O^T), a column of ones in V's padding makes
//     the spare O^T row accumulate the softmax denominator on the MFMA;
//   * the S^T of tile t+1 is issued on the MFMA while tile t's exponentials run on the VALU;
//   * two ways to feed K/V: "resident" (NBUF = 4: grids of at most 4 tiles, e.g. the 14x14 windows)
//     loads every tile in the same round trip as Q and the table and then runs the key loop with no
//     loads and no barriers; "streaming" (NBUF = 2: the 64x64 global grid) double-buffers the tiles,
//     K one tile ahead of V, with the next tiles' global loads in flight during the compute and one
//     barrier per tile;
//   * workgroups are numbered XCD-major, so all query blocks of a head run on one XCD and share its L2.
#include "relpos_geom.hpp"

namespace samhip {

template <int VK> struct KChunk;
template <> struct KChunk<8> { typedef u32x4 type; };
template <> struct KChunk<2> { typedef unsigned int type; };
template <> struct KChunk<1> { typedef unsigned short type; };

constexpr float kRescaleSlack = 8.0f;
constexpr int kMaxWaves = 8;

// LDS strides in elements. A transpose read has each group of 16 lanes fetch 4 rows x 4 chunks of
// 8 bytes; the row strides below move consecutive rows by 8 (or 24) banks of the 32.
constexpr int kKStride = 64 + 16;
template <int HDP> struct VGeom {
  static constexpr int MBO = (HDP + 31) / 32;  // 32-row blocks of O^T
  static constexpr int STRIDE = MBO * 32 + 16;
  static constexpr bool ONES = MBO * 32 > HDP;  // a spare O^T row carries the denominator
};

template <typename T, int HDP, int NBUF>
__host__ __device__ constexpr size_t tiles_lds_bytes() {
  return (size_t)(NBUF * HDP * kKStride + NBUF * 64 * VGeom<HDP>::STRIDE) * sizeof(T);
}

// Workgroup i runs on XCD i % 8; give each XCD a contiguous range of (bh, query block) pairs.
__device__ __forceinline__ int xcd_major_block(int i, int total) {
  const int per = total >> 3, rem = total & 7, x = i & 7, j = i >> 3;
  return x * per + (x < rem ? x : rem) + j;
}

// NBUF = 4: resident (needs ntiles <= 4). FULL: every chunk of every tile is in range (hd == HDP,
// W == padded row width, H a multiple of the rows per tile), so the range checks compile away.
template <typename T, int HDP, int MODE, int VK, bool POS, int NBUF, bool FULL, int NWV>
__global__ __launch_bounds__(NWV * 64) void attn_relpos_kernel(const T* __restrict__ q, const T* __restrict__ kt,
                                                              const T* __restrict__ v, const T* __restrict__ table,
                                                              T* __restrict__ out, int hd, int H, int W,
                                                              float scale, int qblocks) {
  typedef KeyGeom<MODE> G;
  typedef typename Vec<T>::x8 X8;
  constexpr int kWaves = NWV, kThreads = NWV * 64;
  constexpr bool RES = NBUF > 2;
  constexpr bool kSplitP = __is_same(T, bf16);
  constexpr int KS = HDP / 16;
  constexpr int MBO = VGeom<HDP>::MBO;
  constexpr int VSTR = VGeom<HDP>::STRIDE;
  constexpr bool kOnes = VGeom<HDP>::ONES;
  constexpr int KBUF = HDP * kKStride;  // elements per K buffer
  constexpr int VBUF = 64 * VSTR;       // elements per V buffer

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* ks_base = reinterpret_cast<T*>(smem);
  T* vs_base = ks_base + NBUF * KBUF;
  float* rhs_base = reinterpret_cast<float*>(vs_base + NBUF * VBUF);
  T* tbl = ks_base;  // the rel-pos table, during the prologue only (aliases the tile buffers)

  const int N = H * W;
  const int R = H > W ? H : W;  // rows of the per-wave bias scratch
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;
  const int blk = xcd_major_block(blockIdx.x, gridDim.x);
  const long bh = blk / qblocks;
  const int q0 = (blk % qblocks) * (kWaves * 32) + wave * 32;
  const bool active = q0 < N;  // whole wave: at least one of its 32 queries exists
  const int qidx = q0 + n;
  const bool qvalid = qidx < N;
  const int qi = qvalid ? qidx / W : 0, qj = qvalid ? qidx % W : 0;
  float* rhs = rhs_base + wave * (R + 1) * 32;  // [row][query lane]; row R takes discarded scatters
  const int ntiles = (H + G::RPT - 1) / G::RPT;

  // ---- K/V tile staging: global -> registers -> LDS. Loads are unconditional (an out-of-range chunk
  // reads the tile base instead) and the zero fill is applied when the registers are written to LDS,
  // so no branch or early wait sits between a load's issue and the work that hides its latency.
  typedef typename KChunk<VK>::type KV;
  constexpr int KCPR = 64 / VK;  // K chunks per hd row
  constexpr int KCH = HDP * KCPR;
  constexpr int KPT = (KCH + kThreads - 1) / kThreads;
  constexpr int VCPR = HDP / 8;  // V chunks per key slot
  constexpr int VCH = 64 * VCPR;
  constexpr int VPT = (VCH + kThreads - 1) / kThreads;
  constexpr int NSET = RES ? NBUF : 2;  // register sets: every tile (resident) or K(t+2), V(t+1)
  KV kreg[NSET][KPT];
  u32x4 vreg[NSET][VPT];
  bool kok[NSET][KPT], vok[NSET][VPT];
  const T* ktb = kt + bh * hd * (long)N;
  const T* vb = v + bh * (long)N * hd;
  auto load_k = [&](int set, int t) {
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * kThreads;
      const int d = c / KCPR, s0 = (c % KCPR) * VK;
      const int rho = s0 / G::WP, kap = s0 % G::WP, row = t * G::RPT + rho;
      const bool inr = KCH % kThreads == 0 || c < KCH;
      const bool ok = FULL ? inr : (inr && d < hd && kap < W && row < H);
      kok[set][u] = ok;
      kreg[set][u] = *reinterpret_cast<const KV*>(ktb + (ok ? (long)d * N + row * W + kap : 0));
    }
  };
  auto load_v = [&](int set, int t) {
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * kThreads;
      const int sl = c / VCPR, d0 = (c % VCPR) * 8;
      const int rho = sl / G::WP, kap = sl % G::WP, row = t * G::RPT + rho;
      const bool inr = VCH % kThreads == 0 || c < VCH;
      const bool ok = FULL ? inr : (inr && d0 < hd && kap < W && row < H);
      vok[set][u] = ok;
      vreg[set][u] = *reinterpret_cast<const u32x4*>(vb + (ok ? (long)(row * W + kap) * hd + d0 : 0));
    }
  };
  auto store_k = [&](int set, int buf) {
    T* kbuf = ks_base + buf * KBUF;
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * kThreads;
      if (KCH % kThreads == 0 || c < KCH)
        *reinterpret_cast<KV*>(kbuf + (c / KCPR) * kKStride + (c % KCPR) * VK) =
            (FULL || kok[set][u]) ? kreg[set][u] : KV{};
    }
  };
  auto store_v = [&](int set, int buf) {
    T* vbuf = vs_base + buf * VBUF;
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * kThreads;
      if (VCH % kThreads == 0 || c < VCH)
        *reinterpret_cast<u32x4*>(vbuf + (c / VCPR) * VSTR + (c % VCPR) * 8) =
            (FULL || vok[set][u]) ? vreg[set][u] : u32x4{};
    }
  };

  // ---- one round trip for everything the prologue needs: tiles, Q, the table
  if (RES) {
#pragma unroll
    for (int t = 0; t < NBUF; ++t) {
      const int tc = t < ntiles ? t : ntiles - 1;
      load_k(t, tc);
      load_v(t, tc);
    }
  } else {
    load_k(0, 0);
    load_v(0, 0);
    load_k(1, ntiles > 1 ? 1 : 0);
  }
  // Q fragments (B operand of S^T = K Q^T): lane supplies Q[query n][16*ks + 8*hh + j]
  X8 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int c = 16 * s + 8 * hh;
    qf[s] = (qvalid && c < hd) ? __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(q + (bh * N + qidx) * hd + c))
                               : X8{};
  }
  const int trows = 2 * H - 1 + 2 * W - 1;
  {
    // the table (at most (2*64-1) + (2*64-1) = 254 rows) -> LDS rows of HDP elements, zero beyond hd
    constexpr int TCPR = HDP / 8;
    constexpr int TPT = (254 * TCPR + kThreads - 1) / kThreads;
    u32x4 treg[TPT];
#pragma unroll
    for (int u = 0; u < TPT; ++u) {
      const int c = tid + u * kThreads;
      const int r = c / TCPR, col = (c % TCPR) * 8;
      const bool ok = r < trows && col < hd;
      treg[u] = *reinterpret_cast<const u32x4*>(table + (ok ? (long)r * hd + col : 0));
      if (!ok) treg[u] = u32x4{};
    }
#pragma unroll
    for (int u = 0; u < TPT; ++u) {
      const int c = tid + u * kThreads;
      if (c < trows * TCPR) *reinterpret_cast<u32x4*>(tbl + c * 8) = treg[u];
    }
  }
  __syncthreads();

  // ---- prologue: G = T . Q^T on the MFMA, scattered along the diagonal band (log2 units).
  // All row blocks of both tables are multiplied first (independent MFMA chains, the table rows read
  // from LDS without masks: rows past the end hold other rows or zeros and are never scattered); then
  // Rw is scattered into the rhs scratch and copied to registers, and Rh is scattered into rhs, which
  // stays for the loop. Scatter stores are branch-free: entries outside the band go to a junk row.
  // row blocks per table: ceil((2W-1)/32) is 1 for W <= 16, 2 for W <= 32, 4 for W <= 64; resident
  // grids have H <= 16.
  constexpr int MAXBW = MODE == kPair ? 1 : (MODE == kRow32 ? 2 : 4);
  constexpr int MAXBH = RES ? 1 : 4;
  const int nbw = (2 * W - 1 + 31) / 32, nbh = (2 * H - 1 + 31) / 32;
  f32x16 gw[MAXBW], gh[MAXBH];
  if (active) {
#pragma unroll
    for (int b = 0; b < MAXBW; ++b) gw[b] = f32x16{};
#pragma unroll
    for (int b = 0; b < MAXBH; ++b) gh[b] = f32x16{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int b = 0; b < MAXBW; ++b) {
        if (b < nbw) {
          const X8 a = *reinterpret_cast<const X8*>(tbl + (2 * H - 1 + 32 * b + n) * HDP + 16 * s + 8 * hh);
          gw[b] = mma32(a, qf[s], gw[b]);
        }
      }
#pragma unroll
      for (int b = 0; b < MAXBH; ++b) {
        if (b < nbh) {
          const X8 a = *reinterpret_cast<const X8*>(tbl + (32 * b + n) * HDP + 16 * s + 8 * hh);
          gh[b] = mma32(a, qf[s], gh[b]);
        }
      }
    }
  }
  auto scatter = [&](const f32x16* gb, int nb, int maxb, int rows, int base, int len) {
#pragma unroll
    for (int b = 0; b < MAXBW + MAXBH; ++b) {
      if (b >= maxb) break;
      if (b < nb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rr = 32 * b + 8 * (e >> 2) + 4 * hh + (e & 3);
          const int k = base + len - 1 - rr;  // kh = i + H-1 - rr, kw = j + W-1 - rr
          const bool ok = rr < rows && k >= 0 && k < len;
          rhs[(ok ? k : R) * 32 + n] = gb[b][e] * kLog2e;
        }
      }
    }
  };
  if (active) scatter(gw, nbw, MAXBW, 2 * W - 1, qj, W);
  __syncthreads();
  const float sc = scale * kLog2e;
  // POS: the C operand of the S^T MFMAs is Rw / sc, so the accumulator ends as S + Rw/sc.
  // Otherwise the plain Rw values (log2 units), added after the MFMA.
  f32x16 cinit[2];
  {
    const float f = POS ? 1.f / sc : 1.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int c = G::col(mb, e, hh);
        cinit[mb][e] = c < W ? rhs[c * 32 + n] * f : -INFINITY;
      }
  }
  __syncthreads();
  if (active) scatter(gh, nbh, MAXBH, 2 * H - 1, qi, H);
  __syncthreads();  // the table region is free from here on

  // tiles into LDS; V padding columns: a column of ones (the denominator row of O^T) then zeros
  if (RES) {
#pragma unroll
    for (int t = 0; t < NBUF; ++t) {
      store_k(t, t);
      store_v(t, t);
    }
  } else {
    store_k(0, 0);
    store_v(0, 0);
    store_k(1, 1);
  }
  for (int i = tid; i < NBUF * 64; i += kThreads) {
    T* rowp = vs_base + (i >> 6) * VBUF + (i & 63) * VSTR;
    for (int c = HDP; c < VSTR; ++c) rowp[c] = from_f32<T>((kOnes && c == HDP) ? 1.f : 0.f);
  }
  __syncthreads();

  // per-lane constant parts of the transpose-read addresses
  // K (A operand of S^T): source lane (4*s + c) of group g reads hd row 8*(g>>1) + s (+16*ks + 4*r),
  // slots slot(mb, 16*(g&1) + 4*c) .. +3
  int koff[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
    koff[mb] = (8 * (g >> 1) + (gi >> 2)) * kKStride + G::slot(mb, 16 * (g & 1) + 4 * (gi & 3));
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

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[MBO];
#pragma unroll
  for (int ob = 0; ob < MBO; ++ob) o[ob] = f32x16{};

  auto qk = [&](const T* kbuf, f32x16* s) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const T* p = kbuf + koff[mb] + 16 * k * kKStride;
        const X8 a = join8<T>(lds_read_tr16(p), lds_read_tr16(p + 4 * kKStride));
        if (k == 0)
          s[mb] = mma32(a, qf[0], POS ? cinit[mb] : f32x16{});
        else
          s[mb] = mma32(a, qf[k], s[mb]);
      }
    }
  };

  // Softmax and P.V of tile t (scores in s_cur) with the S^T of tile t+1 into s_nxt. Near the end
  // the loads, stores and the next S^T run on clamped tile indices and their results go unused: the
  // loop body stays free of branches around them.
  auto step = [&](int t, f32x16* s_cur, f32x16* s_nxt) {
    const int kb_next = RES ? (t + 1 < ntiles ? t + 1 : t) : ((t + 1) & 1);
    const int vb_cur = RES ? t : (t & 1);
    if (!RES) {
      load_k(0, t + 2 < ntiles ? t + 2 : ntiles - 1);
      load_v(0, t + 1 < ntiles ? t + 1 : ntiles - 1);
    }
    if (active) {
      float rh[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int row = t * G::RPT + G::row(mb, hh);
        rh[mb] = row < H ? rhs[row * 32 + n] : -INFINITY;
      }
      float mt = -INFINITY;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        if (!POS) {
#pragma unroll
          for (int e = 0; e < 16; ++e) s_cur[mb][e] = fmaf(s_cur[mb][e], sc, cinit[mb][e]);
        }
        float mm = s_cur[mb][0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mm = max_nc(mm, s_cur[mb][e]);
        mt = max_nc(mt, POS ? fmaf(mm, sc, rh[mb]) : mm + rh[mb]);
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
      qk(ks_base + kb_next * KBUF, s_nxt);
      float c[2];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) c[mb] = rh[mb] - m_run;
      X8 b[4], blo[4];
      float lsum = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = s_cur[u >> 1][8 * (u & 1) + j];
          pv[j] = exp2_fast(POS ? fmaf(x, sc, c[u >> 1]) : x + c[u >> 1]);
          if (!kOnes && kSplitP) lsum += pv[j];  // bf16: P.V takes hi + lo, P itself to ~16 bits
        }
        b[u] = pack8(pv, (X8*)nullptr);
        if constexpr (!kOnes && !kSplitP) {
          // f16: the sum over P as the P.V product sees it (rounded), as the ones row gives it when hd
          // leaves a spare O^T row: numerator and denominator weigh each key alike
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int j = 0; j < 8; j += 2)
            lsum = __builtin_amdgcn_fdot2(h2{b[u][j], b[u][j + 1]}, h2{(f16)1.f, (f16)1.f}, lsum, false);
        }
        if (kSplitP) {
#pragma unroll
          for (int j = 0; j < 8; ++j) pv[j] -= to_f32(b[u][j]);
          blo[u] = pack8(pv, (X8*)nullptr);
        }
      }
      if (!kOnes) l_run += lsum;
      // O^T += V^T . P^T. In bf16, P (8 significant bits) is split into two bf16 terms, hi + lo, so
      // the product keeps ~16 bits of P: one bf16 rounding of P would cost ~2^-9 of every output.
      const T* vbuf = vs_base + vb_cur * VBUF;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int ob = 0; ob < MBO; ++ob) {
          const T* p0 = vbuf + voff[u][0] + 32 * ob;
          const T* p1 = vbuf + voff[u][1] + 32 * ob;
          const X8 a = join8<T>(lds_read_tr16(p0), lds_read_tr16(p1));
          o[ob] = mma32(a, b[u], o[ob]);
          if (kSplitP) o[ob] = mma32(a, blo[u], o[ob]);
        }
      }
    }
    if (!RES) {
      store_k(0, t & 1);        // K(t+2) replaces K(t), whose scores were taken one step ago
      store_v(0, (t + 1) & 1);  // V(t+1) replaces V(t-1)
      __syncthreads();
    }
  };

  f32x16 sa[2], sb[2];
  if (active) qk(ks_base, sa);
  if (!RES) __syncthreads();  // every wave has read K(0) before step 0 overwrites its buffer with K(2)
  for (int t = 0; t < ntiles; t += 2) {
    step(t, sa, sb);
    if (t + 1 < ntiles) step(t + 1, sb, sa);
  }

  // ---- normalise and store: lane holds O^T[32*ob + 8*a + 4*hh + b][query n]
  if (active) {
    float l;
    if (kOnes) {
      // the denominator is O^T row HDP (= 32*(MBO-1) + 16): element 8 of the lower lane half
      const unsigned x = __float_as_uint(o[MBO - 1][8]);
      auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
      l = __uint_as_float(r[0]);
    } else {
      l = sum_with_partner32(l_run);
    }
    const float inv = 1.f / l;
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
            for (int bb = 0; bb < 4; ++bb) w4[bb] = from_f32<T>(o[ob][4 * a + bb] * inv);
            *reinterpret_cast<typename Vec<T>::x4*>(orow + d0) = w4;
          }
        }
    }
  }
}

// ---------------------------------------------------------------------------------------------- launch

template <typename T, int HDP, int MODE, int VK, bool POS, int NBUF, bool FULL, int NWV>
static hipError_t launch_attn(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                              int hd, int h, int w, float scale, hipStream_t stream) {
  const int rows = h > w ? h : w;
  const size_t lds = tiles_lds_bytes<T, HDP, NBUF>() + (size_t)NWV * (rows + 1) * 32 * sizeof(float);
  auto kern = attn_relpos_kernel<T, HDP, MODE, VK, POS, NBUF, FULL, NWV>;
  static std::atomic<unsigned long long> lds_done{0};  // opt-in to more than 64 KB of dynamic LDS
  {
    const size_t max_lds = tiles_lds_bytes<T, HDP, NBUF>() + (size_t)NWV * 65 * 32 * sizeof(float);
    const hipError_t e = lds_opt_in(lds_done, (const void*)kern, (int)(max_lds < 163840 ? max_lds : 163840));
    if (e != hipSuccess) return e;
  }
  const int n = h * w;
  const int qblocks = (n + NWV * 32 - 1) / (NWV * 32);  // NWV * 32 queries per workgroup
  const long blocks = (long)bh * qblocks;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(NWV * 64), lds, stream, (const T*)q, (const T*)kt,
                     (const T*)v, (const T*)table, (T*)out, hd, h, w, scale, qblocks);
  return hipGetLastError();
}

template <typename T, int HDP, int MODE, int NBUF, int NWV>
static hipError_t pick_vk(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                          int h, int w, float scale, hipStream_t stream) {
  const int n = h * w;
  if (!(scale > 0.f))  // the generic path: any scale, any alignment
    return launch_attn<T, HDP, MODE, 1, false, NBUF, false, NWV>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (w % 8 == 0 && n % 8 == 0) {
    if (NBUF == 2 && hd == HDP && w == KeyGeom<MODE>::WP && h % KeyGeom<MODE>::RPT == 0)
      return launch_attn<T, HDP, MODE, 8, true, NBUF, true, NWV>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
    return launch_attn<T, HDP, MODE, 8, true, NBUF, false, NWV>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  }
  if (w % 2 == 0 && n % 2 == 0)
    return launch_attn<T, HDP, MODE, 2, true, NBUF, false, NWV>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return launch_attn<T, HDP, MODE, 1, true, NBUF, false, NWV>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

template <typename T, int HDP, int MODE>
static hipError_t pick_nbuf(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                            int h, int w, float scale, hipStream_t stream) {
  const int ntiles = (h + KeyGeom<MODE>::RPT - 1) / KeyGeom<MODE>::RPT;
  const int rows = h > w ? h : w;
  const size_t res_lds = tiles_lds_bytes<T, HDP, 4>() + (size_t)kMaxWaves * (rows + 1) * 32 * sizeof(float);
  if (ntiles <= 4 && res_lds <= 163840)
    return pick_vk<T, HDP, MODE, 4, kMaxWaves>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return pick_vk<T, HDP, MODE, 2, kMaxWaves>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

template <typename T, int HDP>
static hipError_t pick_mode(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                            int h, int w, float scale, hipStream_t stream) {
  if (w <= 16) return pick_nbuf<T, HDP, kPair>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (w <= 32) return pick_nbuf<T, HDP, kRow32>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return pick_nbuf<T, HDP, kRow64>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
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

// Shape limits are checked by the caller (sam_hip_abi.cpp): 1 <= h, w <= 128, hd % 8 == 0, hd <= 128.
bool attn_relpos_window(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                        int hd, int h, int w, float scale, hipStream_t stream, hipError_t* err);
bool attn_relpos_global(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                        int hd, int h, int w, float scale, hipStream_t stream, hipError_t* err);

hipError_t attn_relpos_wide(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out,
                            int bh, int hd, int h, int w, float scale, hipStream_t stream);

hipError_t attn_relpos_half(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out,
                            int bh, int hd, int h, int w, float scale, hipStream_t stream) {
  hipError_t e;
  // grids past 64 rows or columns (up to 128): attn_relpos_wide.hip
  if (h > 64 || w > 64) return attn_relpos_wide(dtype, q, kt, v, table, out, bh, hd, h, w, scale, stream);
  // windowed grids (the 14x14 SAM windows): attn_relpos_win.hip; the 64-column global grid:
  // attn_relpos_glob.hip; every other shape: the general kernel below
  if (attn_relpos_window(dtype, q, kt, v, table, out, bh, hd, h, w, scale, stream, &e)) return e;
  if (attn_relpos_global(dtype, q, kt, v, table, out, bh, hd, h, w, scale, stream, &e)) return e;
  if (dtype == kF16) return pick_hd<f16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return pick_hd<bf16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

}  // namespace samhip
