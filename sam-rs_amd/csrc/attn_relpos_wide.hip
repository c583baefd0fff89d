// Fused rel-pos attention for grids wider or taller than 64 (up to 128 x 128), f16 / bf16, for gfx950:
//
//   out[bh, r, :] = softmax_k( scale * q[r] . k[k] + q[r] . Th[i - kh + H-1] + q[r] . Tw[j - kw + W-1] ) . v
//
// the same contract and arithmetic as attn_relpos.hip (the reference's bmm(q, kT) -> relpos_softmax ->
// bmm(P, v), sam1/encoder.rs:79-82, kernels.rs:12-43, 899-924), for the shapes past that kernel's 64 x 64
// limit. The reference's GPU path takes them only up to h*w <= 8192 (the relpos_softmax row limit,
// kernels.rs:14, 1078-1083) and through a materialised score matrix; here the scores never leave the
// chip, so any grid with h, w <= 128 runs.
//
// What changes against attn_relpos.hip's streaming mode:
//   * a key tile is one 64-column segment of one grid row. A grid of width W > 64 is walked in column
//     passes: pass p takes columns [64p, 64p + 64) of every row, so each lane's keys sit at fixed columns
//     within a pass and the Rw part of the bias stays the initial accumulator of the S^T MFMAs. When
//     the next tile starts a new pass, its Rw values are computed for the new columns (after the current
//     tile's scores have used theirs) before its S^T is issued. The online softmax state carries across
//     passes (the order of keys is free);
//   * the bias tables are multiplied by Q on the MFMA one 32-row block at a time, with the table rows read
//     straight from global memory (16-byte A-operand pieces), so the table needs no LDS: Rw for the 64
//     columns of the current pass, and Rh for 32 grid rows at a time (recomputed every 32 tiles), go
//     through a wave-private scratch of 98 rows of 32 floats;
//   * 8 waves (256 queries, two per SIMD) per workgroup up to hd 80, 4 at hd 128, so that the scratch
//     and the double-buffered K/V tiles fit in LDS.
// Limits (checked by the dispatcher): 1 <= H, W <= 128, hd % 8 == 0, hd <= 128.
#include "relpos_geom.hpp"

namespace samhip {

namespace wide {
constexpr int kRwRows = 65;  // Rw scratch: the pass's 64 columns, then a junk row
constexpr int kRhRows = 33;  // Rh scratch: 32 grid rows, then a junk row
constexpr int kKStride = 64 + 16;  // K tile row stride (elements), as attn_relpos.hip
constexpr float kSlack = 8.0f;
template <int HDP> struct VG {
  static constexpr int MBO = (HDP + 31) / 32;
  static constexpr int STRIDE = MBO * 32 + 16;
  static constexpr bool ONES = MBO * 32 > HDP;
};
template <typename T, int HDP, int NW>
constexpr size_t lds_bytes() {
  return (size_t)(2 * HDP * kKStride + 2 * 64 * VG<HDP>::STRIDE) * sizeof(T) +
         (size_t)NW * (kRwRows + kRhRows) * 32 * sizeof(float);
}
template <int VK> struct KC;
template <> struct KC<8> { typedef u32x4 type; };
template <> struct KC<2> { typedef unsigned int type; };
template <> struct KC<1> { typedef unsigned short type; };
}  // namespace wide

__device__ __forceinline__ int wide_xcd_block(int i, int total) {
  const int per = total >> 3, rem = total & 7, x = i & 7, j = i >> 3;
  return x * per + (x < rem ? x : rem) + j;
}

template <typename T, int HDP, int VK, bool POS, int NW>
__global__ __launch_bounds__(NW * 64) void attn_relpos_wide_kernel(const T* __restrict__ q,
                                                                         const T* __restrict__ kt,
                                                                         const T* __restrict__ v,
                                                                         const T* __restrict__ table,
                                                                         T* __restrict__ out, int hd, int H, int W,
                                                                         float scale, int qblocks) {
  using namespace wide;
  constexpr int kWaves = NW, kThreads = NW * 64;
  typedef KeyGeom<kRow64> G;
  typedef typename Vec<T>::x8 X8;
  constexpr bool kSplitP = __is_same(T, bf16);
  constexpr int KS = HDP / 16, MBO = VG<HDP>::MBO, VSTR = VG<HDP>::STRIDE;
  constexpr bool kOnes = VG<HDP>::ONES;
  constexpr int KBUF = HDP * kKStride, VBUF = 64 * VSTR;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* ks_base = reinterpret_cast<T*>(smem);
  T* vs_base = ks_base + 2 * KBUF;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  float* rw_s = reinterpret_cast<float*>(vs_base + 2 * VBUF) + wave * (kRwRows + kRhRows) * 32;
  float* rh_s = rw_s + kRwRows * 32;

  const int N = H * W;
  const int n = lane & 31, hh = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;
  const int blk = wide_xcd_block(blockIdx.x, gridDim.x);
  const long bh = blk / qblocks;
  const int q0 = (blk % qblocks) * (kWaves * 32) + wave * 32;
  const bool active = q0 < N;
  const int qidx = q0 + n;
  const bool qvalid = qidx < N;
  const int qi = qvalid ? qidx / W : 0, qj = qvalid ? qidx % W : 0;
  const int npass = (W + 63) / 64;
  const int ntiles = npass * H;  // tile gt: pass gt / H, grid row gt % H
  const int trows = 2 * H - 1 + 2 * W - 1;

  // ---- K/V staging (global -> registers -> LDS), two register sets: K(t+2) and V(t+1) in flight.
  // Loads are unconditional (an out-of-range chunk reads the tile base) and the zero fill is applied when
  // the registers are written to LDS.
  typedef typename KC<VK>::type KV;
  constexpr int KCPR = 64 / VK;
  constexpr int KCH = HDP * KCPR;
  constexpr int KPT = (KCH + kThreads - 1) / kThreads;
  constexpr int VCPR = HDP / 8;
  constexpr int VCH = 64 * VCPR;
  constexpr int VPT = (VCH + kThreads - 1) / kThreads;
  KV kreg[2][KPT];
  u32x4 vreg[2][VPT];
  bool kok[2][KPT], vok[2][VPT];
  const T* ktb = kt + bh * hd * (long)N;
  const T* vb = v + bh * (long)N * hd;
  auto load_k = [&](int set, int gt) {
    const int row = gt % H, c0 = 64 * (gt / H);
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * kThreads;
      const int d = c / KCPR, col = c0 + (c % KCPR) * VK;
      const bool ok = (KCH % kThreads == 0 || c < KCH) && d < hd && col < W;
      kok[set][u] = ok;
      kreg[set][u] = *reinterpret_cast<const KV*>(ktb + (ok ? (long)d * N + row * W + col : 0));
    }
  };
  auto load_v = [&](int set, int gt) {
    const int row = gt % H, c0 = 64 * (gt / H);
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * kThreads;
      const int col = c0 + c / VCPR, d0 = (c % VCPR) * 8;
      const bool ok = (VCH % kThreads == 0 || c < VCH) && d0 < hd && col < W;
      vok[set][u] = ok;
      vreg[set][u] = *reinterpret_cast<const u32x4*>(vb + (ok ? (long)(row * W + col) * hd + d0 : 0));
    }
  };
  auto store_k = [&](int set, int buf) {
    T* kbuf = ks_base + buf * KBUF;
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * kThreads;
      if (KCH % kThreads == 0 || c < KCH)
        *reinterpret_cast<KV*>(kbuf + (c / KCPR) * kKStride + (c % KCPR) * VK) = kok[set][u] ? kreg[set][u] : KV{};
    }
  };
  auto store_v = [&](int set, int buf) {
    T* vbuf = vs_base + buf * VBUF;
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * kThreads;
      if (VCH % kThreads == 0 || c < VCH)
        *reinterpret_cast<u32x4*>(vbuf + (c / VCPR) * VSTR + (c % VCPR) * 8) = vok[set][u] ? vreg[set][u] : u32x4{};
    }
  };
  auto wave_sync = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  load_k(0, 0);
  load_v(0, 0);
  load_k(1, ntiles > 1 ? 1 : 0);
  // Q fragments (B operand of S^T = K Q^T): lane supplies Q[query n][16*ks + 8*hh + j]
  X8 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int c = 16 * s + 8 * hh;
    qf[s] = (qvalid && c < hd) ? __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(q + (bh * N + qidx) * hd + c))
                               : X8{};
  }

  // (T . Q^T) for table rows row0 .. row0 + 31 on the MFMA: element e of lane (n, hh) is table row
  // row0 + 8 (e >> 2) + 4 hh + (e & 3) against query n. Rows past the table and columns past hd read 0.
  auto table_block = [&](int row0) __attribute__((always_inline)) {
    f32x16 acc = f32x16{};
    const int r = row0 + n;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int c = 16 * s + 8 * hh;
      const X8 a = (r < trows && c < hd) ? __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(table + (long)r * hd + c))
                                        : X8{};
      acc = mma32(a, qf[s], acc);
    }
    return acc;
  };
  const float sc = scale * kLog2e;
  // Rw of pass p: for this lane's query, the bias of key columns 64p .. 64p + 63 (log2 units), scattered
  // into rw_s from the 32-row blocks of Tw . Q^T (column kw takes table row qj + W-1 - kw), then copied
  // to the S^T start values; columns past W start at -inf.
  f32x16 cinit[2];
  auto rw_pass = [&](int p) __attribute__((always_inline)) {
    const int nbw = (2 * W - 1 + 31) / 32, c0 = 64 * p, c1 = min(W, c0 + 64);
    for (int b = 0; b < nbw; ++b) {
      const f32x16 acc = table_block(2 * H - 1 + 32 * b);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = 32 * b + 8 * (e >> 2) + 4 * hh + (e & 3);
        const int k = qj + W - 1 - rr;
        const bool ok = rr < 2 * W - 1 && k >= c0 && k < c1;
        rw_s[(ok ? k - c0 : kRwRows - 1) * 32 + n] = acc[e] * kLog2e;
      }
    }
    wave_sync();
    const float f = POS ? 1.f / sc : 1.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int c = G::col(mb, e, hh);  // < 64
        cinit[mb][e] = c0 + c < W ? rw_s[c * 32 + n] * f : -INFINITY;
      }
    wave_sync();
  };
  // Rh of grid rows r0 .. r0 + 31 for this lane's query (row kh takes table row qi + H-1 - kh), into rh_s
  auto rh_chunk = [&](int r0) __attribute__((always_inline)) {
    const int nbh = (2 * H - 1 + 31) / 32, r1 = min(H, r0 + 32);
    wave_sync();  // every lane has read the previous chunk
    for (int b = 0; b < nbh; ++b) {
      const f32x16 acc = table_block(32 * b);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = 32 * b + 8 * (e >> 2) + 4 * hh + (e & 3);
        const int k = qi + H - 1 - rr;
        const bool ok = rr < 2 * H - 1 && k >= r0 && k < r1;
        rh_s[(ok ? k - r0 : kRhRows - 1) * 32 + n] = acc[e] * kLog2e;
      }
    }
    wave_sync();
  };

  if (active) rw_pass(0);
  store_k(0, 0);
  store_v(0, 0);
  store_k(1, 1);
  // V padding columns: a column of ones (the denominator row of O^T) then zeros
  for (int i = tid; i < 2 * 64; i += kThreads) {
    T* rowp = vs_base + (i >> 6) * VBUF + (i & 63) * VSTR;
    for (int c = HDP; c < VSTR; ++c) rowp[c] = from_f32<T>((kOnes && c == HDP) ? 1.f : 0.f);
  }
  __syncthreads();

  int koff[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
    koff[mb] = (8 * (g >> 1) + (gi >> 2)) * kKStride + G::slot(mb, 16 * (g & 1) + 4 * (gi & 3));
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

  // Softmax and P.V of tile gt (scores in s_cur) with the S^T of tile gt+1 into s_nxt; the loads,
  // stores and the next S^T run on clamped tile indices near the end and their results go unused.
  auto step = [&](int gt, f32x16* s_cur, f32x16* s_nxt) __attribute__((always_inline)) {
    load_k(0, gt + 2 < ntiles ? gt + 2 : ntiles - 1);
    load_v(0, gt + 1 < ntiles ? gt + 1 : ntiles - 1);
    if (active) {
      const int row = gt % H;
      if ((row & 31) == 0) rh_chunk(row);
      const float rh = rh_s[(row & 31) * 32 + n];
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
        mt = max_nc(mt, POS ? fmaf(mm, sc, rh) : mm + rh);
      }
      mt = max_with_partner32(mt);
      if (wave_any(mt > m_run + kSlack)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = exp2_fast(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int ob = 0; ob < MBO; ++ob) o[ob] *= alpha;
        m_run = m_new;
      }
      // a new column pass starts with tile gt+1: its Rw start values first (the scores of tile gt have
      // taken theirs already), then its S^T with them
      if (gt + 1 < ntiles && (gt + 1) % H == 0) rw_pass((gt + 1) / H);
      qk(ks_base + ((gt + 1) & 1) * KBUF, s_nxt);
      const float c = rh - m_run;
      X8 b[4], blo[4];
      float lsum = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = s_cur[u >> 1][8 * (u & 1) + j];
          pv[j] = exp2_fast(POS ? fmaf(x, sc, c) : x + c);
          if (!kOnes && kSplitP) lsum += pv[j];  // bf16: P.V takes hi + lo, P itself to ~16 bits
        }
        b[u] = pack8(pv, (X8*)nullptr);
        if constexpr (!kOnes && !kSplitP) {
          // f16: the sum over P as the P.V product sees it (rounded), so that numerator and
          // denominator weigh each key alike (the ones row does the same when hd leaves one spare):
          // v_dot2 of the packed P with ones, accumulated in f32
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
      const T* vbuf = vs_base + (gt & 1) * VBUF;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int ob = 0; ob < MBO; ++ob) {
          const X8 a = join8<T>(lds_read_tr16(vbuf + voff[u][0] + 32 * ob), lds_read_tr16(vbuf + voff[u][1] + 32 * ob));
          o[ob] = mma32(a, b[u], o[ob]);
          if (kSplitP) o[ob] = mma32(a, blo[u], o[ob]);
        }
      }
    }
    store_k(0, gt & 1);        // K(gt+2) replaces K(gt), whose scores were taken one step ago
    store_v(0, (gt + 1) & 1);  // V(gt+1) replaces V(gt-1)
    __syncthreads();
  };

  f32x16 sa[2], sb[2];
  if (active) qk(ks_base, sa);
  __syncthreads();  // every wave has read K(0) before step 0 overwrites its buffer with K(2)
  for (int gt = 0; gt < ntiles; gt += 2) {
    step(gt, sa, sb);
    if (gt + 1 < ntiles) step(gt + 1, sb, sa);
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

template <typename T, int HDP, int VK, bool POS>
static hipError_t launch_wide(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                              int hd, int h, int w, float scale, hipStream_t stream) {
  // 8 waves (two per SIMD) where their scratch fits beside the tiles, else 4
  constexpr int NW = wide::lds_bytes<T, HDP, 8>() <= 160 * 1024 ? 8 : 4;
  auto kern = attn_relpos_wide_kernel<T, HDP, VK, POS, NW>;
  constexpr size_t lds = wide::lds_bytes<T, HDP, NW>();
  static_assert(lds <= 160 * 1024, "LDS");
  static std::atomic<unsigned long long> lds_done{0};
  if (const hipError_t e = lds_opt_in(lds_done, (const void*)kern, (int)lds); e != hipSuccess) return e;
  const int n = h * w;
  const int qblocks = (n + NW * 32 - 1) / (NW * 32);
  const long blocks = (long)bh * qblocks;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(NW * 64), lds, stream, (const T*)q, (const T*)kt,
                     (const T*)v, (const T*)table, (T*)out, hd, h, w, scale, qblocks);
  return hipGetLastError();
}

template <typename T, int HDP>
static hipError_t wide_vk(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                          int h, int w, float scale, hipStream_t stream) {
  const int n = h * w;
  if (!(scale > 0.f)) return launch_wide<T, HDP, 1, false>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (w % 8 == 0 && n % 8 == 0) return launch_wide<T, HDP, 8, true>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (w % 2 == 0 && n % 2 == 0) return launch_wide<T, HDP, 2, true>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return launch_wide<T, HDP, 1, true>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

template <typename T>
static hipError_t wide_hd(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                          int h, int w, float scale, hipStream_t stream) {
  if (hd <= 16) return wide_vk<T, 16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 32) return wide_vk<T, 32>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 64) return wide_vk<T, 64>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 80) return wide_vk<T, 80>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return wide_vk<T, 128>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

// Checked by the caller: 1 <= h, w <= 128, hd % 8 == 0, hd <= 128, 16-byte aligned pointers.
hipError_t attn_relpos_wide(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out,
                            int bh, int hd, int h, int w, float scale, hipStream_t stream) {
  if (dtype == kF16) return wide_hd<f16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return wide_hd<bf16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

}  // namespace samhip
