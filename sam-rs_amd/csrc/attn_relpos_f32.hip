// Fused SAM ViT attention with the decomposed relative-position bias, f32, for gfx950.
//
// Same decomposition as the f16/bf16 kernel (attn_relpos.hip): S^T = K . Q^T and O^T = V^T . P^T on
// 32x32 MFMA tiles (v_mfma_f32_32x32x2_f32 here), one query per lane, key tiles that cover whole grid
// rows so the Rw bias stays in registers. The f32 path is held to 1e-5 of the reference's exact-f32
// CPU result (kernels.rs:181-220), so the softmax follows the reference's arithmetic: the logit is
// ((s * scale) + rh) + rw rounded after every step, exponentials use the accurate expf in natural
// units, and products are accumulated in f32.
//
// Operand layouts for K = 2 steps: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32]. The head
// dimension is split in halves, hd index = (l / 32) * HDP/2 + step, so each lane's operands are
// contiguous runs (vector LDS and global reads). The K tile is stored [slot][hd] (transposed from the
// reference's kT while staging) and the V tile [slot][hd].
#include "lds_dma.hpp"
#include "relpos_geom.hpp"

namespace samhip {

constexpr float kRescaleSlackNat = 5.5451774f;  // 8 * ln 2: p <= 256

template <int HDP> struct F32Geom {
  static constexpr int HALF = HDP / 2;
  static constexpr int MBO = (HDP + 31) / 32;
  static constexpr int KSTR = HDP + 4;        // floats per K slot row
  static constexpr int VSTR = MBO * 32 + 4;   // floats per V slot row
};

// Window grids (pair mode, 4 waves, hd <= 80) are held to 256 registers per lane, so that two
// workgroups share a CU; the other shapes run one workgroup per CU.
template <int HDP, int MODE, int NW>
constexpr int f32_min_blocks() { return (NW == 4 && MODE == kPair && HDP <= 80) ? 2 : 1; }

template <int HDP, int MODE, int NW>
__global__ __launch_bounds__(NW * 64, (f32_min_blocks<HDP, MODE, NW>())) void attn_relpos_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ kt, const float* __restrict__ v,
    const float* __restrict__ table, float* __restrict__ out, int hd, int H, int W, float scale) {
  typedef KeyGeom<MODE> G;
  typedef F32Geom<HDP> FG;
  constexpr int HALF = FG::HALF, MBO = FG::MBO, KSTR = FG::KSTR, VSTR = FG::VSTR;
  constexpr int NT = NW * 64;
  constexpr int KBUF = 64 * KSTR, VBUF = 64 * VSTR;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* ks_base = reinterpret_cast<float*>(smem);
  float* vs_base = ks_base + 2 * KBUF;
  float* rhs_base = vs_base + 2 * VBUF;

  const int N = H * W;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const long bh = blockIdx.y;
  const int qidx = (blockIdx.x * NW + wave) * 32 + n;
  const bool qvalid = qidx < N;
  const int qi = qvalid ? qidx / W : 0, qj = qvalid ? qidx % W : 0;
  // this wave's bias scratch: one row of 32 per key row / column index, max(H, W) of them
  float* rhs = rhs_base + wave * (H > W ? H : W) * 32;

  // Q fragments: lane supplies Q[query n][hh * HALF + s]
  float qf[HALF];
#pragma unroll
  for (int s = 0; s < HALF; s += 4) {
    const int c = hh * HALF + s;
    f32x4 val = f32x4{};
    if (qvalid && c < hd) val = *reinterpret_cast<const f32x4*>(q + (bh * N + qidx) * hd + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[s + i] = val[i];
  }

  // prologue: G = T . Q^T, scattered along the diagonal band (natural units here)
  const float* th = table;
  const float* tw = table + (long)(2 * H - 1) * hd;
  auto band = [&](const float* tab, int rows, int base, int len) {
    for (int r0 = 0; r0 < rows; r0 += 32) {
      f32x16 acc = {};
      const int r = r0 + n;
#pragma unroll
      for (int s = 0; s < HALF; s += 4) {
        const int c = hh * HALF + s;
        f32x4 a = f32x4{};
        if (r < rows && c < hd) a = *reinterpret_cast<const f32x4*>(tab + (long)r * hd + c);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], qf[s + i], acc, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = r0 + 8 * (e >> 2) + 4 * hh + (e & 3);
        const int k = base + len - 1 - rr;
        if (rr < rows && k >= 0 && k < len) rhs[k * 32 + n] = acc[e];
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
  for (int i = tid; i < 2 * 64; i += NT) {
    float* rowp = vs_base + (i >> 6) * VBUF + (i & 63) * VSTR;
    for (int c = HDP; c < VSTR; ++c) rowp[c] = 0.f;
  }

  // key tiles: K chunk = 4 consecutive keys of one hd row (from kT), V chunk = 4 hd values of one key
  constexpr int KCH = HDP * 16;
  constexpr int KPT = (KCH + NT - 1) / NT;
  constexpr int VCPR = HDP / 4;
  constexpr int VCH = 64 * VCPR;
  constexpr int VPT = (VCH + NT - 1) / NT;
  float kreg[KPT][4];
  f32x4 vreg[VPT];
  const float* ktb = kt + bh * hd * (long)N;
  const float* vb = v + bh * (long)N * hd;
  auto load_tile = [&](int t) {
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * NT;
      const int d = c >> 4, s0 = (c & 15) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sl = s0 + i;
        const int rho = sl / G::WP, kap = sl % G::WP, row = t * G::RPT + rho;
        kreg[u][i] = (c < KCH && d < hd && kap < W && row < H) ? ktb[(long)d * N + row * W + kap] : 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * NT;
      const int sl = c / VCPR, d0 = (c % VCPR) * 4;
      const int rho = sl / G::WP, kap = sl % G::WP, row = t * G::RPT + rho;
      f32x4 val = f32x4{};
      if (c < VCH && d0 < hd && kap < W && row < H) val = *reinterpret_cast<const f32x4*>(vb + (long)(row * W + kap) * hd + d0);
      vreg[u] = val;
    }
  };
  auto store_tile = [&](int buf) {
    float* kbuf = ks_base + buf * KBUF;
    float* vbuf = vs_base + buf * VBUF;
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int c = tid + u * NT;
      if (c < KCH) {
        const int d = c >> 4, s0 = (c & 15) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) kbuf[(s0 + i) * KSTR + d] = kreg[u][i];
      }
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int c = tid + u * NT;
      if (c < VCH) {
        const int sl = c / VCPR, d0 = (c % VCPR) * 4;
        *reinterpret_cast<f32x4*>(vbuf + sl * VSTR + d0) = vreg[u];
      }
    }
  };

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
    const float* kbuf = ks_base + buf * KBUF;
    const float* vbuf = vs_base + buf * VBUF;

    f32x16 s[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      s[mb] = f32x16{};
      const float* krow = kbuf + G::slot(mb, n) * KSTR + hh * HALF;
#pragma unroll
      for (int st = 0; st < HALF; st += 4) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(krow + st);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], qf[st + i], s[mb], 0, 0, 0);
      }
    }

    float rh[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int row = t * G::RPT + G::row(mb, hh);
      rh[mb] = row < H ? rhs[row * 32 + n] : -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = s[mb][e] * scale;  // kernels.rs:202: x * scale + rh[kh] + rw[kw], left to right
        x = x + rh[mb];
        x = x + rw[G::rw_index(mb, e)];
        s[mb][e] = x;
        mt = fmaxf(mt, x);
      }
    mt = max_with_partner32(mt);
    if (wave_any(mt > m_run + kRescaleSlackNat)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = expf(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int ob = 0; ob < MBO; ++ob) o[ob] *= alpha;
      m_run = m_new;
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = expf(s[mb][e] - m_run);
        s[mb][e] = p;
        l_run += p;
      }

    // O^T += V^T . P^T, two logical keys per step: lane half hh supplies S-row 8*(e/4) + 4*hh + e%4
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int sl = G::slot(mb, 8 * (e >> 2) + 4 * hh + (e & 3));
#pragma unroll
        for (int ob = 0; ob < MBO; ++ob)
          o[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(vbuf[sl * VSTR + 32 * ob + n], s[mb][e], o[ob], 0, 0, 0);
      }

    if (t + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  const float inv = 1.f / sum_with_partner32(l_run);
  if (qvalid) {
    float* orow = out + (bh * N + qidx) * hd;
#pragma unroll
    for (int ob = 0; ob < MBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * ob + 8 * a + 4 * hh;
        if (d0 < hd) {
          f32x4 w4;
#pragma unroll
          for (int b = 0; b < 4; ++b) w4[b] = o[ob][4 * a + b] * inv;
          *reinterpret_cast<f32x4*>(orow + d0) = w4;
        }
      }
  }
}

// ---------------------------------------------------------------------------------------------------
// Windows at hd 64 (W <= 16, H * W <= 256: SAM ViT-B and ViT-L f32): a workgroup of 4 waves takes 128
// queries of a unit (two per 14x14 window), every byte moves by 16-byte LDS DMA through a two-buffer
// ring of 32-key tiles (two grid rows of 16 slots), and the workgroup needs 42 KB of LDS and at most
// 168 registers, so three share a CU: the 600 workgroups of a ViT-B layer run in one round.
//   * K tile: [d][32 slots] from kT rows, a 128-byte gap row between d < 32 and d >= 32, so that the two
//     lane halves of an S^T step (dims s and 32 + s) read opposite halves of the banks;
//   * V tile: [32 slots][64] with the 16-byte chunks of slots 16..31 rotated by 8, so that the two lane
//     halves of a P.V step (slots e and 16 + e) read opposite halves of the banks;
//   * S^T row m of a tile is slot 16 ((m >> 2) & 1) + 4 (m >> 3) + (m & 3): accumulator element e of lane
//     (hh, n) is grid row hh of the tile, column e, so the Rw bias of element e is the same in every tile
//     and the Rh bias is one value per lane and tile;
//   * the logit is ((s * scale) + rh) + rw and P = expf(x - m), as in the kernel above.
namespace f32w {
constexpr int kWaves = 4, kThreads = 256, kHD = 64, kHalf = 32, kSlots = 32;
constexpr int kKTile = (kHD + 1) * kSlots;   // floats: 64 rows and the gap row
constexpr int kVTile = kSlots * kHD;
constexpr int kBuf = kKTile + kVTile;
constexpr int kRhs = 16 * 32;                // per-wave bias scratch: 16 rows (columns or grid rows) of 32
constexpr size_t kLdsBytes = (size_t)(2 * kBuf + kWaves * kRhs) * sizeof(float);
static_assert(3 * kLdsBytes <= 160 * 1024, "three workgroups per CU");
__device__ __forceinline__ int slot_of_row(int m) { return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3); }
}  // namespace f32w

__global__ __launch_bounds__(f32w::kThreads, 3) void attn_relpos_f32_win_kernel(
    const float* __restrict__ q, const float* __restrict__ kt, const float* __restrict__ v,
    const float* __restrict__ table, float* __restrict__ out, int H, int W, float scale, int nunits, int halves) {
  using namespace f32w;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* ring = reinterpret_cast<float*>(smem);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* rhs = ring + 2 * kBuf + wave * kRhs;
  const unsigned lds0 = lds_addr(smem);
  const int lane = threadIdx.x & 63, n = lane & 31, hh = lane >> 5;
  const int N = H * W;
  // all first parts of the units go first, then the second parts (lighter at 14x14: 68 queries)
  const long u = blockIdx.x % nunits;
  const int part = blockIdx.x / nunits;
  const int q0 = part * 128 + wave * 32;
  const int qidx = q0 + n;
  const bool qvalid = qidx < N;
  const int qi = qvalid ? qidx / W : 0, qj = qvalid ? qidx - (qidx / W) * W : 0;
  const long unit = (long)N * kHD;

  // q fragments: lane supplies Q[query n][32 hh + s]
  float qf[kHalf];
#pragma unroll
  for (int s = 0; s < kHalf; s += 4) {
    f32x4 val = f32x4{};
    if (qvalid) val = *reinterpret_cast<const f32x4*>(q + u * unit + (long)qidx * kHD + kHalf * hh + s);
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[s + i] = val[i];
  }

  // DMA offsets: wave w moves K units w and w + 4 (8 rows of 128 bytes each) and V units w and w + 4
  // (4 slots of 256 bytes each); the tile's first key is the wave-uniform soffset
  const i32x4 krsrc = buffer_rsrc(kt + u * unit, (unsigned)(sizeof(float) * unit));
  const i32x4 vrsrc = buffer_rsrc(v + u * unit, (unsigned)(sizeof(float) * unit));
  unsigned kdof[2], vdof[2], klds[2], vlds[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int ku = wave + 4 * p;
    const int d = 8 * ku + (lane >> 3), piece = lane & 7;
    kdof[p] = (unsigned)(sizeof(float) * ((long)d * N + (piece >> 2) * W + 4 * (piece & 3)));
    klds[p] = (unsigned)(sizeof(float) * (ku < 4 ? ku * 256 : (ku * 256 + kSlots)));  // rows >= 32 after the gap
    const int slot = 4 * ku + (lane >> 4), pos = lane & 15;
    const int lc = (pos - 8 * (slot >> 4)) & 15;  // the logical chunk stored at position pos
    vdof[p] = (unsigned)(sizeof(float) * (((slot >> 4) * W + (slot & 15)) * kHD + 4 * lc));
    vlds[p] = (unsigned)(sizeof(float) * (kKTile + ku * 256));
  }
  auto tile_dma = [&](int t, int buf) {
    const unsigned kso = (unsigned)(sizeof(float) * 2 * t * W), vso = kso * kHD;
    const unsigned b = lds0 + (unsigned)(sizeof(float) * buf * kBuf);
#pragma unroll
    for (int p = 0; p < 2; ++p) bdma16s(krsrc, kdof[p], kso, b + klds[p]);
#pragma unroll
    for (int p = 0; p < 2; ++p) bdma16s(vrsrc, vdof[p], vso, b + vlds[p]);
  };

  // bias prologue: G = T . Q^T on the MFMA (table rows straight from memory), scattered along the
  // diagonal band into this wave's scratch: Rw by key column, then Rh by key grid row
  auto band = [&](const float* tab, int rows, int base, int len) {
    for (int r0 = 0; r0 < rows; r0 += 32) {
      f32x16 acc = {};
      const int r = r0 + n;
#pragma unroll
      for (int s = 0; s < kHalf; s += 4) {
        f32x4 a = f32x4{};
        if (r < rows) a = *reinterpret_cast<const f32x4*>(tab + (long)r * kHD + kHalf * hh + s);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], qf[s + i], acc, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = r0 + 8 * (e >> 2) + 4 * hh + (e & 3);
        const int k = base + len - 1 - rr;
        if (rr < rows && k >= 0 && k < len) rhs[k * 32 + n] = acc[e];
      }
    }
  };
  const float* th = table;
  const float* tw = table + (long)(2 * H - 1) * kHD;
  const int ntiles = (H + 1) / 2;
  tile_dma(0, 0);
  band(tw, 2 * W - 1, qj, W);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float rw[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) rw[e] = e < W ? rhs[e * 32 + n] : -INFINITY;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  band(th, 2 * H - 1, qi, H);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  const unsigned kread = (unsigned)(sizeof(float) * (hh * (kHalf + 1) * kSlots + slot_of_row(n)));
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[2] = {f32x16{}, f32x16{}};
  const bool active = q0 < N;  // a wave with no valid query moves its tile shares and skips the rest
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    wait_vm<0>();     // this wave's DMAs of tile t have landed
    __syncthreads();  // everyone's tile t is visible; everyone is done with tile t - 1
    if (t + 1 < ntiles) tile_dma(t + 1, buf ^ 1);
    if (!active) continue;
    const float* kb = reinterpret_cast<const float*>(smem + sizeof(float) * buf * kBuf + kread);
    const float* vb = ring + buf * kBuf + kKTile;
    f32x16 s = f32x16{};
#pragma unroll
    for (int st = 0; st < kHalf; ++st) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kb[st * kSlots], qf[st], s, 0, 0, 0);
    const int row = 2 * t + hh;
    const float rh = row < H ? rhs[row * 32 + n] : -INFINITY;
    float mt = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float x = s[e] * scale;  // kernels.rs:202: x * scale + rh[kh] + rw[kw], left to right
      x = x + rh;
      x = x + rw[e];
      s[e] = x;
      mt = fmaxf(mt, x);
    }
    mt = max_with_partner32(mt);
    if (wave_any(mt > m_run + kRescaleSlackNat)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = expf(m_run - m_new);
      l_run *= alpha;
      o[0] *= alpha;
      o[1] *= alpha;
      m_run = m_new;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pe = expf(s[e] - m_run);
      s[e] = pe;
      l_run += pe;
    }
    // O^T += V^T . P^T: step e pairs slot e (lanes hh = 0) with slot 16 + e (hh = 1)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float* vrow = vb + (16 * hh + e) * kHD;
#pragma unroll
      for (int ob = 0; ob < 2; ++ob) {
        const int d = 32 * ob + n;
        o[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[4 * (((d >> 2) + 8 * hh) & 15) + (d & 3)], s[e], o[ob], 0, 0, 0);
      }
    }
  }

  const float inv = 1.f / sum_with_partner32(l_run);
  if (qvalid) {
    float* orow = out + u * unit + (long)qidx * kHD;
#pragma unroll
    for (int ob = 0; ob < 2; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4 w4;
#pragma unroll
        for (int b = 0; b < 4; ++b) w4[b] = o[ob][4 * a + b] * inv;
        *reinterpret_cast<f32x4*>(orow + 32 * ob + 8 * a + 4 * hh) = w4;
      }
  }
}

static hipError_t launch_f32_win(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                                 int h, int w, float scale, hipStream_t stream) {
  static std::atomic<unsigned long long> lds_done{0};
  if (const hipError_t e = lds_opt_in(lds_done, (const void*)attn_relpos_f32_win_kernel, (int)f32w::kLdsBytes);
      e != hipSuccess)
    return e;
  const int parts = (h * w + 127) / 128;
  hipLaunchKernelGGL(attn_relpos_f32_win_kernel, dim3((unsigned)(bh * parts)), dim3(f32w::kThreads), f32w::kLdsBytes,
                     stream, (const float*)q, (const float*)kt, (const float*)v, (const float*)table, (float*)out, h, w,
                     scale, bh, parts);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------
// Global grids at hd 64 (W = 64: SAM ViT-B and ViT-L f32): 16 queries per wave on
// v_mfma_f32_16x16x4_f32, a workgroup of 4 waves takes one grid row of 64 queries, so a ViT-B layer is
// 12 x 64 = 768 workgroups: three per CU, three waves on every SIMD, one round. (With 32 queries per
// wave the 12 heads x 4096 queries come in multiples of 64 queries per SIMD pair, and a quarter of the
// CUs stayed idle.) K and V move by 16-byte LDS DMA through a two-buffer ring of 32-key tiles (half a
// grid row); 48 KB of LDS.
//   * lane (g, i) = (lane / 16, lane % 16) holds query i of its wave; S^T block kb (16 keys) element r is
//     key 16 kb + 4 g + r; Q^T element s of the lane is dim 4 s + g;
//   * K tile [d][32 keys] with the 4-key chunks of rows 2, 3 (mod 4) moved by 4 chunks, V tile
//     [32 keys][64] with the 4-dim chunks of key k moved by 4 ((k >> 2) & 3) chunks: the four lane
//     groups of a read fall on disjoint banks;
//   * the Rw bias of element (kb, r) depends on the tile's half of the grid row only (16 values per
//     lane), the Rh bias is one value per lane and grid row, kept in the wave's scratch;
//   * the logit is ((s * scale) + rh) + rw and P = expf(x - m), as in the kernels above.
namespace f32g {
constexpr int kWaves = 4, kThreads = 256, kHD = 64, kSlots = 32;
constexpr int kKTile = kHD * kSlots, kVTile = kSlots * kHD, kBuf = kKTile + kVTile;
constexpr int kRhs = 64 * 16;  // per wave: [64 rows][16 queries]
constexpr size_t kLdsBytes = (size_t)(2 * kBuf + kWaves * kRhs) * sizeof(float);
static_assert(3 * kLdsBytes <= 160 * 1024, "three workgroups per CU");
}  // namespace f32g

__global__ __launch_bounds__(f32g::kThreads, 3) void attn_relpos_f32_glob16_kernel(
    const float* __restrict__ q, const float* __restrict__ kt, const float* __restrict__ v,
    const float* __restrict__ table, float* __restrict__ out, int H, float scale) {
  using namespace f32g;
  constexpr int W = 64;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* ring = reinterpret_cast<float*>(smem);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* rhs = ring + 2 * kBuf + wave * kRhs;
  const unsigned lds0 = lds_addr(smem);
  const int lane = threadIdx.x & 63, g = lane >> 4, li = lane & 15;
  const int N = H * W;
  // workgroups in contiguous ranges per XCD, so that the query rows of a head share an L2
  const int total = (int)gridDim.x, per = total >> 3, rem = total & 7, xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int blk = xcd * per + (xcd < rem ? xcd : rem) + j;
  const long bh = blk / H;
  const int qi = blk % H, qj = 16 * wave + li;
  const long unit = (long)N * kHD;
  const float* qrow = q + bh * unit + (long)(qi * W + qj) * kHD;

  float qf[16];  // Q^T[4 s + g][query]
#pragma unroll
  for (int s = 0; s < 16; ++s) qf[s] = qrow[4 * s + g];

  // DMA: wave w moves K units w, w + 4 (rows 8u .. 8u+7, 128 bytes each) and V units w, w + 4 (keys
  // 4u .. 4u+3, 256 bytes each) of a tile; the tile's first key is the wave-uniform soffset
  const i32x4 krsrc = buffer_rsrc(kt + bh * unit, (unsigned)(sizeof(float) * unit));
  const i32x4 vrsrc = buffer_rsrc(v + bh * unit, (unsigned)(sizeof(float) * unit));
  unsigned kdof[2], vdof[2], klds[2], vlds[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int u = wave + 4 * p;
    const int d = 8 * u + (lane >> 3), pos = lane & 7;
    const int lc = pos ^ (4 * ((d >> 1) & 1));  // the 4-key chunk stored at position pos
    kdof[p] = (unsigned)(sizeof(float) * ((long)d * N + 4 * lc));
    klds[p] = (unsigned)(sizeof(float) * u * 256);
    const int key = 4 * u + (lane >> 4), vpos = lane & 15;
    const int vlc = vpos ^ (4 * ((key >> 2) & 3));
    vdof[p] = (unsigned)(sizeof(float) * (key * kHD + 4 * vlc));
    vlds[p] = (unsigned)(sizeof(float) * (kKTile + u * 256));
  }
  auto tile_dma = [&](int t, int buf) {
    const unsigned kso = (unsigned)(sizeof(float) * kSlots * t), vso = kso * kHD;
    const unsigned b = lds0 + (unsigned)(sizeof(float) * buf * kBuf);
#pragma unroll
    for (int p = 0; p < 2; ++p) bdma16s(krsrc, kdof[p], kso, b + klds[p]);
#pragma unroll
    for (int p = 0; p < 2; ++p) bdma16s(vrsrc, vdof[p], vso, b + vlds[p]);
  };
  const int ntiles = 2 * H;
  tile_dma(0, 0);

  // bias prologue: G = T . Q^T on the MFMA, 16 table rows per block (table rows straight from memory),
  // scattered along the diagonal band: Rw into the scratch by key column, read into registers, then Rh
  // by key grid row, which stays in the scratch
  auto wsync = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  auto band = [&](const float* tab, int rows, int base, int len) {
    for (int r0 = 0; r0 < rows; r0 += 16) {
      const int r = min(r0 + li, rows - 1);
      f32x4 acc = f32x4{};
#pragma unroll
      for (int s = 0; s < 16; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(tab[(long)r * kHD + 4 * s + g], qf[s], acc, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rr = r0 + 4 * g + e;
        const int k = base + len - 1 - rr;
        if (rr < rows && k >= 0 && k < len) rhs[k * 16 + li] = acc[e];
      }
    }
  };
  band(table + (long)(2 * H - 1) * kHD, 2 * W - 1, qj, W);
  wsync();
  float rw[16];  // [tile half][kb][r]: key column 32 h + 16 kb + 4 g + r
#pragma unroll
  for (int e = 0; e < 16; ++e) rw[e] = rhs[(32 * (e >> 3) + 16 * ((e >> 2) & 1) + 4 * g + (e & 3)) * 16 + li];
  wsync();
  band(table, 2 * H - 1, qi, H);
  wsync();

  // per-lane LDS read offsets (floats): K row 4 s + g, key 16 kb + li (swizzled, one offset per kb); V
  // key 16 kb + 4 g + r, dim 16 db + li (swizzled)
  const int kofs0 = g * kSlots + (li ^ (16 * ((g >> 1) & 1)));
  const int kofs1 = g * kSlots + ((16 + li) ^ (16 * ((g >> 1) & 1)));
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[4] = {f32x4{}, f32x4{}, f32x4{}, f32x4{}};
  // tile t is the half t & 1 of grid row t >> 1 and sits in ring buffer t & 1
  auto step = [&](int t, auto half_c) {
    constexpr int buf = decltype(half_c)::value;
    wait_vm<0>();     // this wave's DMAs of tile t have landed
    __syncthreads();  // everyone's tile t is visible; everyone is done with tile t - 1
    if (t + 1 < ntiles) tile_dma(t + 1, buf ^ 1);
    const float* kb0 = ring + buf * kBuf + kofs0;
    const float* kb1 = ring + buf * kBuf + kofs1;
    const float* vb = ring + buf * kBuf + kKTile;
    f32x4 sacc[2] = {f32x4{}, f32x4{}};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      sacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(kb0[s * 4 * kSlots], qf[s], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kb1[s * 4 * kSlots], qf[s], sacc[1], 0, 0, 0);
    }
    const float rh = rhs[(t >> 1) * 16 + li];
    float x[8];
    float mt = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float y = sacc[e >> 2][e & 3] * scale;  // kernels.rs:202: x * scale + rh[kh] + rw[kw], left to right
      y = y + rh;
      y = y + rw[8 * buf + e];
      x[e] = y;
      mt = fmaxf(mt, y);
    }
    mt = max_over_rows16(mt);
    if (wave_any(mt > m_run + kRescaleSlackNat)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = expf(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
      m_run = m_new;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = expf(x[e] - m_run);
      l_run += x[e];
    }
    // O^T += V^T . P^T: step (kb, r) pairs the keys 16 kb + 4 g + r of the four lane groups
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float* vrow = vb + (16 * (e >> 2) + 4 * g + (e & 3)) * kHD;
#pragma unroll
      for (int db = 0; db < 4; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * (db ^ g) + li], x[e], o[db], 0, 0, 0);
    }
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(t, std::integral_constant<int, 0>());
    step(t + 1, std::integral_constant<int, 1>());
  }

  const float inv = 1.f / sum_over_rows16(l_run);
  float* orow = out + bh * unit + (long)(qi * W + qj) * kHD;
#pragma unroll
  for (int db = 0; db < 4; ++db) *reinterpret_cast<f32x4*>(orow + 16 * db + 4 * g) = o[db] * inv;
}

static hipError_t launch_f32_glob16(const void* q, const void* kt, const void* v, const void* table, void* out,
                                    int bh, int h, float scale, hipStream_t stream) {
  static std::atomic<unsigned long long> lds_done{0};
  if (const hipError_t e = lds_opt_in(lds_done, (const void*)attn_relpos_f32_glob16_kernel, (int)f32g::kLdsBytes);
      e != hipSuccess)
    return e;
  hipLaunchKernelGGL(attn_relpos_f32_glob16_kernel, dim3((unsigned)(bh * h)), dim3(f32g::kThreads), f32g::kLdsBytes,
                     stream, (const float*)q, (const float*)kt, (const float*)v, (const float*)table, (float*)out, h,
                     scale);
  return hipGetLastError();
}

template <int HDP, int MODE, int NW>
static hipError_t launch_f32(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                             int hd, int h, int w, float scale, hipStream_t stream) {
  typedef F32Geom<HDP> FG;
  // K and V double buffers, then max(h, w) scratch rows per wave: a 14x14 window needs 14 (two
  // workgroups fit on a CU), a 64-column grid 64
  const size_t tiles = (size_t)(2 * 64 * FG::KSTR + 2 * 64 * FG::VSTR) * sizeof(float);
  const size_t lds = tiles + (size_t)NW * (h > w ? h : w) * 32 * sizeof(float);
  auto kern = attn_relpos_f32_kernel<HDP, MODE, NW>;
  static std::atomic<unsigned long long> lds_done{0};  // opt-in to the largest size this instantiation asks for
  {
    const int most = (int)(tiles + (size_t)NW * 64 * 32 * sizeof(float));
    const hipError_t e = lds_opt_in(lds_done, (const void*)kern, most);
    if (e != hipSuccess) return e;
  }
  const int n = h * w;
  dim3 grid((n + 32 * NW - 1) / (32 * NW), bh);
  hipLaunchKernelGGL(kern, grid, dim3(NW * 64), lds, stream, (const float*)q, (const float*)kt, (const float*)v,
                     (const float*)table, (float*)out, hd, h, w, scale);
  return hipGetLastError();
}

template <int HDP, int MODE>
static hipError_t f32_pick_nw(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                              int hd, int h, int w, float scale, hipStream_t stream) {
  // LDS: two K and two V tiles of 64 x HDP floats plus up to 8 KB of bias scratch per wave must fit in
  // 160 KB
  if (HDP > 80) return launch_f32<HDP, MODE, 2>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (h * w > 1024) return launch_f32<HDP, MODE, 8>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return launch_f32<HDP, MODE, 4>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

template <int HDP>
static hipError_t f32_pick_mode(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                                int hd, int h, int w, float scale, hipStream_t stream) {
  if (w <= 16) return f32_pick_nw<HDP, kPair>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (w <= 32) return f32_pick_nw<HDP, kRow32>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return f32_pick_nw<HDP, kRow64>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

// Shape limits are checked by the caller: 1 <= h, w <= 64, hd % 4 == 0, hd <= 128.
hipError_t attn_relpos_f32(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                           int h, int w, float scale, hipStream_t stream) {
  if (hd <= 16) return f32_pick_mode<16>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 32) return f32_pick_mode<32>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd == 64 && w <= 16 && h <= 16 && h * w <= 256)
    return launch_f32_win(q, kt, v, table, out, bh, h, w, scale, stream);
  if (hd == 64 && w == 64) {
    // 64 queries per workgroup, three per CU, against 256 queries per workgroup, one per CU: the
    // former per round takes about 0.8 of the latter's round time (ViT-B, where each is one round),
    // so it is taken unless it needs more rounds than that makes up for (ViT-L: 1024 workgroups are
    // 1.33 rounds against one round of 256)
    const long cus = device_cu_count(), g16 = (long)bh * h, g8 = (long)bh * ((h * 64 + 255) / 256);
    const long rounds16 = (g16 + 3 * cus - 1) / (3 * cus), rounds8 = (g8 + cus - 1) / cus;
    if (4 * rounds16 <= 5 * rounds8) return launch_f32_glob16(q, kt, v, table, out, bh, h, scale, stream);
  }
  if (hd <= 64) return f32_pick_mode<64>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  if (hd <= 80) return f32_pick_mode<80>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
  return f32_pick_mode<128>(q, kt, v, table, out, bh, hd, h, w, scale, stream);
}

}  // namespace samhip
