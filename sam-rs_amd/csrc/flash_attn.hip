// Flash attention for gfx950, f16 / bf16: out = softmax(scale * q k^T [+ mask]) v per (batch, head).
//
// The GPU counterpart of the reference's three attention back ends on [B, L, H, D] tensors:
// candle_flash_attn::flash_attn(q, k, v, scale, false) (sam2/hiera.rs:143-151, sam3/nn.rs:65-71,
// sam3/vision.rs:116-121), kernels::flash_attn_cpu (kernels.rs:910-915 -> cpu_gemm.rs:361-417) and
// sam3::nn::sdpa (sam3/nn.rs:26-34), without a mask (SAM 2 memory attention calls it that way through
// RopeAttn::forward, sam3/video.rs:129-145) or with an additive one (SAM 3's DETR text mask, TinyViT's
// attention biases), which the MASK instances add to the scaled scores. Any (batch, row, head) strides are accepted, so both the
// [B, L, H, D] and the [B, H, L, D] layouts are read in place; the head dimension is contiguous.
//
// Work decomposition: one workgroup = NW waves = NW * 32 queries of one (batch, head) and one range of
// keys ("split"). Each wave owns 32 queries and computes S^T = K . Q^T on v_mfma_f32_32x32x16 with Q in
// registers (B operand) and K read from LDS as the A operand, so a lane holds one query and 16 keys per
// 32-key block, and the row softmax needs one cross-lane exchange (v_permlane32_swap). O^T = V^T . P^T
// takes the S^T accumulators as its B operand directly under a fixed key permutation that the V^T
// transpose reads (ds_read_b64_tr_b16) follow, so P never moves between lanes. K and V tiles of 64 keys
// are double-buffered in LDS with K one tile ahead of V: the global loads of K(t+2) and V(t+1) are in
// flight while tile t's softmax and P.V run, and the S^T of tile t+1 is issued on the MFMA while tile
// t's exponentials run on the VALU. Online softmax in the exp2 domain; the running max only moves when
// a tile exceeds it by more than 8 (log2 units), so the O rescale is skipped on almost every tile.
//
// Few query blocks (SAM 2 memory attention: one head, 4096 queries, 4096 or 28736 keys) would leave
// most of the 256 CUs idle, so the keys are split across workgroups; each split writes a partial O
// (unnormalised, in f32) with its
// running max and sum, and flash_combine_kernel merges the splits by log-sum-exp. Workgroups are
// numbered XCD-major with all query blocks of one (head, split) adjacent, so the K/V range of a split
// is fetched into one XCD's L2 and shared there.
//
// Optional RoPE on the queries (the first n_rope_q rows, table row = query % rope_rows) is applied while
// Q is loaded, in f32 with the reference's rounding (x*cos + rot(x)*sin, rot([x0,x1]) = [-x1,x0],
// sam3/video.rs:106-113) and then rounded to the element type as the reference's rope does. Keys are
// rotated beforehand by rope_shared_kernel (rope.hip).
#include "flash_attn.hpp"

namespace samhip {

constexpr float kFlashSlack = 8.0f;
constexpr float kFlashLog2e = 1.4426950408889634f;

template <typename T, int DP, int NW>
struct FlashGeom {
  static constexpr int KS = DP / 16;        // k-steps of S^T = K Q^T
  static constexpr int MBO = DP / 32;       // 32-row blocks of O^T
  static constexpr int KSTR = DP + 8;       // K tile row stride (elements): rows 16 bytes apart mod 128
  static constexpr int VSTR = DP + 16;      // V tile row stride: transpose reads shift 8 banks per row
  static constexpr int KBUF = 64 * KSTR;
  static constexpr int VBUF = 64 * VSTR;
  static constexpr int NT = NW * 64;
  static constexpr size_t LDS = (size_t)(2 * KBUF + 2 * VBUF) * sizeof(T);
  static constexpr int CPR = DP / 8;        // 16-byte chunks per key row
  static constexpr int CH = 64 * CPR;       // chunks per tile
  static constexpr int PT = (CH + NT - 1) / NT;
};

// Workgroup i runs on XCD i % 8; give each XCD a contiguous range of the linear work index.
__device__ __forceinline__ int flash_xcd_block(int i, int total) {
  const int per = total >> 3, rem = total & 7, x = i & 7, j = i >> 3;
  return x * per + (x < rem ? x : rem) + j;
}

// Reference rounding of one rotated pair: (x0*c0 + (-x1)*s0, x1*c1 + x0*s1), no contraction.
__device__ __forceinline__ void rope_pair(float x0, float x1, float c0, float s0, float c1, float s1, float& y0,
                                          float& y1) {
#pragma clang fp contract(off)
  y0 = x0 * c0 + -x1 * s0;
  y1 = x1 * c1 + x0 * s1;
}

// f16 4-wave workgroups (head dims up to 64) are held to 168 registers, so that three share a CU (bf16,
// whose P.V takes P as hi + lo, would spill there and runs two to a CU).
template <typename T, int DP, int NW, bool ROPEQ, bool MASK>
__global__ __launch_bounds__(NW * 64, NW == 4 && DP <= 64 && __is_same(T, f16) ? 3 : 1) void flash_fwd_kernel(
    FlashParams p) {
  typedef FlashGeom<T, DP, NW> FG;
  typedef typename Vec<T>::x8 X8;
  constexpr bool kSplitP = __is_same(T, bf16);
  constexpr int KS = FG::KS, MBO = FG::MBO, KSTR = FG::KSTR, VSTR = FG::VSTR;
  constexpr int KBUF = FG::KBUF, VBUF = FG::VBUF, NT = FG::NT;
  constexpr int CPR = FG::CPR, CH = FG::CH, PT = FG::PT;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* ks_base = reinterpret_cast<T*>(smem);
  T* vs_base = ks_base + 2 * KBUF;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;

  const int lin = flash_xcd_block(blockIdx.x, gridDim.x);
  const int qb = lin % p.qblocks;
  const int split = (lin / p.qblocks) % p.nsplit;
  const int bhi = lin / (p.qblocks * p.nsplit);
  const int bi = bhi / p.h, head = bhi % p.h;
  const int d = p.d;

  const int q0 = qb * (NW * 32) + wave * 32;
  const bool active = q0 < p.lq;
  const int qidx = q0 + n;
  const bool qvalid = qidx < p.lq;

  const int t_begin = split * p.tps;
  const int ntiles_all = (p.lk + 63) >> 6;
  const int t_end = min(ntiles_all, t_begin + p.tps);
  const int ntiles = t_end - t_begin;
  const int kend = p.lk;  // keys >= kend are masked (only the last tile can hold such keys)

  const T* qbase = reinterpret_cast<const T*>(p.q) + bi * p.sq[0] + head * p.sq[2];
  const T* kbase = reinterpret_cast<const T*>(p.k) + bi * p.sk[0] + head * p.sk[2];
  const T* vbase = reinterpret_cast<const T*>(p.v) + bi * p.sv[0] + head * p.sv[2];

  // ---- K/V tile staging: global -> registers -> LDS, zero outside [0, kend) x [0, d). Loads are
  // unconditional (an out-of-range chunk reads the head's first row) so no branch sits between a
  // load's issue and the work that hides its latency; the zero fill is applied at the LDS store.
  u32x4 kreg[PT], vreg[PT];
  bool kok[PT], vok[PT];
  auto load_k = [&](int t) {
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      const int r = c / CPR, c8 = (c % CPR) * 8;
      const int key = (t << 6) + r;
      const bool ok = (CH % NT == 0 || c < CH) && key < kend && c8 < d;
      kok[u] = ok;
      kreg[u] = *reinterpret_cast<const u32x4*>(kbase + (ok ? (long)key * p.sk[1] + c8 : 0));
    }
  };
  auto load_v = [&](int t) {
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      const int r = c / CPR, c8 = (c % CPR) * 8;
      const int key = (t << 6) + r;
      const bool ok = (CH % NT == 0 || c < CH) && key < kend && c8 < d;
      vok[u] = ok;
      vreg[u] = *reinterpret_cast<const u32x4*>(vbase + (ok ? (long)key * p.sv[1] + c8 : 0));
    }
  };
  auto store_k = [&](int buf) {
    T* kb = ks_base + buf * KBUF;
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      if (CH % NT == 0 || c < CH)
        *reinterpret_cast<u32x4*>(kb + (c / CPR) * KSTR + (c % CPR) * 8) = kok[u] ? kreg[u] : u32x4{};
    }
  };
  auto store_v = [&](int buf) {
    T* vb = vs_base + buf * VBUF;
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      if (CH % NT == 0 || c < CH)
        *reinterpret_cast<u32x4*>(vb + (c / CPR) * VSTR + (c % CPR) * 8) = vok[u] ? vreg[u] : u32x4{};
    }
  };

  // The first K and V tiles, the second K tile (in a register set of its own) and the Q fragments are
  // all in flight together, so that the key loop starts one memory latency after the workgroup does
  // (a short key range, such as Hiera's or SAM 3's windows, is mostly this prologue).
  const int tl = t_end - 1;
  load_k(t_begin);
  load_v(t_begin);
  u32x4 kreg1[PT];
  bool kok1[PT];
  {
    const int t1 = min(t_begin + 1, tl);
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      const int r = c / CPR, c8 = (c % CPR) * 8;
      const int key = (t1 << 6) + r;
      const bool ok = (CH % NT == 0 || c < CH) && key < kend && c8 < d;
      kok1[u] = ok;
      kreg1[u] = *reinterpret_cast<const u32x4*>(kbase + (ok ? (long)key * p.sk[1] + c8 : 0));
    }
  }

  // Q fragments (B operand of S^T = K Q^T): lane supplies Q[query n][16*s + 8*hh + j], j = 0..7
  X8 qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int c = 16 * s + 8 * hh;
    X8 val = X8{};
    if (qvalid && c < d) {
      val = __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(qbase + (long)qidx * p.sq[1] + c));
      if (ROPEQ && qidx < p.nrq) {
        const long tr = (long)(qidx % p.rrows) * d + c;
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(p.rcos + tr);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(p.rcos + tr + 4);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(p.rsin + tr);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(p.rsin + tr + 4);
        const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
        const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; j += 2)
          rope_pair(to_f32(val[j]), to_f32(val[j + 1]), cs[j], sn[j], cs[j + 1], sn[j + 1], y[j], y[j + 1]);
        val = pack8(y, (X8*)nullptr);
      }
    }
    qf[s] = val;
  }
  store_k(0);
  store_v(0);
  {
    T* kb = ks_base + KBUF;
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      if (CH % NT == 0 || c < CH)
        *reinterpret_cast<u32x4*>(kb + (c / CPR) * KSTR + (c % CPR) * 8) = kok1[u] ? kreg1[u] : u32x4{};
    }
  }
  __syncthreads();

  // per-lane constant parts of the LDS addresses
  // K (A operand of S^T): lane reads K row 32*mb + n, columns 16*k + 8*hh .. +7 (one 16-byte read)
  int koff[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) koff[mb] = (32 * mb + n) * KSTR + 8 * hh;
  // V^T (A operand of O^T): source lane (4*s + c) of group g reads key row
  // 32*(u>>1) + 16*(u&1) + 8*r + 4*(g>>1) + s, columns 32*ob + 16*(g&1) + 4*c .. +3
  int voff[4][2];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int key = 32 * (u >> 1) + 16 * (u & 1) + 8 * r + 4 * (g >> 1) + (gi >> 2);
      voff[u][r] = key * VSTR + 16 * (g & 1) + 4 * (gi & 3);
    }

  const float sc = p.sc;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[MBO];
#pragma unroll
  for (int ob = 0; ob < MBO; ++ob) o[ob] = f32x16{};

  auto qk = [&](const T* kb, f32x16* s) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const X8 a = *reinterpret_cast<const X8*>(kb + koff[mb] + 16 * k);
        s[mb] = mma32(a, qf[k], k == 0 ? f32x16{} : s[mb]);
      }
    }
  };

  // Softmax and P.V of tile t (scores in s_cur, buffers t&1) with the S^T of tile t+1 into s_nxt.
  // Past the last tile the loads and the next S^T run on clamped indices and their results go unused.
  auto step = [&](int t, f32x16* s_cur, f32x16* s_nxt) {
    const int i = t - t_begin;
    load_k(min(t + 2, tl));
    X8 b[4], blo[4];
    {
      // keys past the end of the last tile: -inf scores
      if ((t << 6) + 64 > kend) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if ((t << 6) + 32 * mb + 8 * (e >> 2) + 4 * hh + (e & 3) >= kend) s_cur[mb][e] = -INFINITY;
      }
      if constexpr (MASK) {
        // sdpa's additive mask (sam3/nn.rs:29-32) joins the scaled scores in log2 units:
        // s <- s * scale * log2(e) + mask * log2(e); the softmax below then takes s as it is
        const T* mrow = reinterpret_cast<const T*>(p.mask) + bi * p.sm[0] + head * p.sm[1] +
                        (long)(qvalid ? qidx : 0) * p.sm[2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = (t << 6) + 32 * mb + 8 * (e >> 2) + 4 * hh + (e & 3);
            const float mv = key < kend ? to_f32(mrow[(long)key * p.sm[3]]) : 0.f;
            s_cur[mb][e] = fmaf(s_cur[mb][e], sc, mv * kFlashLog2e);
          }
      }
      float mm = s_cur[0][0];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e) mm = max_nc(mm, s_cur[mb][e]);
      const float mt = max_with_partner32(MASK ? mm : mm * sc);
      if (wave_any(mt > m_run + kFlashSlack)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = exp2_fast(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int ob = 0; ob < MBO; ++ob) o[ob] *= alpha;
        m_run = m_new;
      }
      qk(ks_base + ((i + 1) & 1) * KBUF, s_nxt);
      // with a mask, whole tiles (a row's first ones included) can be -inf: m_run is still -inf there
      const float c = MASK && m_run == -INFINITY ? 0.f : -m_run;
      constexpr float one = 1.f;
      const float scs = MASK ? one : sc;  // the masked scores are scaled already
      // P, and its sum as the P.V product sees it: f16 sums the rounded P (v_dot2 with ones), so that
      // numerator and denominator weigh each key alike (a dominant key's rounding cancels); bf16 (P as
      // hi + lo) sums the f32 P
      float lsum = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = exp2_fast(fmaf(s_cur[u >> 1][8 * (u & 1) + j], scs, c));
        b[u] = pack8(pv, (X8*)nullptr);
        if constexpr (kSplitP) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            lsum += pv[j];
            pv[j] -= to_f32(b[u][j]);
          }
          blo[u] = pack8(pv, (X8*)nullptr);
        } else {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int j = 0; j < 8; j += 2)
            lsum = __builtin_amdgcn_fdot2(h2{b[u][j], b[u][j + 1]}, h2{(f16)1.f, (f16)1.f}, lsum, false);
        }
      }
      l_run += lsum;
    }
    // K(t+2) replaces K(t), whose scores were taken one step ago; only then is V(t+1) fetched, so at
    // most one tile's staging registers are live
    store_k(i & 1);
    load_v(min(t + 1, tl));
    {
      // O^T += V^T . P^T; in bf16, P is split into hi + lo bf16 terms so the product keeps ~16 bits of P
      const T* vb = vs_base + (i & 1) * VBUF;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int ob = 0; ob < MBO; ++ob) {
          const T* p0 = vb + voff[u][0] + 32 * ob;
          const T* p1 = vb + voff[u][1] + 32 * ob;
          const X8 a = join8<T>(lds_read_tr16(p0), lds_read_tr16(p1));
          o[ob] = mma32(a, b[u], o[ob]);
          if (kSplitP) o[ob] = mma32(a, blo[u], o[ob]);
        }
      }
    }
    store_v((i + 1) & 1);  // V(t+1) replaces V(t-1)
    __syncthreads();
  };

  // A wave whose 32 queries are all past the end computes on zero queries (no divergent branch in the
  // loop) and stores nothing.
  f32x16 sa[2], sb[2];
  qk(ks_base, sa);
  __syncthreads();  // every wave has read K(0) before step 0 overwrites its buffer with K(2)
  for (int t = t_begin; t < t_end; t += 2) {
    step(t, sa, sb);
    if (t + 1 < t_end) step(t + 1, sb, sa);
  }
  (void)ntiles;

  if (!active) return;
  // lane holds O^T[32*ob + 8*a + 4*hh + b][query n]
  const float l = sum_with_partner32(l_run);
  if (!qvalid) return;
  if (p.nsplit == 1) {
    const float inv = 1.f / l;
    T* orow = reinterpret_cast<T*>(p.out) + bi * p.so[0] + head * p.so[2] + (long)qidx * p.so[1];
#pragma unroll
    for (int ob = 0; ob < MBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * ob + 8 * a + 4 * hh;
        if (d0 < d) {
          typename Vec<T>::x4 w4;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) w4[bb] = from_f32<T>(o[ob][4 * a + bb] * inv);
          *reinterpret_cast<typename Vec<T>::x4*>(orow + d0) = w4;
        }
      }
  } else {
    // partial O [split][bh][q][DP] (unnormalised, f32) and (max, sum) [split][bh][q][2]
    const long row = ((long)split * p.b * p.h + bhi) * p.lq + qidx;
    float* prow = p.opart + row * DP;
#pragma unroll
    for (int ob = 0; ob < MBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * ob + 8 * a + 4 * hh;
        f32x4 w4;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) w4[bb] = o[ob][4 * a + bb];
        *reinterpret_cast<f32x4*>(prow + d0) = w4;
      }
    if (hh == 0) {
      float2 ml;
      ml.x = m_run;
      ml.y = l;
      *reinterpret_cast<float2*>(p.ml + row * 2) = ml;
    }
  }
}

// out[b, q, h, :] = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, M = max_s m_s, with O_s the
// unnormalised f32 partial. A row takes DP / 8 lanes of 8 consecutive columns each (two 16-byte reads
// per split), so a workgroup merges 256 / (DP / 8) rows.
template <typename T, int DP>
__global__ __launch_bounds__(256) void flash_combine_kernel(FlashParams p) {
  constexpr int LPR = DP / 8;     // lanes per row
  constexpr int RPB = 256 / LPR;  // rows per workgroup (DP 96: 21, and 4 idle threads)
  if (threadIdx.x >= RPB * LPR) return;
  const int c = 8 * (threadIdx.x % LPR);
  const long row = (long)blockIdx.x * RPB + threadIdx.x / LPR;  // (bh, q)
  const long rows = (long)p.b * p.h * p.lq;
  if (row >= rows) return;
  const long plane = rows;
  // splits in chunks of 8: every (max, sum) and partial read of a chunk is issued before any is used;
  // a later chunk with a larger max rescales what is summed so far (one chunk up to 8 splits)
  float mx = -INFINITY, den = 0.f;
  float acc[8] = {};
  for (int s0 = 0; s0 < p.nsplit; s0 += 8) {
    float2 ml[8];
    float o[8][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const long r = ((long)(s0 + j) * plane + row);
      if (s0 + j < p.nsplit) {
        ml[j] = *reinterpret_cast<const float2*>(p.ml + r * 2);
        const f32x4* src = reinterpret_cast<const f32x4*>(p.opart + r * DP + c);
        const f32x4 a = src[0], b = src[1];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          o[j][k] = a[k];
          o[j][4 + k] = b[k];
        }
      } else {
        ml[j] = make_float2(-INFINITY, 0.f);
#pragma unroll
        for (int k = 0; k < 8; ++k) o[j][k] = 0.f;
      }
    }
    float cm = mx;
#pragma unroll
    for (int j = 0; j < 8; ++j) cm = fmaxf(cm, ml[j].x);
    // a split (or padding slot) whose keys are all masked has max -inf and sum 0: it weighs exactly 0,
    // also while every split so far is of that kind (mx = -inf), so that no -inf - -inf reaches exp2
    if (s0 > 0) {
      const float r = mx == -INFINITY ? 0.f : exp2_fast(mx - cm);
      den *= r;
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] *= r;
    }
    mx = cm;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float w = ml[j].x == -INFINITY ? 0.f : exp2_fast(ml[j].x - mx);
      const float wl = w * ml[j].y;
      den += wl;
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] += w * o[j][k];
    }
  }
  if (c >= p.d) return;
  const float inv = 1.f / den;
  const int bhi = (int)(row / p.lq), q = (int)(row % p.lq);
  const int bi = bhi / p.h, head = bhi % p.h;
  T* orow = reinterpret_cast<T*>(p.out) + bi * p.so[0] + head * p.so[2] + (long)q * p.so[1];
  typename Vec<T>::x8 w8;
#pragma unroll
  for (int j = 0; j < 8; ++j) w8[j] = from_f32<T>(acc[j] * inv);
  *reinterpret_cast<typename Vec<T>::x8*>(orow + c) = w8;
}

// ---------------------------------------------------------------------------------------------- launch

template <typename T, int DP, int NW>
static hipError_t launch_flash(FlashParams p, bool ropeq, hipStream_t stream) {
  typedef FlashGeom<T, DP, NW> FG;
  hipError_t e;
  if (DP == 256 && !p.mask && flash256_eligible(p, (int)sizeof(T))) {
    e = flash256_launch(__is_same(T, f16) ? kF16 : kBF16, p, ropeq, stream);
  } else {
    const int which = p.mask ? 2 : ropeq ? 1 : 0;  // a masked call has no RoPE
    auto kern = which == 2   ? flash_fwd_kernel<T, DP, NW, false, true>
                : which == 1 ? flash_fwd_kernel<T, DP, NW, true, false>
                             : flash_fwd_kernel<T, DP, NW, false, false>;
    static std::atomic<unsigned long long> lds_done[3];  // opt-in to more than 64 KB of dynamic LDS
    e = lds_opt_in(lds_done[which], (const void*)kern, (int)FG::LDS);
    if (e != hipSuccess) return e;
    const long blocks = (long)p.b * p.h * p.qblocks * p.nsplit;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(FG::NT), FG::LDS, stream, p);
    e = hipGetLastError();
  }
  if (e != hipSuccess || p.nsplit == 1) return e;
  const long rows = (long)p.b * p.h * p.lq;
  constexpr int kRowsPerBlock = 256 / (DP / 8);
  hipLaunchKernelGGL((flash_combine_kernel<T, DP>), dim3((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                     dim3(256), 0, stream, p);
  return hipGetLastError();
}

// Waves per workgroup of the f16 / bf16 kernel. Up to head dim 64 a wave needs 161-176 registers, so
// two 8-wave workgroups (four waves per SIMD) would not fit a CU and an 8-wave workgroup runs alone on
// it; 4-wave workgroups run two or three to a CU, each on its own barrier schedule. Head dims 96 and
// 128 need 221-240 registers, two waves per SIMD either way: 8 waves (each K/V tile serves twice the
// queries) for key ranges past 16 tiles, 4 for shorter ones (Hiera's windows at head dim 72), where
// the query blocks of 256 leave CUs idle or padded (measured: 196 x 196 windows 32.3 -> 23.1 us with 4,
// 4096 x 4096 over 16 heads at 128 179 -> 220 us). Head dim 256 takes 4.
int flash_padded_dim(int d) { return d <= 32 ? 32 : d <= 64 ? 64 : d <= 96 ? 96 : d <= 128 ? 128 : 256; }

// Queries per workgroup: 32 per wave (the f32 kernel keeps 8 waves up to head dim 128).
int flash_queries_per_block(int dtype, int d, int lk) {
  const int dp = flash_padded_dim(d);
  if (dtype == kF32) return 32 * (dp <= 128 ? 8 : 4);
  return 32 * (dp <= 64 ? 4 : dp <= 128 ? (lk <= 16 * 64 ? 4 : 8) : 4);
}

// Key splits, at least 2 key tiles per split. 4-wave f16 / bf16 workgroups (three resident per CU in
// f16 up to head dim 64, two otherwise): as many splits as still fit one round of resident workgroups,
// none once the query blocks alone fill it. Measured on f16 against other split counts: a short key
// range (SAM 3's 576-token windows) loses 35% when split in two, and 4096 x 4096 over 16 heads 9%,
// while 12 heads (384 query blocks) gain 13% from two splits. Otherwise (8 waves, f32, head dim 256):
// enough workgroups to give every CU its resident share (one workgroup per CU at head dim 256, two
// below).
void flash_plan(int dtype, int b, int h, int lq, int lk, int d, int cus, int* qblocks, int* nsplit, int* tps) {
  const int qpb = flash_queries_per_block(dtype, d, lk);
  *qblocks = (lq + qpb - 1) / qpb;
  const int tiles = (lk + 63) / 64;
  const long base = (long)b * h * *qblocks;
  const int dp = flash_padded_dim(d);
  int ns = 1;
  if (dtype != kF32 && dp <= 128 && qpb == 128) {
    const long slots = (long)cus * (dtype == kF16 && dp <= 64 ? 3 : 2);
    if (base < slots) ns = (int)(slots / base);
  } else {
    const long target = (long)cus * (dp <= 128 ? 2 : 1);
    if (base < target) ns = (int)((target + base - 1) / base);
  }
  const int maxs = tiles / 2 > 1 ? tiles / 2 : 1;
  if (ns > maxs) ns = maxs;
  if (ns > 64) ns = 64;
  int t = (tiles + ns - 1) / ns;
  *tps = t;
  *nsplit = (tiles + t - 1) / t;
}

size_t flash_partial_bytes(int b, int h, int lq, int d, int nsplit) {
  if (nsplit <= 1) return 0;
  return (size_t)nsplit * b * h * lq * (flash_padded_dim(d) + 2) * sizeof(float);
}

// The waves of the plan's query blocks (flash_queries_per_block) pick the instance.
template <typename T>
static hipError_t flash_dispatch(FlashParams p, bool ropeq, hipStream_t s) {
  const bool four = flash_queries_per_block(__is_same(T, f16) ? kF16 : kBF16, p.d, p.lk) == 128;
  switch (flash_padded_dim(p.d)) {
    case 32: return launch_flash<T, 32, 4>(p, ropeq, s);
    case 64: return launch_flash<T, 64, 4>(p, ropeq, s);
    case 96: return four ? launch_flash<T, 96, 4>(p, ropeq, s) : launch_flash<T, 96, 8>(p, ropeq, s);
    case 128: return four ? launch_flash<T, 128, 4>(p, ropeq, s) : launch_flash<T, 128, 8>(p, ropeq, s);
    default: return launch_flash<T, 256, 4>(p, ropeq, s);
  }
}

template <int DP>
static hipError_t combine_f32(FlashParams p, hipStream_t stream) {
  const long rows = (long)p.b * p.h * p.lq;
  constexpr int kRowsPerBlock = 256 / (DP / 8);
  hipLaunchKernelGGL((flash_combine_kernel<float, DP>), dim3((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                     dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t flash_combine_f32(FlashParams p, int dp, hipStream_t stream) {
  switch (dp) {
    case 32: return combine_f32<32>(p, stream);
    case 64: return combine_f32<64>(p, stream);
    case 96: return combine_f32<96>(p, stream);
    case 128: return combine_f32<128>(p, stream);
    default: return combine_f32<256>(p, stream);
  }
}

hipError_t flash_attn_half(int dtype, FlashParams p, bool ropeq, hipStream_t stream) {
  if (dtype == kF16) return flash_dispatch<f16>(p, ropeq, stream);
  return flash_dispatch<bf16>(p, ropeq, stream);
}

}  // namespace samhip
