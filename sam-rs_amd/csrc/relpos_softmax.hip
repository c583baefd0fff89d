// Softmax over materialised scores with the decomposed relative-position bias, for gfx950:
//
//   out[r, k] = softmax_k( scale * s[r, k] + q[r] . Th[i - kh + H-1] + q[r] . Tw[j - kw + W-1] )
//
// for score rows r (i = (r mod N) / W, j = r mod W, N = H*W) and keys k = kh*W + kw. This is the
// contract of the reference's relpos_softmax (kernels.rs:12-43; its CPU twin kernels.rs:62-105), for
// callers that already hold the score matrix; the fused attention never materialises it.
//
// The work is streaming: each row is read once and written once (2 * N elements), so the kernel is
// built around HBM traffic rather than arithmetic.
//   * A wave owns 32 consecutive rows (16 for 16-bit rows of one vector per lane that the next kernel
//     does not take: the waves then cover twice as many rows in flight). Their bias dot products are one small GEMM, G = Table . Q^T
//     (all (2H-1) + (2W-1) table rows against the 32 q rows), on the MFMA (32x32x16 f16/bf16,
//     32x32x2 f32), one 32-row block of the table at a time. Each lane then holds one q row's
//     products with 16 table rows and scatters those that fall on the row's diagonal band into a
//     wave-private LDS array, bias[row][kw] (Rw) and bias[row][W + kh] (Rh). q rows are indexed by the
//     global row r, so a wave's rows may straddle windows or heads.
//   * Rows then stream through registers as 16-byte (or, when a row is not a multiple of 16 bytes,
//     8-byte) vectors: a lane owns vectors lane, lane + 64, ...; a vector's (kh, kw) is fixed per lane
//     for all rows. Max and sum are reduced over the wave on the VALU (DPP row rotations, then
//     v_permlane16_swap and v_permlane32_swap); no LDS reductions and no workgroup barriers.
//   * Several rows are in flight per wave: rows are loaded in groups of up to 8 vectors per lane, two
//     groups ahead of the one being computed (a ring of three register buffers).
//   * Rows that are not a multiple of 8 bytes, or that would need more than 16 vectors per lane, take a
//     two-pass loop (online max and sum, then the outputs) over scalars.
//   * 16-bit rows of at most 64 vectors (the 14x14 windows) take relpos_softmax_quad_kernel: 16 lanes
//     per row, four rows per instruction, reductions inside a 16-lane group.
// Arithmetic: the logit is (s * scale + Rh) + Rw with separate f32 roundings, as the reference's CPU
// path computes it; exp(x - max) as exp2((x - max) * log2 e); P = e * (1 / sum).
#include "common.hpp"

#pragma clang diagnostic ignored "-Wunused-parameter"

namespace samhip {

namespace rsm {
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaves = 4;   // waves per workgroup (independent)
constexpr int kRows = 32;   // rows per wave (bias scratch and the MFMA bias prologue: one 32-row block)
// Rows a wave of the vector kernel runs. 16-bit rows of one vector per lane (ITEMS == 1, the 14x14
// windows) are short, so a wave spends its time waiting on each group's loads and reductions; 16 rows
// per wave double the waves in flight (the prologue's other 16 bias rows are computed and not used). In
// f32 the prologue runs on the 32x32x2 MFMA and costs more than the waves gain, so f32 keeps 32.
constexpr int vec_rows_per_wave(int items, int elem_bytes) { return items == 1 && elem_bytes == 2 ? 16 : kRows; }
}  // namespace rsm

// Wave64 reductions on the VALU, with no LDS round trip: DPP row rotations by 1, 2, 4 and 8 reduce each
// row of 16 lanes (every lane ends with its row's result), then v_permlane16_swap and
// v_permlane32_swap combine the rows.
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 | N, 0xf, 0xf, false));
}
__device__ __forceinline__ float partner16(float v, bool take_max) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return take_max ? fmaxf(a, b) : a + b;
}
__device__ __forceinline__ float wave_max64(float v) {
  v = fmaxf(v, row_ror<1>(v));
  v = fmaxf(v, row_ror<2>(v));
  v = fmaxf(v, row_ror<4>(v));
  v = fmaxf(v, row_ror<8>(v));
  return max_with_partner32(partner16(v, true));
}
__device__ __forceinline__ float wave_sum64(float v) {
  v += row_ror<1>(v);
  v += row_ror<2>(v);
  v += row_ror<4>(v);
  v += row_ror<8>(v);
  return sum_with_partner32(partner16(v, false));
}

// 8 consecutive elements of a row of `ld` elements (zero past `len`), as an MFMA operand.
template <typename T>
__device__ __forceinline__ typename Vec<T>::x8 load8(const T* row, int k, int len, bool vec) {
  typedef typename Vec<T>::x8 X8;
  if (vec && k + 8 <= len) return *reinterpret_cast<const X8*>(row + k);
  X8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = k + e < len ? row[k + e] : (T)0.f;
  return r;
}

// The wave's bias rows: bias[row][0 .. W) = Rw, bias[row][rho .. rho+H) = Rh (rho >= W), row pitch bst
// floats (a multiple of 4, so a row's Rw run can be read as 16-byte vectors). Lane l holds, per 32-row
// block tb of the table, G[tb + m][row n] for m = 8 (e/4) + 4 (l/32) + e%4 (n = l % 32), the products of
// the wave's q row n with table rows tb .. tb+31, and scatters those on the row's diagonal band.
__device__ __forceinline__ void scatter_band(const f32x16& g, float* brow, int tb, int hh, int i, int j, int H,
                                             int W, int rho) {
  const int th = 2 * H - 1, trows = th + 2 * W - 1;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int tr = tb + 8 * (e >> 2) + 4 * hh + (e & 3);
    if (tr < th) {
      const int kh = i + H - 1 - tr;
      if (kh >= 0 && kh < H) brow[rho + kh] = g[e];
    } else if (tr < trows) {
      const int kw = j + W - 1 - (tr - th);
      if (kw >= 0 && kw < W) brow[kw] = g[e];
    }
  }
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Head dims up to 128 and a multiple of 8 (SAM's 64 and 80): the q fragments are loaded once, and
// every operand load of a table block is issued before its MFMAs, so the prologue waits on memory
// about once per block instead of once per k-step. Rows past the table read its last row (not
// scattered).
template <typename T>
__device__ __forceinline__ void build_bias_short(const T* qrow, const T* tab, float* brow, int i, int j, int H, int W,
                                                 int HD, int rho) {
  const int lane = threadIdx.x & 63, n = lane & 31, hh = lane >> 5;
  const int trows = 2 * H - 1 + 2 * W - 1;
  if constexpr (__is_same(T, float)) {
    // 32x32x2 f32: MFMA step t pairs dim t (lanes 0-31) with dim HD/2 + t (lanes 32-63) of the q row
    // (B) and of the table row (A); HD/2 is a multiple of 4, so each half moves as 16-byte vectors
    const int half = HD / 2, base = hh * half;
    float qv[64];
#pragma unroll
    for (int c = 0; c < 64; c += 4) {
      const f32x4 v = c < half ? *reinterpret_cast<const f32x4*>(qrow + base + c) : f32x4{};
#pragma unroll
      for (int u = 0; u < 4; ++u) qv[c + u] = v[u];
    }
    for (int tb = 0; tb < trows; tb += 32) {
      const float* trow = tab + (long)min(tb + n, trows - 1) * HD;
      float tv[64];
#pragma unroll
      for (int c = 0; c < 64; c += 4) {
        const f32x4 v = c < half ? *reinterpret_cast<const f32x4*>(trow + base + c) : f32x4{};
#pragma unroll
        for (int u = 0; u < 4; ++u) tv[c + u] = v[u];
      }
      f32x16 g = f32x16{};
#pragma unroll
      for (int t = 0; t < 64; ++t)
        if (t < half) g = __builtin_amdgcn_mfma_f32_32x32x2f32(tv[t], qv[t], g, 0, 0, 0);
      scatter_band(g, brow, tb, hh, i, j, H, W, rho);
    }
  } else {
    typedef typename Vec<T>::x8 X8;
    const int ks = (HD + 15) / 16;  // k-steps; at HD % 16 == 8 the last one's upper half is zero
    X8 qf[8], a[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int k = 16 * s + 8 * hh;
      qf[s] = k < HD ? *reinterpret_cast<const X8*>(qrow + k) : X8{};
    }
    for (int tb = 0; tb < trows; tb += 32) {
      const T* trow = tab + (long)min(tb + n, trows - 1) * HD;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int k = 16 * s + 8 * hh;
        a[s] = k < HD ? *reinterpret_cast<const X8*>(trow + k) : X8{};
      }
      f32x16 g = f32x16{};
#pragma unroll
      for (int s = 0; s < 8; ++s)
        if (s < ks) g = mma32(a[s], qf[s], g);
      scatter_band(g, brow, tb, hh, i, j, H, W, rho);
    }
  }
}

// Any head dim (up to 256): one k-step at a time.
template <typename T>
__device__ __forceinline__ void build_bias_long(const T* qrow, const T* tab, float* brow, int i, int j, int H, int W,
                                                int HD, int rho) {
  const int lane = threadIdx.x & 63, n = lane & 31, hh = lane >> 5;
  const int trows = 2 * H - 1 + 2 * W - 1;
  for (int tb = 0; tb < trows; tb += 32) {
    const T* trow = tab + (long)min(tb + n, trows - 1) * HD;
    f32x16 g = f32x16{};
    if constexpr (__is_same(T, float)) {
      for (int k0 = 0; k0 < HD; k0 += 2) {
        const int k = k0 + hh;
        g = __builtin_amdgcn_mfma_f32_32x32x2f32(k < HD ? trow[k] : 0.f, k < HD ? qrow[k] : 0.f, g, 0, 0, 0);
      }
    } else {
      for (int k0 = 0; k0 < HD; k0 += 16) {
        const int k = k0 + 8 * hh;
        g = mma32(load8(trow, k, HD, HD % 8 == 0), load8(qrow, k, HD, HD % 8 == 0), g);
      }
    }
    scatter_band(g, brow, tb, hh, i, j, H, W, rho);
  }
}

template <typename T>
__device__ __forceinline__ void build_bias(const T* q, const T* tab, float* bias, long r0, long rows, int H, int W,
                                           int HD, int bst, int rho) {
  const int lane = threadIdx.x & 63, n = lane & 31;
  const int N = H * W;
  const long rq = min(r0 + n, rows - 1);
  const int rem = (int)(rq % N);
  const int i = rem / W, j = rem - (rem / W) * W;
  const T* qrow = q + rq * HD;
  float* brow = bias + n * bst;
  if (HD <= 128 && HD % 8 == 0)
    build_bias_short(qrow, tab, brow, i, j, H, W, HD, rho);
  else
    build_bias_long(qrow, tab, brow, i, j, H, W, HD, rho);
  wave_sync();
}

template <typename T, int VB> struct Raw;  // VB bytes of a row as loaded
template <typename T> struct Raw<T, 16> { typedef u32x4 type; };
template <typename T> struct Raw<T, 8> { typedef u32x2 type; };

template <typename T, int VB>
__device__ __forceinline__ float raw_elem(const typename Raw<T, VB>::type& v, int e) {
  typedef T TV __attribute__((ext_vector_type(VB / sizeof(T))));
  return to_f32(__builtin_bit_cast(TV, v)[e]);
}

// Vectorised rows: VB-byte vectors of VE = VB / sizeof(T) elements, ITEMS vectors per lane and row.
// AW: W is a multiple of VE, so every vector lies in one grid row (one Rh value, VE consecutive Rw).
template <typename T, int VB, int ITEMS, bool AW>
__global__ __launch_bounds__(rsm::kWaves * 64) void relpos_softmax_vec_kernel(const T* __restrict__ s,
                                                                             const T* __restrict__ q,
                                                                             const T* __restrict__ tab,
                                                                             T* __restrict__ out, long rows, int H,
                                                                             int W, int HD, float scale, int bst) {
#pragma clang fp contract(off)
  using namespace rsm;
  typedef typename Raw<T, VB>::type RV;
  constexpr int VE = VB / (int)sizeof(T);
  constexpr int G = ITEMS >= 8 ? 1 : 8 / ITEMS;  // rows per load group
  static_assert(!AW || VE % 4 == 0, "vector Rw reads cover whole 16-byte runs");
  extern __shared__ float bias_lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int RPW = vec_rows_per_wave(ITEMS, (int)sizeof(T));
  const long r0 = ((long)blockIdx.x * kWaves + wave) * RPW;
  if (r0 >= rows) return;  // the waves of a workgroup share nothing
  float* bias = bias_lds + wave * kRows * bst;
  const int N = H * W, nvec = N / VE;
  const int nrows = (int)min((long)RPW, rows - r0);
  // (kh << 16 | kw) of the first element of each of this lane's vectors: the same for every row
  int khw[ITEMS];
#pragma unroll
  for (int t = 0; t < ITEMS; ++t) {
    const int k = (lane + 64 * t) * VE;
    const int kh = k / W;
    khw[t] = (kh << 16) | (k - kh * W);
  }
  auto load_group = [&](int g0, RV (&buf)[G][ITEMS]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int rl = g0 + g;
      const T* srow = s + (r0 + (rl < nrows ? rl : 0)) * (long)N;
#pragma unroll
      for (int t = 0; t < ITEMS; ++t) {
        const int v = lane + 64 * t;
        buf[g][t] = v < nvec ? *reinterpret_cast<const RV*>(srow + v * VE) : RV{};
      }
    }
  };
  // logits of row g0 + g into x (padding lanes -inf); returns this lane's max
  auto logits = [&](int rl, const RV (&raw)[ITEMS], float (&x)[ITEMS][VE]) {
    const float* brow = bias + min(rl, nrows - 1) * bst;
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < ITEMS; ++t) {
      const bool ok = lane + 64 * t < nvec;
      int kh = khw[t] >> 16, kw = khw[t] & 0xffff;
      if constexpr (AW) {
        const float rh = brow[W + kh];
        float rw[VE];
#pragma unroll
        for (int e4 = 0; e4 < VE; e4 += 4) {
          const f32x4 r4 = *reinterpret_cast<const f32x4*>(brow + kw + e4);
#pragma unroll
          for (int u = 0; u < 4; ++u) rw[e4 + u] = r4[u];
        }
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          const float v = (raw_elem<T, VB>(raw[t], e) * scale + rh) + rw[e];
          x[t][e] = ok ? v : -INFINITY;
          m = fmaxf(m, x[t][e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          const float v = (raw_elem<T, VB>(raw[t], e) * scale + brow[W + kh]) + brow[kw];
          x[t][e] = ok ? v : -INFINITY;
          m = fmaxf(m, x[t][e]);
          if (++kw == W) {
            kw = 0;
            ++kh;
          }
        }
      }
    }
    return m;
  };
  // the reductions, exponentials and stores of a whole group: each step runs for all of the group's
  // rows before the next, so the rows' cross-lane exchanges overlap (one basic block, no early exits)
  auto finish = [&](int g0, float (&x)[G][ITEMS][VE], float (&m)[G]) {
#pragma unroll
    for (int g = 0; g < G; ++g) m[g] = wave_max64(m[g]);
    float sum[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sum[g] = 0.f;
#pragma unroll
      for (int t = 0; t < ITEMS; ++t)
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          x[g][t][e] = exp2_fast((x[g][t][e] - m[g]) * kLog2e);
          sum[g] += x[g][t][e];
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) sum[g] = 1.f / wave_sum64(sum[g]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      T* orow = out + (r0 + min(g0 + g, nrows - 1)) * (long)N;
#pragma unroll
      for (int t = 0; t < ITEMS; ++t) {
        const int v = lane + 64 * t;
        if (v < nvec && g0 + g < nrows) {
          typedef T TV __attribute__((ext_vector_type(VE)));
          TV o;
#pragma unroll
          for (int e = 0; e < VE; ++e) o[e] = from_f32<T>(x[g][t][e] * sum[g]);
          *reinterpret_cast<TV*>(orow + v * VE) = o;
        }
      }
    }
  };
  // A ring of three load buffers: two groups are in flight while a third is computed. A group's buffer
  // is refilled (with the group three ahead) as soon as its logits are formed, so the loads land while
  // this group's reductions, exponentials and stores run and while the next group is computed. The
  // first two groups' loads go out before the bias prologue.
  RV b0[G][ITEMS], b1[G][ITEMS], b2[G][ITEMS];
  load_group(0, b0);
  if (G < nrows) load_group(G, b1);
  build_bias(q, tab, bias, r0, rows, H, W, HD, bst, W);
  auto step = [&](int g0, RV (&cur)[G][ITEMS], RV (&spare)[G][ITEMS]) {
    if (g0 >= nrows) return;
    float x[G][ITEMS][VE], m[G];
#pragma unroll
    for (int g = 0; g < G; ++g) m[g] = logits(g0 + g, cur[g], x[g]);
    if (g0 + 2 * G < nrows) load_group(g0 + 2 * G, spare);
    finish(g0, x, m);
  };
  for (int g0 = 0; g0 < nrows; g0 += 3 * G) {
    step(g0, b0, b2);
    step(g0 + G, b1, b0);
    step(g0 + 2 * G, b2, b1);
  }
}

// Short 16-bit rows (at most 64 vectors, W >= the vector's element count: the 14x14 windows' 196 keys
// are 49 vectors of 8 bytes): 16 lanes per row, so one instruction covers four rows and a row's max and
// sum take four DPP rotations inside its 16-lane group, with no permlane steps. A wave owns the 32 rows
// of its bias block and runs them as 8 quads of rows.
// Bias rows: Rw at [0, W) and repeated at [W, W + VE), so that a vector's VE Rw values are consecutive
// even where it wraps into the next grid row; Rh at [W + VE, W + VE + H); one spare float after it.
template <typename T, int VB, int VPL>
__global__ __launch_bounds__(rsm::kWaves * 64) void relpos_softmax_quad_kernel(const T* __restrict__ s,
                                                                              const T* __restrict__ q,
                                                                              const T* __restrict__ tab,
                                                                              T* __restrict__ out, long rows, int H,
                                                                              int W, int HD, float scale, int bst) {
#pragma clang fp contract(off)
  using namespace rsm;
  typedef typename Raw<T, VB>::type RV;
  constexpr int VE = VB / (int)sizeof(T);
  constexpr int kQuads = kRows / 4;
  extern __shared__ float bias_lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long r0 = ((long)blockIdx.x * kWaves + wave) * kRows;
  if (r0 >= rows) return;  // the waves of a workgroup share nothing
  float* bias = bias_lds + wave * kRows * bst;
  const int N = H * W, nvec = N / VE;
  const int nrows = (int)min((long)kRows, rows - r0);
  const int rq = lane >> 4, li = lane & 15;
  RV raw[kQuads][VPL];
  auto load_quad = [&](int qd) {
    const int rl = 4 * qd + rq;
    const T* srow = s + (r0 + (rl < nrows ? rl : 0)) * (long)N;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int v = li + 16 * j;
      raw[qd][j] = v < nvec ? *reinterpret_cast<const RV*>(srow + v * VE) : RV{};
    }
  };
  // Half the quads are requested before the bias prologue and half after it: all eight before it
  // keep 196 registers live through the prologue's operands (two waves per SIMD, a second round of
  // workgroups at the 14x14 window layer's 2450 waves), none before it leaves the first loads exposed.
  constexpr int kPre = 4;
#pragma unroll
  for (int qd = 0; qd < kPre; ++qd) load_quad(qd);
  const int rho = W + VE;
  build_bias(q, tab, bias, r0, rows, H, W, HD, bst, rho);
#pragma unroll
  for (int qd = kPre; qd < kQuads; ++qd) load_quad(qd);
  if (lane < 32) {
#pragma unroll
    for (int e = 0; e < VE; ++e) bias[lane * bst + W + e] = bias[lane * bst + e];
  }
  wave_sync();
  // this lane's vectors: grid row and column of the first element, and the first element that lies in
  // the next grid row (vectors past the row read row 0's bias and are discarded)
  int kh0[VPL], kw0[VPL], wrap[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int v = li + 16 * j;
    const int k = v < nvec ? v * VE : 0;
    kh0[j] = k / W;
    kw0[j] = k - kh0[j] * W;
    wrap[j] = W - kw0[j];
  }
#pragma unroll
  for (int qd = 0; qd < kQuads; ++qd) {
    const int rl = 4 * qd + rq;
    const float* brow = bias + min(rl, nrows - 1) * bst;
    float x[VPL][VE];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const bool ok = li + 16 * j < nvec;
      const float rh0 = brow[rho + kh0[j]], rh1 = brow[rho + kh0[j] + 1];
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const float v = (raw_elem<T, VB>(raw[qd][j], e) * scale + (e < wrap[j] ? rh0 : rh1)) + brow[kw0[j] + e];
        x[j][e] = ok ? v : -INFINITY;
        m = fmaxf(m, x[j][e]);
      }
    }
    m = fmaxf(m, row_ror<1>(m));
    m = fmaxf(m, row_ror<2>(m));
    m = fmaxf(m, row_ror<4>(m));
    m = fmaxf(m, row_ror<8>(m));
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        x[j][e] = exp2_fast((x[j][e] - m) * kLog2e);
        sum += x[j][e];
      }
    sum += row_ror<1>(sum);
    sum += row_ror<2>(sum);
    sum += row_ror<4>(sum);
    sum += row_ror<8>(sum);
    const float inv = 1.f / sum;
    if (rl < nrows) {
      T* orow = out + (r0 + rl) * (long)N;
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        const int v = li + 16 * j;
        if (v < nvec) {
          typedef T TV __attribute__((ext_vector_type(VE)));
          TV o;
#pragma unroll
          for (int e = 0; e < VE; ++e) o[e] = from_f32<T>(x[j][e] * inv);
          *reinterpret_cast<TV*>(orow + v * VE) = o;
        }
      }
    }
  }
}

// Any row length: an online (max, sum) pass over the row, then a pass that writes the outputs.
template <typename T>
__global__ __launch_bounds__(rsm::kWaves * 64) void relpos_softmax_scalar_kernel(const T* __restrict__ s,
                                                                                const T* __restrict__ q,
                                                                                const T* __restrict__ tab,
                                                                                T* __restrict__ out, long rows,
                                                                                int H, int W, int HD, float scale,
                                                                                int bst) {
#pragma clang fp contract(off)
  using namespace rsm;
  extern __shared__ float bias_lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long r0 = ((long)blockIdx.x * kWaves + wave) * kRows;
  if (r0 >= rows) return;
  float* bias = bias_lds + wave * kRows * bst;
  build_bias(q, tab, bias, r0, rows, H, W, HD, bst, W);
  const int N = H * W;
  const int nrows = (int)min((long)kRows, rows - r0);
  for (int rl = 0; rl < nrows; ++rl) {
    const T* srow = s + (r0 + rl) * (long)N;
    const float* brow = bias + rl * bst;
    float m = -INFINITY, sum = 0.f;
    for (int k = lane; k < N; k += 64) {
      const int kh = k / W, kw = k - kh * W;
      const float x = (to_f32(srow[k]) * scale + brow[W + kh]) + brow[kw];
      // a -inf score adds nothing (also while m is still -inf); a NaN score makes the sum NaN, so the
      // row comes out NaN as the reference's softmax returns it
      if (x > m) {
        sum = sum * exp2_fast((m - x) * kLog2e) + 1.f;
        m = x;
      } else if (x != -INFINITY) {
        sum += exp2_fast((x - m) * kLog2e);
      }
    }
    const float mw = wave_max64(m);
    // a lane with no finite score (m = -inf) holds 0, or NaN after a NaN score
    sum = m == -INFINITY ? sum : sum * exp2_fast((m - mw) * kLog2e);
    const float inv = 1.f / wave_sum64(sum);
    T* orow = out + (r0 + rl) * (long)N;
    for (int k = lane; k < N; k += 64) {
      const int kh = k / W, kw = k - kh * W;
      const float x = (to_f32(srow[k]) * scale + brow[W + kh]) + brow[kw];
      orow[k] = from_f32<T>(f32_result(exp2_fast((x - mw) * kLog2e) * inv));
    }
  }
}

template <typename T, int VB, int ITEMS, bool AW>
static hipError_t launch_vec(const void* s, const void* q, const void* tab, void* out, long rows, int h, int w, int hd,
                             float scale, unsigned blocks, size_t lds, int bst, hipStream_t stream) {
  auto kern = relpos_softmax_vec_kernel<T, VB, ITEMS, AW>;
  static std::atomic<unsigned long long> done{0};
  if (const hipError_t e = lds_opt_in(done, (const void*)kern, (int)lds); e != hipSuccess) return e;
  (void)blocks;  // the 32-row count of the scalar kernel; this kernel's waves run vec_rows_per_wave rows
  const long rows_per_block = (long)rsm::kWaves * rsm::vec_rows_per_wave(ITEMS, (int)sizeof(T));
  const unsigned nblocks = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL(kern, dim3(nblocks), dim3(rsm::kWaves * 64), lds, stream, (const T*)s, (const T*)q,
                     (const T*)tab, (T*)out, rows, h, w, hd, scale, bst);
  return hipGetLastError();
}

template <typename T, int VB, bool AW>
static hipError_t pick_items(int items, const void* s, const void* q, const void* tab, void* out, long rows, int h,
                             int w, int hd, float scale, unsigned blocks, size_t lds, int bst, hipStream_t st) {
  switch (items) {
    case 1: return launch_vec<T, VB, 1, AW>(s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, st);
    case 2: return launch_vec<T, VB, 2, AW>(s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, st);
    case 4: return launch_vec<T, VB, 4, AW>(s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, st);
    case 8: return launch_vec<T, VB, 8, AW>(s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, st);
    default:
      if constexpr (AW) return launch_vec<T, VB, 16, AW>(s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, st);
      return hipErrorInvalidValue;  // not dispatched: such rows take the scalar kernel
  }
}

template <typename T>
static hipError_t launch_relpos_softmax(const void* s, const void* q, const void* tab, void* out, long rows, int h,
                                        int w, int hd, float scale, hipStream_t stream) {
  const int n = h * w;
  const int bst = (h + w + 3) / 4 * 4 + 4;  // 16-byte rows; consecutive rows 4 banks apart for the scatter
  const long rows_per_block = (long)rsm::kWaves * rsm::kRows;
  const unsigned blocks = (unsigned)((rows + rows_per_block - 1) / rows_per_block);
  const size_t lds = (size_t)rsm::kWaves * rsm::kRows * bst * sizeof(float);
  const long row_bytes = (long)n * (long)sizeof(T);
  const int vb = row_bytes % 16 == 0 ? 16 : (row_bytes % 8 == 0 ? 8 : 0);
  // 16-bit rows of at most 64 vectors whose vectors wrap at most once: 16 lanes per row
  if constexpr (sizeof(T) == 2) {
    if (vb && n / (vb / 2) <= 64 && w >= vb / 2) {
      const int ve = vb / 2, nvec = n / ve;
      const int bq = (w + ve + h + 1 + 3) / 4 * 4 + 4;
      const size_t lq = (size_t)rsm::kWaves * rsm::kRows * bq * sizeof(float);
      const int vpl = nvec <= 16 ? 1 : nvec <= 32 ? 2 : 4;
      auto go = [&](auto kern) {
        static std::atomic<unsigned long long> done{0};
        if (const hipError_t e = lds_opt_in(done, (const void*)kern, (int)lq); e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(rsm::kWaves * 64), lq, stream, (const T*)s, (const T*)q,
                           (const T*)tab, (T*)out, rows, h, w, hd, scale, bq);
        return hipGetLastError();
      };
      if (vb == 16)
        return vpl == 1 ? go(relpos_softmax_quad_kernel<T, 16, 1>)
                        : vpl == 2 ? go(relpos_softmax_quad_kernel<T, 16, 2>) : go(relpos_softmax_quad_kernel<T, 16, 4>);
      return vpl == 1 ? go(relpos_softmax_quad_kernel<T, 8, 1>)
                      : vpl == 2 ? go(relpos_softmax_quad_kernel<T, 8, 2>) : go(relpos_softmax_quad_kernel<T, 8, 4>);
    }
  }
  if (vb) {
    const int ve = vb / (int)sizeof(T);
    const int nvec = n / ve;
    int items = 1;
    while (items * 64 < nvec) items *= 2;
    const bool aw = w % ve == 0 && ve % 4 == 0;  // each vector inside one grid row, whole Rw runs
    // 16 vectors per lane without whole-row vectors would spill: those rows take the scalar kernel
    if (items < 16 || (items == 16 && aw)) {
      if (vb == 16)
        return aw ? pick_items<T, 16, true>(items, s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, stream)
                  : pick_items<T, 16, false>(items, s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, stream);
      if constexpr ((8 / sizeof(T)) % 4 == 0) {
        if (aw) return pick_items<T, 8, true>(items, s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, stream);
      }
      return pick_items<T, 8, false>(items, s, q, tab, out, rows, h, w, hd, scale, blocks, lds, bst, stream);
    }
  }
  auto kern = relpos_softmax_scalar_kernel<T>;
  static std::atomic<unsigned long long> done{0};
  if (const hipError_t e = lds_opt_in(done, (const void*)kern, (int)lds); e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(rsm::kWaves * 64), lds, stream, (const T*)s, (const T*)q,
                     (const T*)tab, (T*)out, rows, h, w, hd, scale, bst);
  return hipGetLastError();
}

// Checked by the caller: rows % (h*w) == 0, h, w <= 128, hd <= 256, 16-byte aligned pointers.
hipError_t relpos_softmax(int dtype, const void* s, const void* q, const void* tab, void* out, long rows, int h, int w,
                          int hd, float scale, hipStream_t stream) {
  if (dtype == kF32) return launch_relpos_softmax<float>(s, q, tab, out, rows, h, w, hd, scale, stream);
  if (dtype == kF16) return launch_relpos_softmax<f16>(s, q, tab, out, rows, h, w, hd, scale, stream);
  return launch_relpos_softmax<bf16>(s, q, tab, out, rows, h, w, hd, scale, stream);
}

}  // namespace samhip
