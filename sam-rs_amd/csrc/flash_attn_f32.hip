// Flash attention in f32 for gfx950: out = softmax(scale * q k^T [+ mask]) v per (batch, head).
//
// The f32 counterpart of flash_fwd_kernel (flash_attn.hip) for the reference's f32 GPU path: with
// `--dtype f32` on a GPU every attention of the reference runs as sam3::nn::sdpa (sam3/nn.rs:26-34),
// candle's f32 matmul, softmax_last_dim and matmul (the flash back ends take f16/bf16 only,
// sam3/nn.rs:65-71). Held to 1e-5 relative of the reference's exact f32 result, so the arithmetic
// follows it: logits (q . k) * scale [+ mask] in natural units, accurate expf, P and O in f32.
//
// Same decomposition as the 16-bit kernels: S^T = K . Q^T and O^T = V^T . P^T on
// v_mfma_f32_32x32x2_f32, one query per lane (lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32];
// it receives D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32] in element i).
//   * S^T: k-step s covers head-dim columns s and DP/2 + s (lanes of half 0 and 1), so a lane's Q
//     operands are a contiguous half row (DP/2 registers) and its K operands come from one K row by
//     16-byte LDS reads (4 k-steps each).
//   * O^T: k-step j takes keys 8 (j / 4) + (j % 4) (half 0) and that + 4 (half 1), the keys a lane
//     of either half holds in its S^T element j, so P is element j itself. V is stored transposed in
//     LDS ([head dim][32 keys]), so a lane's V operands of 4 k-steps are one 16-byte read.
// Key tiles of 32 are staged through registers (the next tile's loads in flight during the current
// tile), one LDS buffer, two barriers per tile. Optional RoPE on the queries is applied as Q is loaded
// (f32, the reference's rounding); rotated keys come from rope_rows beforehand. Key splits write f32
// partials (unnormalised O, max in log2 units, sum) for flash_combine_kernel.
#include "flash_attn.hpp"

namespace samhip {

namespace ff32 {
constexpr float kSlack = 5.5451774f;  // 8 ln 2: P <= 256 between rescales
constexpr float kLog2e = 1.4426950408889634f;

template <int DP> struct Geom {
  static constexpr int NW = DP <= 128 ? 8 : 4;  // the query blocks of flash_queries_per_block
  static constexpr int NT = NW * 64;
  static constexpr int HALF = DP / 2;
  static constexpr int MBO = DP / 32;           // 32-row blocks of O^T
  static constexpr int KSTR = DP + 4;           // floats per K row in LDS (rows 16 bytes apart mod 256)
  static constexpr int VSTR = 36;               // floats per V^T row (32 keys + 4: 9 16-byte units)
  static constexpr int KFL = 32 * KSTR;         // K tile floats
  static constexpr size_t LDS = (size_t)(KFL + DP * VSTR) * sizeof(float);
  static constexpr int CH = 32 * DP / 4;        // 16-byte chunks of a 32-key tile (K or V)
  static constexpr int PT = (CH + NT - 1) / NT; // chunks per thread
};
}  // namespace ff32

__device__ __forceinline__ f32x16 mma32f(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Two rotated pairs with the reference's rounding: (x0 c0 + (-x1) s0, x1 c1 + x0 s1), no contraction.
__device__ __forceinline__ f32x4 ff32_rope4(f32x4 x, f32x4 cs, f32x4 sn) {
#pragma clang fp contract(off)
  const float y0 = x[0] * cs[0] + -x[1] * sn[0], y1 = x[1] * cs[1] + x[0] * sn[1];
  const float y2 = x[2] * cs[2] + -x[3] * sn[2], y3 = x[3] * cs[3] + x[2] * sn[3];
  return f32x4{y0, y1, y2, y3};
}

__device__ __forceinline__ int ff32_xcd_block(int i, int total) {
  const int per = total >> 3, rem = total & 7, x = i & 7, j = i >> 3;
  return x * per + (x < rem ? x : rem) + j;
}

template <int DP, bool ROPEQ, bool MASK>
__global__ __launch_bounds__(ff32::Geom<DP>::NT) void flash_f32_kernel(FlashParams p) {
  using namespace ff32;
  typedef Geom<DP> G;
  constexpr int NW = G::NW, NT = G::NT, HALF = G::HALF, MBO = G::MBO, KSTR = G::KSTR, VSTR = G::VSTR;
  constexpr int CH = G::CH, PT = G::PT;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* ks = reinterpret_cast<float*>(smem);
  float* vts = ks + G::KFL;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hh = lane >> 5;

  const int lin = ff32_xcd_block(blockIdx.x, gridDim.x);
  const int qb = lin % p.qblocks;
  const int split = (lin / p.qblocks) % p.nsplit;
  const int bhi = lin / (p.qblocks * p.nsplit);
  const int bi = bhi / p.h, head = bhi % p.h;
  const int d = p.d;

  const int q0 = qb * (NW * 32) + wave * 32;
  const bool active = q0 < p.lq;
  const int qidx = q0 + n;
  const bool qvalid = qidx < p.lq;

  // this split's keys, in tiles of 32 (the plan counts tiles of 64)
  const int k_begin = split * p.tps * 64;
  const int k_end = min(p.lk, k_begin + p.tps * 64);
  const int kend = p.lk;

  const float* qbase = reinterpret_cast<const float*>(p.q) + bi * p.sq[0] + head * p.sq[2];
  const float* kbase = reinterpret_cast<const float*>(p.k) + bi * p.sk[0] + head * p.sk[2];
  const float* vbase = reinterpret_cast<const float*>(p.v) + bi * p.sv[0] + head * p.sv[2];

  // ---- staging of a 32-key tile: chunk c = key (c / (DP/4)), columns 4 (c % (DP/4)) .. +3; keys past
  // the end and columns past d are zero
  f32x4 kreg[PT], vreg[PT];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      const int r = c / (DP / 4), c4 = (c % (DP / 4)) * 4;
      const int key = k0 + r;
      const bool ok = (CH % NT == 0 || c < CH) && key < kend && c4 < d;
      kreg[u] = ok ? *reinterpret_cast<const f32x4*>(kbase + (long)key * p.sk[1] + c4) : f32x4{0.f, 0.f, 0.f, 0.f};
      vreg[u] = ok ? *reinterpret_cast<const f32x4*>(vbase + (long)key * p.sv[1] + c4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int u = 0; u < PT; ++u) {
      const int c = tid + u * NT;
      if (CH % NT == 0 || c < CH) {
        const int r = c / (DP / 4), c4 = (c % (DP / 4)) * 4;
        *reinterpret_cast<f32x4*>(ks + r * KSTR + c4) = kreg[u];
#pragma unroll
        for (int e = 0; e < 4; ++e) vts[(c4 + e) * VSTR + r] = vreg[u][e];
      }
    }
  };

  load_tile(k_begin);

  // Q operands: lane supplies Q[query n][HALF hh + s] for k-step s (a contiguous half row), rotated as
  // the reference's rope does when asked
  float qf[HALF];
  {
    const float* qrow = qbase + (long)(qvalid ? qidx : 0) * p.sq[1] + HALF * hh;
#pragma unroll
    for (int s4 = 0; s4 < HALF; s4 += 4) {
      f32x4 x = f32x4{0.f, 0.f, 0.f, 0.f};
      if (qvalid && HALF * hh + s4 < d) x = *reinterpret_cast<const f32x4*>(qrow + s4);
      if (ROPEQ && qvalid && qidx < p.nrq && HALF * hh + s4 < d) {
        const long tr = (long)(qidx % p.rrows) * d + HALF * hh + s4;
        x = ff32_rope4(x, *reinterpret_cast<const f32x4*>(p.rcos + tr), *reinterpret_cast<const f32x4*>(p.rsin + tr));
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) qf[s4 + e] = x[e];
    }
  }

  store_tile();
  __syncthreads();

  const float scale = p.fscale;
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[MBO];
#pragma unroll
  for (int ob = 0; ob < MBO; ++ob) o[ob] = f32x16{};
  const float* mrow = nullptr;
  if constexpr (MASK)
    mrow = reinterpret_cast<const float*>(p.mask) + bi * p.sm[0] + head * p.sm[1] + (long)(qvalid ? qidx : 0) * p.sm[2];

  for (int k0 = k_begin; k0 < k_end; k0 += 32) {
    const bool more = k0 + 32 < k_end;
    if (more) load_tile(k0 + 32);  // in flight while tile k0 is computed
    if (active) {
      // S^T: lane holds key k0 + 8 (i / 4) + 4 hh + (i % 4) for query n in s[i]
      f32x16 s = f32x16{};
      const float* krow = ks + n * KSTR + HALF * hh;
#pragma unroll
      for (int s4 = 0; s4 < HALF; s4 += 4) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(krow + s4);
#pragma unroll
        for (int e = 0; e < 4; ++e) s = mma32f(kv[e], qf[s4 + e], s);
      }
      // logits in natural units as the reference forms them: (q . k) * scale, then + mask
      float mm = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = k0 + 8 * (i >> 2) + 4 * hh + (i & 3);
        float x = s[i] * scale;
        if constexpr (MASK) x = key < kend ? x + mrow[(long)key * p.sm[3]] : x;
        s[i] = key < kend ? x : -INFINITY;
        mm = fmaxf(mm, s[i]);
      }
      const float mt = max_with_partner32(mm);
      if (wave_any(mt > m_run + kSlack)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int ob = 0; ob < MBO; ++ob) o[ob] *= alpha;
        m_run = m_new;
      }
      // with a mask a tile (the first ones included) can be all -inf while m_run is still -inf
      const float c = m_run == -INFINITY ? 0.f : m_run;
      float lsum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[i] = expf(s[i] - c);
        lsum += s[i];
      }
      l_run += lsum;
      // O^T += V^T . P^T: k-step j = 4 jg + e takes the keys of S^T element j in both halves
#pragma unroll
      for (int ob = 0; ob < MBO; ++ob) {
        const float* vrow = vts + (32 * ob + n) * VSTR + 4 * hh;
#pragma unroll
        for (int jg = 0; jg < 4; ++jg) {
          const f32x4 vv = *reinterpret_cast<const f32x4*>(vrow + 8 * jg);
#pragma unroll
          for (int e = 0; e < 4; ++e) o[ob] = mma32f(vv[e], s[4 * jg + e], o[ob]);
        }
      }
    }
    __syncthreads();  // every wave is done with the tile in LDS
    if (more) {
      store_tile();
      __syncthreads();
    }
  }

  if (!active) return;
  // lane holds O^T[32 ob + 8 a + 4 hh + bb][query n] in o[ob][4 a + bb]
  const float l = sum_with_partner32(l_run);
  if (!qvalid) return;
  if (p.nsplit == 1) {
    const float inv = 1.f / l;
    float* orow = reinterpret_cast<float*>(p.out) + bi * p.so[0] + head * p.so[2] + (long)qidx * p.so[1];
#pragma unroll
    for (int ob = 0; ob < MBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * ob + 8 * a + 4 * hh;
        if (d0 < d) {
          f32x4 w4;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) w4[bb] = o[ob][4 * a + bb] * inv;
          *reinterpret_cast<f32x4*>(orow + d0) = w4;
        }
      }
  } else {
    // partial O [split][bh][q][DP] (unnormalised) and (max in log2 units, sum) [split][bh][q][2]
    const long row = ((long)split * p.b * p.h + bhi) * p.lq + qidx;
    float* prow = p.opart + row * DP;
#pragma unroll
    for (int ob = 0; ob < MBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        f32x4 w4;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) w4[bb] = o[ob][4 * a + bb];
        *reinterpret_cast<f32x4*>(prow + 32 * ob + 8 * a + 4 * hh) = w4;
      }
    if (hh == 0) {
      float2 ml;
      ml.x = m_run * kLog2e;
      ml.y = l;
      *reinterpret_cast<float2*>(p.ml + row * 2) = ml;
    }
  }
}

template <int DP>
static hipError_t launch_f32(FlashParams p, bool ropeq, hipStream_t stream) {
  typedef ff32::Geom<DP> G;
  const int which = p.mask ? 2 : ropeq ? 1 : 0;  // a masked call has no RoPE
  auto kern = which == 2   ? flash_f32_kernel<DP, false, true>
              : which == 1 ? flash_f32_kernel<DP, true, false>
                           : flash_f32_kernel<DP, false, false>;
  static std::atomic<unsigned long long> lds_done[3];
  if (const hipError_t e = lds_opt_in(lds_done[which], (const void*)kern, (int)G::LDS); e != hipSuccess) return e;
  const long blocks = (long)p.b * p.h * p.qblocks * p.nsplit;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(G::NT), G::LDS, stream, p);
  if (const hipError_t e = hipGetLastError(); e != hipSuccess || p.nsplit == 1) return e;
  return flash_combine_f32(p, DP, stream);
}

hipError_t flash_attn_f32(FlashParams p, bool ropeq, hipStream_t stream) {
  switch (flash_padded_dim(p.d)) {
    case 32: return launch_f32<32>(p, ropeq, stream);
    case 64: return launch_f32<64>(p, ropeq, stream);
    case 96: return launch_f32<96>(p, ropeq, stream);
    case 128: return launch_f32<128>(p, ropeq, stream);
    default: return launch_f32<256>(p, ropeq, stream);
  }
}

}  // namespace samhip
