// Flash attention for head dim 256 on gfx950 (SAM 2.1 memory attention: d_model 256, one head), f16 / bf16.
//
// Same contract and numerics as flash_fwd_kernel (flash_attn.hip): out = softmax(scale q k^T) v per
// (batch, head), the reference's mask-free sdpa / flash_attn (sam3/nn.rs:26-34, sam3/video.rs:129-145),
// exp2-domain online softmax with a lazy rescale, optional RoPE on q, and key splits merged by
// flash_combine_kernel. What differs is the register and staging plan, chosen for d = 256 where the O^T
// accumulators alone take 128 registers per lane:
//
// - One wave per SIMD (4 waves x 32 queries). O^T (128) and the scores S^T (32) live in accumulation
//   registers; Q (64), addresses and the softmax work in arithmetic registers. No C++ arithmetic touches
//   O^T inside the key loop (the rare rescale is done by accumulation-register reads and writes), so the
//   compiler keeps O^T where the MFMAs accumulate it instead of shadowing it in arithmetic registers.
// - K and V tiles (64 keys x 512 bytes) go from global memory straight into LDS by buffer-descriptor
//   DMA (buffer_load_dwordx4 ... lds), so no staging registers are live. The descriptor of a tile ends
//   after the last valid key row, so rows past the end read as zero.
// - The 512-byte rows are stored unpadded (a DMA writes 1 KB contiguously) with the 16-byte chunks of a
//   row permuted by an XOR of the row index: chunk ^ (row & 15) for K (its rows are read 16 bytes per
//   lane, 32 rows at once) and chunk ^ 4 (row & 7) for V (its transpose reads touch 8 rows x 64 bytes).
//   Both read patterns then spread over all banks.
// - Buffers: V0, V1, K0, K1, 32 KB each, so every LDS read is one of 16 per-lane base registers plus an
//   instruction offset.
// - One barrier per tile: step t issues the DMAs of tile t+1 into the buffers that step t-1 finished
//   with, computes S^T = K Q^T, the softmax and O^T += V^T P^T of tile t, then waits for its DMAs.
#include "flash_attn.hpp"
#include "lds_dma.hpp"

namespace samhip {

namespace f256 {
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kRow = 512;                     // bytes per key row (256 x 16-bit)
constexpr int kTileBytes = 64 * kRow;         // 32 KB
constexpr int kV0 = 0, kK0 = 2 * kTileBytes;  // V0, V1, K0, K1
constexpr int kLds = 4 * kTileBytes;          // 128 KB
constexpr float kSlack = 8.0f;
constexpr int kQkAhead = 5;  // k-steps of K fragments in flight ahead of the S^T MFMAs
// Where in a step the four DMA groups of the next tile (K rows 0-7, K 8-15, V 0-7, V 8-15 of each
// wave's share) are issued: 0 top of the step, 1 after S^T, 2 after the softmax, 3 halfway through P.V,
// 4 inside S^T right after its first K reads.
constexpr int kDmaAt[4] = {0, 0, 1, 1};
}  // namespace f256

// Workgroup i runs on XCD i % 8; give each XCD a contiguous range of the linear work index.
__device__ __forceinline__ int f256_xcd_block(int i, int total) {
  const int per = total >> 3, rem = total & 7, x = i & 7, j = i >> 3;
  return x * per + (x < rem ? x : rem) + j;
}

__device__ __forceinline__ void f256_rope_pair(float x0, float x1, float c0, float s0, float c1, float s1, float& y0,
                                               float& y1) {
#pragma clang fp contract(off)
  y0 = x0 * c0 + -x1 * s0;
  y1 = x1 * c1 + x0 * s1;
}

// o[ob] *= alpha, element by element in accumulation registers. The leading s_nops cover the
// MFMA-result-to-read latency (at most 19 wait states), the trailing one the write-to-MFMA-source latency.
__device__ __forceinline__ void f256_rescale(f32x16* o, float alpha) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int ob = 0; ob < 8; ++ob)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float tmp;
      asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                   : "+a"(o[ob][e]), "=&v"(tmp)
                   : "v"(alpha));
    }
  asm volatile("s_nop 4" ::: "memory");
}

template <typename T, bool ROPEQ>
__global__ __launch_bounds__(f256::kThreads) void flash256_kernel(FlashParams p) {
  using namespace f256;
  typedef typename Vec<T>::x8 X8;
  typedef __attribute__((address_space(3))) X8 lds_x8;
  constexpr bool kSplitP = __is_same(T, bf16);
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const unsigned lds0 = lds_addr(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, hh = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;

  const int lin = f256_xcd_block(blockIdx.x, gridDim.x);
  const int qb = lin % p.qblocks;
  const int split = (lin / p.qblocks) % p.nsplit;
  const int bhi = lin / (p.qblocks * p.nsplit);
  const int bi = bhi / p.h, head = bhi % p.h;

  const int q0 = qb * (kWaves * 32) + wave * 32;
  const bool active = q0 < p.lq;
  const int qidx = q0 + n;
  const bool qvalid = qidx < p.lq;

  const int t_begin = split * p.tps;
  const int t_end = min((p.lk + 63) >> 6, t_begin + p.tps);
  const int kend = p.lk;

  const T* qbase = reinterpret_cast<const T*>(p.q) + bi * p.sq[0] + head * p.sq[2];
  const T* kbase = reinterpret_cast<const T*>(p.k) + bi * p.sk[0] + head * p.sk[2];
  const T* vbase = reinterpret_cast<const T*>(p.v) + bi * p.sv[0] + head * p.sv[2];
  const long krow = p.sk[1] * (long)sizeof(T), vrow = p.sv[1] * (long)sizeof(T);  // row strides, bytes

  // ---- DMA of one tile: 32 blocks of 1 KB (two key rows each); wave w moves rows 16w .. 16w+15.
  // Block j of the wave holds rows 16w + 2j + hh; lane slot n of a row holds the row's chunk n ^ swz(row).
  // The wave's LDS base is re-derived per call (opaque), so the 16 per-block LDS addresses are formed
  // next to their DMAs instead of being held in scalar registers across the loop.
  auto dma_tile = [&](const T* base, long rowb, int t, unsigned lds_tile, bool is_k, int j0, int j1) {
    const long r0 = (long)t * 64;
    const unsigned bytes = (unsigned)min((kend - 1 - r0) * rowb + kRow, 0xffffffffL);  // through the last valid row
    const i32x4 rs = buffer_rsrc(reinterpret_cast<const char*>(base) + r0 * rowb, bytes);
    unsigned lb = lds_tile + 16 * wave * kRow;
    asm volatile("" : "+s"(lb));
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      const int row = 16 * wave + 2 * j + hh;
      const int swz = is_k ? ((2 * j + hh) & 15) : 4 * ((2 * j + hh) & 7);
      const unsigned off = (unsigned)(row * rowb) + 16u * (unsigned)(n ^ swz);
      bdma16(rs, off, lb + 2 * j * kRow);
    }
  };
  // part i (0..3) of the DMAs of tile t into buffers buf: half i & 1 of K (i < 2) or of V (i >= 2)
  auto dma_part = [&](int t, int buf, int i) {
    const int j0 = 4 * (i & 1);
    if (i < 2) dma_tile(kbase, krow, t, lds0 + kK0 + buf * kTileBytes, true, j0, j0 + 4);
    else dma_tile(vbase, vrow, t, lds0 + kV0 + buf * kTileBytes, false, j0, j0 + 4);
  };

#pragma unroll
  for (int i = 0; i < 4; ++i) dma_part(t_begin, 0, i);

  // Q fragments (B operand of S^T = K Q^T): lane supplies Q[query n][16*s + 8*hh + j], j = 0..7
  X8 qf[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const int c = 16 * s + 8 * hh;
    X8 val = X8{};
    if (qvalid) {
      val = __builtin_bit_cast(X8, *reinterpret_cast<const u32x4*>(qbase + (long)qidx * p.sq[1] + c));
      if (ROPEQ && qidx < p.nrq) {
        const long tr = (long)(qidx % p.rrows) * 256 + c;
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(p.rcos + tr);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(p.rcos + tr + 4);
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(p.rsin + tr);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(p.rsin + tr + 4);
        const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
        const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; j += 2)
          f256_rope_pair(to_f32(val[j]), to_f32(val[j + 1]), cs[j], sn[j], cs[j + 1], sn[j + 1], y[j], y[j + 1]);
        val = pack8(y, (X8*)nullptr);
      }
    }
    qf[s] = val;
  }

  // ---- per-lane LDS read addresses
  // K (A operand of S^T): row r = 32 mb + n, chunk 2k + hh, stored at chunk slot (2k + hh) ^ (n & 15)
  //   = ((hh ^ n) & 1) + 2 ((k & 7) ^ ((n >> 1) & 7)) + 16 (k >> 3).
  unsigned kad[8];
#pragma unroll
  for (int k7 = 0; k7 < 8; ++k7)
    kad[k7] = opaque(lds0 + kK0 + n * kRow + 16 * ((hh ^ n) & 1) + 32 * (k7 ^ ((n >> 1) & 7)));
  // V^T (A operand of O^T), transpose reads: source lane (4 s + c) of group g reads key row
  // R0 + z (z = 4 (g >> 1) + s, R0 a multiple of 8) at columns 32 ob + 16 (g & 1) + 4 c .. +3; with the
  // chunk swizzle the byte address is (R0 + z) 512 + 64 (ob ^ z) + 32 (g & 1) + 8 c.
  unsigned vad[8];
  {
    const int z = 4 * (g >> 1) + (gi >> 2);
#pragma unroll
    for (int ob = 0; ob < 8; ++ob)
      vad[ob] = opaque(lds0 + kV0 + z * kRow + 64 * (ob ^ z) + 32 * (g & 1) + 8 * (gi & 3));
  }

  // S^T = K(buffer buf) Q^T. K fragments are read kQkAhead k-steps ahead of their MFMAs; the scheduling
  // groups keep that order (the compiler otherwise issues half of the reads right before their MFMAs).
  auto qk = [&](int buf, f32x16* s, auto&& after_first_reads) {
    __builtin_amdgcn_sched_barrier(0);
    auto kread = [&](int k, int mb) {
      return *(const lds_x8*)(size_t)(kad[k & 7] + buf * kTileBytes + mb * 32 * kRow + 256 * (k >> 3));
    };
    constexpr int R = kQkAhead + 1;
    X8 kf[R][2];
#pragma unroll
    for (int k = 0; k < kQkAhead; ++k) {
      kf[k][0] = kread(k, 0);
      kf[k][1] = kread(k, 1);
    }
    after_first_reads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k + kQkAhead < 16) {
        kf[(k + kQkAhead) % R][0] = kread(k + kQkAhead, 0);
        kf[(k + kQkAhead) % R][1] = kread(k + kQkAhead, 1);
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) s[mb] = mma32(kf[k % R][mb], qf[k], k == 0 ? f32x16{} : s[mb]);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kQkAhead, 0);  // LDS reads of the first k-steps
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k + kQkAhead < 16) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // reads of k-step k + ahead
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);                         // MFMAs of k-step k
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // scaled row max of tile t (log2 units), the keys past the end set to -inf first
  auto tile_max = [&](int t, f32x16* s) {
    if ((t << 6) + 64 > kend) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if ((t << 6) + 32 * mb + 8 * (e >> 2) + 4 * hh + (e & 3) >= kend) s[mb][e] = -INFINITY;
    }
    float mm = s[0][0];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mm = fmaxf(mm, s[mb][e]);
    return max_with_partner32(mm * p.sc);
  };

  float m_run = -INFINITY, l_run = 0.f;
  // O^T starts as an MFMA on zero operands, so that every definition of it is an accumulation register
  f32x16 o[8];
#pragma unroll
  for (int ob = 0; ob < 8; ++ob) o[ob] = mma32(X8{}, X8{}, f32x16{});

  // Step of tile t, whose K and V are in buffers buf.
  auto step = [&](int t, int buf) {
    // tile t+1 into the other buffers, released by the barrier that ended the previous step; its 16
    // DMAs per wave go out in four groups spread over the step, since a burst of them stalls the wave
    const bool more = t + 1 < t_end;
    auto dma_at = [&](int point) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (kDmaAt[i] == point && more) dma_part(t + 1, buf ^ 1, i);
    };
    dma_at(0);
    f32x16 s[2];
    qk(buf, s, [&] { dma_at(4); });
    dma_at(1);
    X8 b[4], blo[4];
    {
      const float mt = tile_max(t, s);
      if (wave_any(mt > m_run + kSlack)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = exp2_fast(m_run - m_new);
        l_run *= alpha;
        f256_rescale(o, alpha);
        m_run = m_new;
      }
      const float c = -m_run;
      float lsum = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pv[j] = exp2_fast(fmaf(s[u >> 1][8 * (u & 1) + j], p.sc, c));
          lsum += pv[j];
        }
        b[u] = pack8(pv, (X8*)nullptr);
        if (kSplitP) {
#pragma unroll
          for (int j = 0; j < 8; ++j) pv[j] -= to_f32(b[u][j]);
          blo[u] = pack8(pv, (X8*)nullptr);
        }
      }
      l_run += lsum;
    }
    dma_at(2);
    // O^T += V^T . P^T over the tile's 4 groups of 16 keys; in bf16, P is split into hi + lo terms
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u == 2) dma_at(3);
#pragma unroll
      for (int ob = 0; ob < 8; ++ob) {
        const unsigned r0 = buf * kTileBytes + (32 * (u >> 1) + 16 * (u & 1)) * kRow;
        const X8 a = join8<T>(lds_read_tr16_at(vad[ob] + r0), lds_read_tr16_at(vad[ob] + r0 + 8 * kRow));
        o[ob] = mma32(a, b[u], o[ob]);
        if (kSplitP) o[ob] = mma32(a, blo[u], o[ob]);
      }
    }
    wait_vm<0>();
    __syncthreads();
  };

  // All of this wave's loads (tile t0, Q, RoPE tables) done. A compiler-visible wait, so that the
  // compiler's own load tracking does not carry the Q loads into the loop.
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  for (int t = t_begin; t < t_end; t += 2) {
    step(t, 0);
    if (t + 1 < t_end) step(t + 1, 1);
  }

  if (!active) return;
  // lane holds O^T[32*ob + 8*a + 4*hh + b][query n]
  const float l = sum_with_partner32(l_run);
  if (!qvalid) return;
  if (p.nsplit == 1) {
    const float inv = 1.f / l;
    T* orow = reinterpret_cast<T*>(p.out) + bi * p.so[0] + head * p.so[2] + (long)qidx * p.so[1];
#pragma unroll
    for (int ob = 0; ob < 8; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int d0 = 32 * ob + 8 * a + 4 * hh;
        typename Vec<T>::x4 w4;
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) w4[bb] = from_f32<T>(o[ob][4 * a + bb] * inv);
        *reinterpret_cast<typename Vec<T>::x4*>(orow + d0) = w4;
      }
  } else {
    // partial O [split][bh][q][256] and (max, sum) [split][bh][q][2]: f16 stores O / sum (a convex
    // combination of f16 values of v, so it stays in range), bf16 the unnormalised O in f32
    const long row = ((long)split * p.b * p.h + bhi) * p.lq + qidx;
    if constexpr (__is_same(T, f16)) {
      const float inv = 1.f / l;
      f16* prow = reinterpret_cast<f16*>(p.opart) + row * 256;
#pragma unroll
      for (int ob = 0; ob < 8; ++ob)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d0 = 32 * ob + 8 * a + 4 * hh;
          Vec<f16>::x4 w4;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) w4[bb] = (f16)(o[ob][4 * a + bb] * inv);
          *reinterpret_cast<Vec<f16>::x4*>(prow + d0) = w4;
        }
    } else {
      float* prow = p.opart + row * 256;
#pragma unroll
      for (int ob = 0; ob < 8; ++ob)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int d0 = 32 * ob + 8 * a + 4 * hh;
          f32x4 w4;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) w4[bb] = o[ob][4 * a + bb];
          *reinterpret_cast<f32x4*>(prow + d0) = w4;
        }
    }
    if (hh == 0) {
      float2 ml;
      ml.x = m_run;
      ml.y = l;
      *reinterpret_cast<float2*>(p.ml + row * 2) = ml;
    }
  }
}

// True when flash256_kernel takes this problem: head dim exactly 256 and per-tile byte offsets of K and
// V (64 rows) inside the 32-bit range of a buffer descriptor.
bool flash256_eligible(const FlashParams& p, int elem_bytes) {
  const long lim = 1L << 30;
  return p.d == 256 && p.sk[1] >= 0 && p.sv[1] >= 0 && 64L * p.sk[1] * elem_bytes < lim &&
         64L * p.sv[1] * elem_bytes < lim;
}

template <typename T>
static hipError_t launch256(FlashParams p, bool ropeq, hipStream_t stream) {
  auto kern = ropeq ? flash256_kernel<T, true> : flash256_kernel<T, false>;
  static std::atomic<unsigned long long> lds_done[2];  // opt-in to more than 64 KB of dynamic LDS
  if (const hipError_t e = lds_opt_in(lds_done[ropeq], (const void*)kern, f256::kLds); e != hipSuccess) return e;
  const long blocks = (long)p.b * p.h * p.qblocks * p.nsplit;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(f256::kThreads), f256::kLds, stream, p);
  return hipGetLastError();
}

hipError_t flash256_launch(int dtype, FlashParams p, bool ropeq, hipStream_t stream) {
  if (dtype == kF16) return launch256<f16>(p, ropeq, stream);
  return launch256<bf16>(p, ropeq, stream);
}

}  // namespace samhip
