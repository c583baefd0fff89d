// Flash attention for head dim 256 on gfx950 (SAM 2.1 memory attention: d_model 256, one head), f16 / bf16.
//
// Same contract and numerics as flash_fwd_kernel (flash_attn.hip): out = softmax(scale q k^T) v per
// (batch, head), the reference's mask-free sdpa / flash_attn (sam3/nn.rs:26-34, sam3/video.rs:129-145),
// exp2-domain online softmax with a lazy rescale, optional RoPE on q, and key splits merged by
// flash_combine_kernel. What differs is the register and LDS plan, chosen for d = 256, where a wave of
// 32 queries needs 128 registers per lane for O^T alone and so runs alone on its SIMD:
//
// - Two waves per SIMD (8 waves x 16 queries, 128 queries per workgroup, the query block of the other
//   kernels). A wave holds S^T (16 registers), O^T (64) and its Q fragments (32) for
//   v_mfma_f32_16x16x32; with about half the register file per wave, one wave's LDS and MFMA latency
//   is covered by the other's work.
// - Every LDS read is a 16-byte ds_read_b128 whose row is the MFMA's reduction dimension. K rows
//   (key-major, d contiguous) already are. V is not: a pass before the kernel writes each 64-key tile
//   of V as V^T, 256 rows of 64 keys, in the exact byte image the kernel wants in LDS (flash_vt.hpp),
//   so the tile moves by plain 1 KB DMAs. The pass rides in the launch that rotates the keys when
//   there is one, else it is a launch of its own. Against transpose reads (ds_read_b64_tr_b16, 8
//   bytes per lane) this halves the LDS read instructions of P.V, which with 16 queries per wave
//   would otherwise bound the kernel.
// - K and V^T tiles (32 KB each) go from global memory straight into LDS by DMA (buffer_load_dwordx4
//   ... lds / global_load_lds_dwordx4), double-buffered: K0, K1, V0, V1 = 128 KB, one workgroup per
//   CU. The K descriptor of a tile ends after the last valid key row, so rows past the end read as 0.
// - Bank layout: K rows are 512 bytes; 16-byte chunk c of row r is stored at c ^ (r & 15), so the 16
//   rows at one chunk that a quarter wave reads fall on 16 distinct 16-byte bank groups. V^T rows are
//   128 bytes; chunk q of row r at q ^ ((r >> 1) & 7) does the same.
// - One barrier per tile: step t issues the DMAs of tile t+1 into the buffers that step t-1 finished
//   with, computes S^T = K Q^T, the softmax and O^T += V^T P^T of tile t, then waits for its DMAs.
#include "flash_attn.hpp"
#include "flash_vt.hpp"
#include "lds_dma.hpp"

namespace samhip {

namespace f256 {
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kQ = 16;                        // queries per wave
constexpr int kRow = 512;                     // bytes per K row (256 x 16-bit)
constexpr int kVRow = 128;                    // bytes per V^T row (64 keys x 16-bit)
constexpr int kTileBytes = 64 * kRow;         // 32 KB: a K tile, or a V^T tile (256 rows)
constexpr int kK0 = 0, kV0 = 2 * kTileBytes;  // K0, K1, V0, V1
constexpr int kLds = 4 * kTileBytes;          // 128 KB
constexpr float kSlack = 8.0f;
constexpr int kAhead = 8;  // LDS fragments in flight ahead of their MFMAs
static_assert(kWaves * kQ == 128, "the query block of flash_queries_per_block(256)");

static_assert(kTileBytes == vtl::kTileBytes, "V^T tile size");
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

// The V^T tile pass as a launch of its own (calls whose keys are not rotated).
__global__ __launch_bounds__(256) void flash256_vt_kernel(VtJob j) { flash256_vt_quarter(j, blockIdx.x); }

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
  const int n = lane & 15, g = lane >> 4;     // MFMA column (query of the wave) and row group
  const int n32 = lane & 31, hh = lane >> 5;  // DMA: 16-byte slot of a 512-byte row, and which row

  const int lin = f256_xcd_block(blockIdx.x, gridDim.x);
  const int qb = lin % p.qblocks;
  const int split = (lin / p.qblocks) % p.nsplit;
  const int bhi = lin / (p.qblocks * p.nsplit);
  const int bi = bhi / p.h, head = bhi % p.h;

  const int q0 = qb * (kWaves * kQ) + wave * kQ;
  const bool active = q0 < p.lq;
  const int qidx = q0 + n;
  const bool qvalid = qidx < p.lq;

  const int ntiles = (p.lk + 63) >> 6;
  const int t_begin = split * p.tps;
  const int t_end = min(ntiles, t_begin + p.tps);
  const int kend = p.lk;

  const T* qbase = reinterpret_cast<const T*>(p.q) + bi * p.sq[0] + head * p.sq[2];
  const T* kbase = reinterpret_cast<const T*>(p.k) + bi * p.sk[0] + head * p.sk[2];
  const char* vtbase = reinterpret_cast<const char*>(p.vt) + (size_t)bhi * ntiles * kTileBytes;
  const long krow = p.sk[1] * (long)sizeof(T);  // K row stride, bytes

  // K tile t into buffer buf: wave w moves rows 8w .. 8w+7 as 4 blocks of 1 KB (block j: rows
  // 8w + 2j + hh); lane slot n32 of a row holds the row's chunk n32 ^ (row & 15)
  auto dma_k = [&](int t, int buf) {
    const long r0 = (long)t * 64;
    const unsigned bytes = (unsigned)min((kend - 1 - r0) * krow + kRow, 0xffffffffL);  // through the last valid row
    const i32x4 rs = buffer_rsrc(reinterpret_cast<const char*>(kbase) + r0 * krow, bytes);
    unsigned lb = lds0 + kK0 + buf * kTileBytes + 8 * wave * kRow;
    asm volatile("" : "+s"(lb));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 8 * wave + 2 * j + hh;
      bdma16(rs, (unsigned)(row * krow) + 16u * (unsigned)(n32 ^ (row & 15)), lb + 2 * j * kRow);
    }
  };
  // V^T tile t into buffer buf: the tile is stored as its LDS image; wave w moves bytes [4 KB w, +4 KB)
  auto dma_v = [&](int t, int buf) {
    const char* src = vtbase + (size_t)t * kTileBytes + 4096 * wave;
    unsigned lb = lds0 + kV0 + buf * kTileBytes + 4096 * wave;
    asm volatile("" : "+s"(lb));
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16(src, (unsigned)(1024 * j + 16 * lane), lb + 1024 * j);
  };

  dma_k(t_begin, 0);
  dma_v(t_begin, 0);

  // Q fragments (B operand of S^T = K Q^T): lane supplies Q[query n][32 ks + 8 g + j], j = 0..7
  X8 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const int c = 32 * ks + 8 * g;
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
    qf[ks] = val;
  }

  // ---- per-lane LDS read addresses; buffers, blocks and k-steps are instruction offsets (< 64 KB)
  // K (A operand of S^T): block kb reads row 16 kb + n at chunk 4 ks + g, stored at (4 ks + g) ^ n =
  // 16 (ks >> 2) + 4 ((ks & 3) ^ (n >> 2)) + (g ^ (n & 3)).
  unsigned kad[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) kad[j] = opaque(lds0 + kK0 + n * kRow + 64 * (j ^ (n >> 2)) + 16 * (g ^ (n & 3)));
  auto kread = [&](int buf, int kb, int ks) {
    return *(const lds_x8*)(size_t)(kad[ks & 3] + buf * kTileBytes + kb * 16 * kRow + 256 * (ks >> 2));
  };
  // V^T (A operand of O^T): block db reads row 16 db + n at chunk 4 u + g (keys vtl::vt_key(4 u + g, j))
  unsigned vad[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) vad[u] = opaque(lds0 + kV0 + n * kVRow + 16 * vtl::vt_pos(4 * u + g, n));
  auto vread = [&](int buf, int db, int u) {
    return *(const lds_x8*)(size_t)(vad[u] + buf * kTileBytes + db * 16 * kVRow);
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[16];
#pragma unroll
  for (int db = 0; db < 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Step of tile t, whose K and V^T are in buffers buf.
  auto step = [&](int t, int buf) {
    if (t + 1 < t_end) {  // tile t+1 into the other buffers, released by the barrier that ended step t-1
      dma_k(t + 1, buf ^ 1);
      dma_v(t + 1, buf ^ 1);
    }
    if (active) {
      // S^T: lane holds key 16 kb + 4 g + i of the tile for query n in s[kb][i]. MFMA i (k-step i / 4,
      // block i % 4) reads its K fragment kAhead MFMAs earlier; the scheduling groups hold that order
      // (left alone, the compiler issues each read right before its MFMA and waits for it).
      f32x4 s[4];
      {
        __builtin_amdgcn_sched_barrier(0);
        X8 kf[32];
#pragma unroll
        for (int i = 0; i < kAhead; ++i) kf[i] = kread(buf, i & 3, i >> 2);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int kb = i & 3, ks = i >> 2;
          s[kb] = mma16(kf[i], qf[ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[kb]);
          if (i + kAhead < 32) kf[i + kAhead] = kread(buf, (i + kAhead) & 3, (i + kAhead) >> 2);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (i + kAhead < 32) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // the first V^T fragments of P.V, read while the softmax runs
      X8 vf[32];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) vf[i] = vread(buf, i & 15, i >> 4);
      if ((t << 6) + 64 > kend) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if ((t << 6) + 16 * kb + 4 * g + i >= kend) s[kb][i] = -INFINITY;
      }
      float mm = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) mm = max_nc(mm, s[kb][i]);
      const float mt = max_over_rows16(mm) * p.sc;
      if (wave_any(mt > m_run + kSlack)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = exp2_fast(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 16; ++db) o[db] *= alpha;
        m_run = m_new;
      }
      // P, and its sum as the P.V product sees it: f16 sums the rounded P (v_dot2), so that the weights
      // of the numerator and of the denominator are the same numbers; bf16 (P as hi + lo) the f32 P
      const float c = -m_run;
      X8 b[2], blo[2];
      float lsum = 0.f;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = exp2_fast(fmaf(s[2 * u + (j >> 2)][j & 3], p.sc, c));
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
      // O^T += V^T . P^T (MFMA i: block i % 16, fragment u = i / 16), each V^T fragment read kAhead
      // MFMAs earlier; in bf16, P is split into hi + lo terms
      {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int db = i & 15, u = i >> 4;
          o[db] = mma16(vf[i], b[u], o[db]);
          if (kSplitP) o[db] = mma16(vf[i], blo[u], o[db]);
          if (i + kAhead < 32) vf[i + kAhead] = vread(buf, (i + kAhead) & 15, (i + kAhead) >> 4);
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, kSplitP ? 2 : 1, 0);
          if (i + kAhead < 32) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_vm<0>();
    __syncthreads();
  };

  // All of this wave's loads (tile t_begin, Q, RoPE tables) done. A compiler-visible wait, so that the
  // compiler's own load tracking does not carry the Q loads into the loop.
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();
  for (int t = t_begin; t < t_end; t += 2) {
    step(t, 0);
    if (t + 1 < t_end) step(t + 1, 1);
  }

  if (!active) return;
  // lane holds O^T[16 db + 4 g + i][query n]; the four row groups of a query hold parts of its sum
  const float l = sum_over_rows16(l_run);
  if (!qvalid) return;
  if (p.nsplit == 1) {
    const float inv = 1.f / l;
    T* orow = reinterpret_cast<T*>(p.out) + bi * p.so[0] + head * p.so[2] + (long)qidx * p.so[1];
#pragma unroll
    for (int db = 0; db < 16; ++db) {
      typename Vec<T>::x4 w4;
#pragma unroll
      for (int i = 0; i < 4; ++i) w4[i] = from_f32<T>(o[db][i] * inv);
      *reinterpret_cast<typename Vec<T>::x4*>(orow + 16 * db + 4 * g) = w4;
    }
  } else {
    // partial O [split][bh][q][256] (unnormalised, f32) and (max, sum) [split][bh][q][2]
    const long row = ((long)split * p.b * p.h + bhi) * p.lq + qidx;
    float* prow = p.opart + row * 256;
#pragma unroll
    for (int db = 0; db < 16; ++db) *reinterpret_cast<f32x4*>(prow + 16 * db + 4 * g) = o[db];
    if (g == 0) {
      float2 ml;
      ml.x = m_run;
      ml.y = l;
      *reinterpret_cast<float2*>(p.ml + row * 2) = ml;
    }
  }
}

size_t flash256_vt_bytes(int b, int h, int lk, int d) {
  if (d != 256) return 0;
  return (size_t)b * h * ((lk + 63) / 64) * f256::kTileBytes;
}

// True when flash256_kernel takes this problem: head dim exactly 256, room for the V^T tiles, and
// per-tile byte offsets of K (64 rows) inside the 32-bit range of a buffer descriptor.
bool flash256_eligible(const FlashParams& p, int elem_bytes) {
  const long lim = 1L << 30;
  return p.d == 256 && p.vt != nullptr && p.sk[1] >= 0 && 64L * p.sk[1] * elem_bytes < lim;
}

long flash256_vt_blocks(const VtJob& j) { return (long)j.b * j.h * ((j.lk + 63) / 64) * 4; }

hipError_t flash256_vt(const VtJob& j, hipStream_t stream) {
  hipLaunchKernelGGL(flash256_vt_kernel, dim3((unsigned)flash256_vt_blocks(j)), dim3(256), 0, stream, j);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch256(FlashParams p, bool ropeq, hipStream_t stream) {
  if (!p.vt_ready) {
    VtJob j{p.v, {p.sv[0], p.sv[1], p.sv[2]}, p.b, p.h, p.lk, p.vt};
    if (const hipError_t e = flash256_vt(j, stream); e != hipSuccess) return e;
  }
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
