// Fused rel-pos attention for the global 64-column grid of the SAM ViT (64x64 tokens, hd 80 for ViT-H,
// hd 64 for ViT-B and ViT-L), f16 / bf16, for gfx950.
//
//   out[bh, r, :] = softmax_k( scale * q[r] . k[k] + q[r] . Th[i - kh + H-1] + q[r] . Tw[j - kw + W-1] ) . v
//
// the arithmetic of the reference's bmm(q, kT) -> relpos_softmax -> bmm(P, v) (sam1/encoder.rs:79-82,
// kernels.rs:12-43, 899-924) fused: a workgroup of 8 waves owns 256 queries of one head; a key tile is
// one grid row of 64 keys, so the Rh bias is one value per query and tile and the Rw bias repeats in
// every tile. S^T = K . Q^T on v_mfma_f32_32x32x16 (lane = query), online exp2 softmax with a lazy
// rescale, O^T = V^T . P^T with P straight from the S^T accumulators; the S^T of tile t+1 is issued on
// the MFMA while tile t's exponentials run.
//
// On gfx950 the MFMA and the VALU work of a SIMD barely overlap (measured: the time of a loop is close
// to the sum of its MFMA and VALU times), and exp2 issues at a quarter of the FMA rate, so the kernel
// keeps the per-score VALU work to exp2 with its fma, the tile max and the f32 -> f16 packing:
//   * q stays exact: the MFMA starts from Rw*log2(e)/(scale*log2(e)) and one fma per score applies the
//     scale and Rh - m_run in f32. (Pre-scaling q in f16 would save that fma, 2.5% of the ViT-H global
//     layer, but its rounding moves a logit by about 2^-12 of |scale * q . k|: q and k of standard
//     deviation 3, or scale 1 on unit inputs, came out 8e-3 beyond the output's rounding.)
//   * hd 80: the softmax denominator comes out of the P.V product: the V^T rows 80..95 of the third
//     32-row block read a ones vector, so O^T rows 80..95 are the running sums of P (as rounded for the
//     MFMA). hd 64 has no spare rows (two full blocks), so a lane sums its P values on the VALU (v_dot2
//     of the packed f16 P with ones; bf16 adds the f32 values) and the two lanes of a query add their
//     halves at the end.
// The tiles reach LDS by 16-byte LDS DMA (global_load_lds_dwordx4) through a ring of 4 buffers, three
// tiles ahead, the DMAs of a step spread over it: no staging registers and no LDS stores in the loop;
// each wave waits only for its own DMAs of the tile it needs next (s_waitcnt vmcnt, then the one
// barrier per tile). kT tiles are stored [d][64] with 8-byte chunks XOR-swizzled by row
// (conflict-free transpose reads at a 128-byte pitch); V tiles are [64][hd] with chunk-rotated rows
// (conflict-free at a 160- or 128-byte pitch), followed by ones (hd 80). Workgroups are numbered
// XCD-major so that the 16 query blocks of a head share one XCD's L2.
// Limits (checked by the dispatcher): W == 64, 1 <= H <= 64, hd 80 or 64, 2^-6 <= scale*log2(e) <= 4.
#include "lds_dma.hpp"
#include "relpos_geom.hpp"

namespace samhip {

namespace glob {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRing = 4;
constexpr int kRhsRows = 65;  // per-wave Rh scratch: 64 key rows + a junk row
constexpr float kSlack = 8.0f;

template <int HD> struct Shape {
  static constexpr int kKS = HD / 16;
  static constexpr bool kOnesRows = HD % 32 != 0;  // the P sums ride in V^T rows past hd
  static constexpr int kMBO = (HD + 31) / 32;      // 32-row blocks of O^T
  static constexpr int kTile = HD * 64;            // elements of a kT tile [hd][64] and of a V tile [64][hd]
  static constexpr int kVStride = kTile + 128;     // a V buffer and 128 ones (a multiple of 256 bytes)
  static constexpr int kUnits = HD / 4;            // 1 KB DMA units of a tile: hd/8 of kT, hd/8 of V
  static constexpr int kChunks = HD / 4;           // 8-byte chunks of a V row
  static constexpr int kVOff = kRing * kTile;
  static constexpr int kRhsOff = kVOff + kRing * kVStride;  // elements
  static constexpr size_t kLdsBytes = (size_t)kRhsOff * 2 + (size_t)kWaves * kRhsRows * 32 * sizeof(float);
  static_assert(HD == 80 || HD == 64, "head dims");
  static_assert(254 * HD <= kVOff, "the table must fit in the kT ring during the prologue");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
  // DMAs of a wave per tile: parts p = 0, 1, 2 move unit wave + 8p while it is below kUnits
  static constexpr int dmas(int wave) { return (wave < kUnits) + (wave + 8 < kUnits) + (wave + 16 < kUnits); }
  // Chunk rotation of V rows: chunk c of key row r is stored at (c + vrot(r)) % kChunks, so that the
  // 4 rows x 8 chunks a half wave's transpose read touches fall on 64 distinct banks for every column
  // block. 160-byte pitch (hd 80, 20 chunks): even rows move by 4 chunks. 128-byte pitch (hd 64, 16
  // chunks): rows 2, 3 (mod 4) move by 8, onto the banks that rows 0, 1 leave free.
  static constexpr int vrot(int r) { return HD == 80 ? ((r & 1) ? 0 : 4) : (((r >> 1) & 1) ? 8 : 0); }
};

// Chunk swizzle of kT rows (128-byte pitch): 8-byte chunk c of row d is stored at c ^ kswz(d).
__host__ __device__ constexpr int kswz(int d) { return 2 * (d & 1) + 8 * ((d >> 1) & 1) + 4 * ((d >> 3) & 1); }

}  // namespace glob

__device__ __forceinline__ int glob_xcd_block(int i, int total) {
  const int per = total >> 3, rem = total & 7, x = i & 7, j = i >> 3;
  return x * per + (x < rem ? x : rem) + j;
}

template <typename T, int HD>
__global__ __launch_bounds__(glob::kThreads) void attn_relpos_glob_kernel(const T* __restrict__ q,
                                                                         const T* __restrict__ kt,
                                                                         const T* __restrict__ v,
                                                                         const T* __restrict__ table,
                                                                         T* __restrict__ out, int H, float scale,
                                                                         int qblocks) {
  using namespace glob;
  typedef Shape<HD> S;
  constexpr int kKS = S::kKS, kMBO = S::kMBO, kTile = S::kTile, kVStride = S::kVStride, kVOff = S::kVOff;
  constexpr int kUnitsK = HD / 8;  // DMA units of the kT part of a tile
  typedef typename Vec<T>::x8 X8;
  constexpr bool kF16 = __is_same(T, f16);
  constexpr bool kSplitP = !kF16;           // bf16: P as hi + lo for the P.V product
  constexpr int W = 64;
  constexpr unsigned short kOne = kF16 ? 0x3C00 : 0x3F80;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* kring = reinterpret_cast<T*>(smem);
  T* vring = kring + kVOff;
  T* tbl = kring;  // the table, during the prologue only
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* rhs = reinterpret_cast<float*>(kring + S::kRhsOff) + wave * kRhsRows * 32;
  const unsigned lds0 = lds_addr(smem);

  const int N = H * W;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int n = lane & 31, hh = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;
  const int blk = glob_xcd_block(blockIdx.x, gridDim.x);
  const long bh = blk / qblocks;
  const int qidx = (blk % qblocks) * (kWaves * 32) + wave * 32 + n;
  const bool qvalid = qidx < N;
  const int qi = qvalid ? qidx / W : 0, qj = qvalid ? qidx % W : 0;
  const float sc = scale * kLog2e;
  const int ntiles = H;

  // ---- prologue (plain loads; no DMA is in flight yet): q fragments, the table into LDS, the ones
  X8 qf[kKS];
  {
    const T* qrow = q + (bh * N + (qvalid ? qidx : 0)) * HD;
#pragma unroll
    for (int s = 0; s < kKS; ++s) qf[s] = *reinterpret_cast<const X8*>(qrow + 16 * s + 8 * hh);
  }
  const int trows = 2 * H - 1 + 2 * W - 1;
  for (int c = tid; c < trows * (HD / 8); c += kThreads)
    *reinterpret_cast<u32x4*>(tbl + c * 8) = *reinterpret_cast<const u32x4*>(table + c * 8);
  static_assert(kThreads == kRing * (kVStride - kTile), "one thread per ones element");
  if constexpr (S::kOnesRows) reinterpret_cast<unsigned short*>(vring)[(tid >> 7) * kVStride + kTile + (tid & 127)] = kOne;
  __syncthreads();

  // G = T . Q^T on the MFMA (4 row blocks of each table), scattered along the diagonal band
  f32x16 gw[4], gh[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    gw[b] = f32x16{};
    gh[b] = f32x16{};
  }
#pragma unroll
  for (int s = 0; s < kKS; ++s) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      // rows past the end of a table hold other rows or stale data and are never scattered
      const X8 aw = *reinterpret_cast<const X8*>(tbl + (2 * H - 1 + 32 * b + n) * HD + 16 * s + 8 * hh);
      const X8 ah = *reinterpret_cast<const X8*>(tbl + (32 * b + n) * HD + 16 * s + 8 * hh);
      gw[b] = mma32(aw, qf[s], gw[b]);
      gh[b] = mma32(ah, qf[s], gh[b]);
    }
  }
  auto scatter = [&](const f32x16* gb, int rows, int base, int len) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = 32 * b + 8 * (e >> 2) + 4 * hh + (e & 3);
        const int k = base + len - 1 - rr;  // kh = i + H-1 - rr, kw = j + W-1 - rr
        const bool ok = rr < rows && k >= 0 && k < len;
        rhs[(ok ? k : 64) * 32 + n] = gb[b][e] * kLog2e;
      }
  };
  auto wave_sync = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  scatter(gw, 2 * W - 1, qj, W);
  wave_sync();
  // a lane's key columns in 32-key block mb: 32*mb + 8*(e>>2) + 4*hh + (e&3); the accumulator starts at
  // Rw*log2(e) / sc
  f32x16 cinit[2];
  {
    const float f = 1.f / sc;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) cinit[mb][e] = rhs[(32 * mb + 8 * (e >> 2) + 4 * hh + (e & 3)) * 32 + n] * f;
  }
  wave_sync();
  scatter(gh, 2 * H - 1, qi, H);
  __syncthreads();  // every wave is done with the table: the kT ring is free

  // ---- the DMA ring: tile t (grid row t) into buffer t % 4; past the last tile, reload the last.
  // A tile is hd/4 units of 1 KB moved by 16-byte DMAs: units u < hd/8 are kT rows 8u .. 8u+7, the
  // others the V elements [512 (u - hd/8), + 512). Wave w moves units w, w+8 and w+16 while they exist
  // (hd 80: 20 units, waves 0..3 move three; hd 64: 16 units, two each). The swizzle and the rotation
  // move 16-byte pairs of 8-byte chunks together, so every lane's 16 bytes are 8 consecutive keys (kT)
  // or 8 consecutive columns (V) in global memory. Per-lane byte offsets are fixed; the tile moves the
  // scalar base.
  const char* kbase = reinterpret_cast<const char*>(kt + bh * HD * (long)N);
  const char* vbase = reinterpret_cast<const char*>(v + bh * (long)N * HD);
  unsigned dofs[3];
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    const int u = wave + 8 * p;
    if (u < kUnitsK) {
      const int d = 8 * u + (lane >> 3);
      const int c = (2 * (lane & 7)) ^ kswz(d);  // first of the two logical 8-byte chunks
      dofs[p] = (unsigned)(sizeof(T) * (d * N + 4 * c));
    } else {
      const int e = (u - kUnitsK) * 512 + 8 * lane;
      const int row = e / HD, ch = (e % HD) >> 2;
      dofs[p] = (unsigned)(sizeof(T) * (row * HD + 4 * ((ch + S::kChunks - S::vrot(row)) % S::kChunks)));
    }
  }
  // part p of this wave's share of tile t (into buffer buf)
  auto dma_part = [&](int t, int buf, int p) {
    const int tt = t < ntiles ? t : ntiles - 1;
    const int u = wave + 8 * p;
    if (u < kUnitsK)
      dma16(kbase + sizeof(T) * tt * W, dofs[p], lds0 + (buf * kTile + u * 512) * 2);
    else if (u < S::kUnits)
      dma16(vbase + sizeof(T) * tt * W * HD, dofs[p],
            lds0 + (kVOff + buf * kVStride + (u - kUnitsK) * 512) * 2);
  };
  auto dma_tile = [&](int t, int buf) {
#pragma unroll
    for (int p = 0; p < 3; ++p) dma_part(t, buf, p);
  };
  // this wave's DMAs per tile (S::dmas); waits for all but the last n tiles
  auto wait_tiles = [&](auto n) {
    if (S::dmas(wave) == 3)
      wait_vm<3 * decltype(n)::value>();
    else
      wait_vm<2 * decltype(n)::value>();
  };
  static_assert(S::dmas(0) >= 2 && S::dmas(7) >= 2 && S::dmas(0) <= 3, "two or three DMAs per wave and tile");
#pragma unroll
  for (int t = 0; t < 3; ++t) dma_tile(t, t);

  // per-lane byte addresses of the transpose reads in buffer 0; buffers, k-steps and column blocks
  // are instruction offsets (all below 64 KB)
  unsigned kaddr[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int d = 8 * (g >> 1) + (gi >> 2);  // + 16k (+4): the swizzle bits of d are lane constant
    const int key = 32 * mb + 16 * (g & 1) + 4 * (gi & 3);
    kaddr[mb] = opaque(lds0 + 2 * (d * 64 + (((key >> 2) ^ kswz(d)) << 2)));
  }
  // V^T: block ob reads columns 32*ob + 16*(g&1) + 4*(gi&3), logical chunk 8*ob + c0 of the key row.
  // hd 80: block 1 is 8 chunks after block 0 in every row (no wrap: c0 + vrot <= 11), so vaddr serves
  // both; in block 2 the groups with g&1 (V^T rows 80..95) read the ones that follow the buffer.
  // hd 64: the rotation wraps, so each block has its own addresses (vaddr for block 0, vaddr2 for 1).
  unsigned vaddr[4][2], vaddr2[4][2];
#pragma unroll
  for (int w4 = 0; w4 < 4; ++w4)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int key = 32 * (w4 >> 1) + 16 * (w4 & 1) + 8 * r + 4 * (g >> 1) + (gi >> 2);
      const int c0 = 4 * (g & 1) + (gi & 3);  // this lane's chunk in block 0
      const auto at = [&](int c) { return 4 * ((c + S::vrot(key)) % S::kChunks); };
      vaddr[w4][r] = opaque(lds0 + 2 * (kVOff + key * HD + at(c0)));
      if constexpr (S::kOnesRows) {
        // block 2: data lanes read chunk 16 + (gi&3); the ones lanes of each half wave read a ones
        // element whose bank the half wave's data does not use (banks 0..31 in the first half, 32..63
        // in the second; the V buffers are 256-byte multiples apart, so this holds in every buffer)
        const int e2 = key * HD + at(16 + (gi & 3));
        vaddr2[w4][r] = opaque(lds0 + 2 * (kVOff + ((g & 1) ? kTile + (g == 1 ? 64 : 0) : e2)));
      } else {
        vaddr2[w4][r] = opaque(lds0 + 2 * (kVOff + key * HD + at(8 + c0)));
      }
    }
  float m_run = 0.f;
  float lsum = 0.f;  // hd 64: this lane's share of the softmax denominator
  f32x16 o[kMBO];
#pragma unroll
  for (int ob = 0; ob < kMBO; ++ob) o[ob] = f32x16{};
  // S^T of tile t from buffer buf (t past the last tile: a discarded product of the reloaded last tile)
  // K . Q^T part of a tile's S^T from buffer buf (past the last tile: a product of the reloaded last
  // tile, masked by the bias); it does not depend on the softmax state, so it is issued first
  auto qk_k = [&](int buf, f32x16* s) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int k = 0; k < kKS; ++k) {
        const unsigned p = kaddr[mb] + 2 * (buf * kTile + 16 * k * 64);
        const X8 a = join8<T>(lds_read_tr16_at(p), lds_read_tr16_at(p + 2 * 4 * 64));
        s[mb] = mma32(a, qf[k], k == 0 ? cinit[mb] : s[mb]);
      }
    }
    // the transpose reads run three MFMAs ahead, so that the LDS latency hides behind the MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
    for (int i = 0; i < 2 * kKS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
  };
  // Softmax and P.V of tile t (scores in s_cur, K/V in buffer buf = t % 4) with the S^T of tile t+1
  // into s_nxt.
  auto step = [&](int t, int buf, f32x16* s_cur, f32x16* s_nxt) {
    wait_tiles(std::integral_constant<int, 1>());  // this wave's tile t+1 has landed (t+2 may be in flight)
    __syncthreads();  // everyone's tile t+1 is visible; everyone is done with tile t-1
    // tile t+3 into the buffer tile t-1 just freed, in three parts spread over the step
    dma_part(t + 3, (buf + 3) & 3, 0);
    qk_k((buf + 1) & 3, s_nxt);
    dma_part(t + 3, (buf + 3) & 3, 1);
    // exp2 argument: s*sc + c, relative to m_run
    const float c = t < ntiles ? rhs[t * 32 + n] - m_run : -INFINITY;
    float mm = s_cur[0][0];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mm = max_nc(mm, s_cur[mb][e]);
    const float mt = max_with_partner32(fmaf(mm, sc, c));
    float cc = c;
    if (wave_any(t == 0 || mt > kSlack)) {
      // the first tile sets m_run; later ones raise it when a score exceeds it by more than the slack
      const float delta = t == 0 ? mt : fmaxf(mt, 0.f);
      const float alpha = t == 0 ? 0.f : exp2_fast(-delta);
#pragma unroll
      for (int ob = 0; ob < kMBO; ++ob) o[ob] *= alpha;
      if constexpr (!S::kOnesRows) lsum *= alpha;
      m_run += delta;
      cc -= delta;
    }
    dma_part(t + 3, (buf + 3) & 3, 2);
    X8 b[4], blo[4];
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = s_cur[w4 >> 1][8 * (w4 & 1) + e];
        pv[e] = exp2_fast(fmaf(x, sc, cc));
      }
      b[w4] = pack8(pv, (X8*)nullptr);
      if constexpr (!S::kOnesRows) {
        if constexpr (kF16) {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int e = 0; e < 8; e += 2)
            lsum = __builtin_amdgcn_fdot2(h2{b[w4][e], b[w4][e + 1]}, h2{(f16)1.f, (f16)1.f}, lsum, false);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) lsum += pv[e];
        }
      }
      if (kSplitP) {
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] -= to_f32(b[w4][e]);
        blo[w4] = pack8(pv, (X8*)nullptr);
      }
    }
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4)
#pragma unroll
      for (int ob = 0; ob < kMBO; ++ob) {
        unsigned p0, p1;
        if constexpr (S::kOnesRows) {
          p0 = (ob == 2 ? vaddr2[w4][0] : vaddr[w4][0] + 64 * ob) + 2 * buf * kVStride;
          p1 = (ob == 2 ? vaddr2[w4][1] : vaddr[w4][1] + 64 * ob) + 2 * buf * kVStride;
        } else {
          p0 = (ob == 1 ? vaddr2[w4][0] : vaddr[w4][0]) + 2 * buf * kVStride;
          p1 = (ob == 1 ? vaddr2[w4][1] : vaddr[w4][1]) + 2 * buf * kVStride;
        }
        const X8 a = join8<T>(lds_read_tr16_at(p0), lds_read_tr16_at(p1));
        o[ob] = mma32(a, b[w4], o[ob]);
        if (kSplitP) o[ob] = mma32(a, blo[w4], o[ob]);
      }
    if constexpr (!kSplitP) {  // reads three MFMAs ahead, as in qk_k
      __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
      for (int i = 0; i < 4 * kMBO; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
    }
  };

  f32x16 sa[2], sb[2];
  wait_tiles(std::integral_constant<int, 2>());  // tile 0 has landed (tiles 1, 2 may be in flight)
  __syncthreads();
  qk_k(0, sa);
  // unrolled by the ring depth, so that every buffer offset is a constant; tiles past the last (up to
  // the next multiple of 4) are masked: their bias is -inf, so they add nothing
  for (int t = 0; t < ntiles; t += 4) {
    step(t, 0, sa, sb);
    step(t + 1, 1, sb, sa);
    step(t + 2, 2, sa, sb);
    step(t + 3, 3, sb, sa);
  }
  wait_vm<0>();  // the last DMAs (reloads) must land before the workgroup's LDS is released

  // ---- normalise and store: lane holds O^T[32*ob + 8*a + 4*hh + b][query n]; hd 80: rows 80..95 hold
  // the sum; hd 64: the lanes l and l ^ 32 of a query hold the two halves of its sum
  float l;
  if constexpr (S::kOnesRows)
    l = o[2][8];
  else
    l = sum_with_partner32(lsum);
  const float inv = 1.f / l;
  if (qvalid) {
    T* orow = out + (bh * N + qidx) * HD;
#pragma unroll
    for (int ob = 0; ob < kMBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        if (32 * ob + 8 * a < HD) {
          typename Vec<T>::x4 w4;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) w4[bb] = from_f32<T>(o[ob][4 * a + bb] * inv);
          *reinterpret_cast<typename Vec<T>::x4*>(orow + 32 * ob + 8 * a + 4 * hh) = w4;
        }
      }
  }
}

template <typename T, int HD>
static hipError_t launch_glob(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                              int h, float scale, hipStream_t stream) {
  auto kern = attn_relpos_glob_kernel<T, HD>;
  constexpr size_t lds = glob::Shape<HD>::kLdsBytes;
  static std::atomic<unsigned long long> lds_done{0};
  if (const hipError_t e = lds_opt_in(lds_done, (const void*)kern, (int)lds); e != hipSuccess) return e;
  const int qblocks = (h * 64 + glob::kWaves * 32 - 1) / (glob::kWaves * 32);
  hipLaunchKernelGGL(kern, dim3((unsigned)(bh * qblocks)), dim3(glob::kThreads), lds, stream,
                     (const T*)q, (const T*)kt, (const T*)v, (const T*)table, (T*)out, h, scale, qblocks);
  return hipGetLastError();
}

// The 64-column global grid (W == 64, H <= 64, hd 80 or 64); returns false (nothing launched) for shapes
// it does not take. The accumulator starts at Rw*log2(e) / (scale*log2(e)), so the factor must be
// positive; 2^-6 <= scale*log2(e) <= 4 (SAM's hd^-0.5 * log2(e) = 0.16) keeps that start value and the
// scaled logits of ordinary size. Other scales take the general kernel.
bool attn_relpos_global(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                        int hd, int h, int w, float scale, hipStream_t stream, hipError_t* err) {
  const float sc = scale * kLog2e;
  if ((hd != 80 && hd != 64) || w != 64 || h < 1 || h > 64 || !(sc >= 0.015625f && sc <= 4.f)) return false;
  if (hd == 80)
    *err = dtype == kF16 ? launch_glob<f16, 80>(q, kt, v, table, out, bh, h, scale, stream)
                         : launch_glob<bf16, 80>(q, kt, v, table, out, bh, h, scale, stream);
  else
    *err = dtype == kF16 ? launch_glob<f16, 64>(q, kt, v, table, out, bh, h, scale, stream)
                         : launch_glob<bf16, 64>(q, kt, v, table, out, bh, h, scale, stream);
  return true;
}

}  // namespace samhip
