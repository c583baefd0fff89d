// Fused rel-pos attention for the 14x14 windows of the SAM ViT (hd 80 for ViT-H, hd 64 for ViT-B and
// ViT-L), f16 / bf16, for gfx950.
//
//   out[u, r, :] = softmax_k( scale * q[r] . k[k] + q[r] . Th[i - kh + H-1] + q[r] . Tw[j - kw + W-1] ) . v
//
// for every unit u = (batch, window, head), the same arithmetic as attn_relpos.hip (the reference's
// bmm(q, kT) -> relpos_softmax -> bmm(P, v), sam1/encoder.rs:79-82, kernels.rs:12-43, 899-924), and
// the same key loop: tiles of 4 grid rows padded to 16 columns, S^T = K . Q^T on v_mfma_f32_32x32x16
// with the Rw bias as the initial accumulator and the Rh bias one value per 32-key block (both from a
// Q . T^T prologue on the MFMA, scattered along the diagonal band in a wave-private scratch), online
// exp2 softmax with a lazy rescale, O^T = V^T . P^T with P taken straight from the S^T accumulators.
//
// A windowed layer is bound by HBM and by latency: a unit is 125 KB of q, kT, v and out for 12 MFLOP,
// and there are only 400 of them per ViT-H layer. So the kernel is built for overlap between
// workgroups rather than for a single one:
//   * a workgroup of 4 waves takes half a unit (query blocks 0-3 or 4-7, one per wave) and needs
//     80 KB (hd 80) or 48 KB (hd 64) of LDS, so two (hd 80) or three (hd 64) fit on a CU: one loads
//     while another computes, and the 800 half units of a ViT-H layer fill the 512 workgroup slots of
//     the chip in one and a half rounds instead of two full ones (the 600 of a ViT-B layer fit the 768
//     slots at hd 64 in one);
//   * all data moves by LDS DMA (global_load_lds): the q rows, the table and tile 0 are requested at
//     once, q into ring buffer 1 and the table into buffer 2 (hd 80: into its own area), which tiles
//     1 and 2 take over once the bias prologue has read them; tile 3 then goes into buffer 0. At hd 80
//     the ring carries V only: the unit's whole kT is requested with the q rows, two contiguous rows
//     per DMA, and stays resident (a tile's kT is 80 runs of 112 bytes at a 392-byte pitch, which
//     costs more to fetch per tile than whole rows once). Both halves of a unit run on one
//     XCD. In a grid of more than two rounds they are adjacent workgroups, so the second half's K and
//     V come from L2. In a smaller grid all first halves go first, so that the last round holds the
//     lighter second halves;
//   * each wave waits only for its own DMAs of what it needs next (s_waitcnt vmcnt: a wave's vector
//     memory operations complete in issue order), then one barrier publishes everyone's share;
//   * kT tiles are stored [d][64 slots] (hd 80: [d][4 tiles][64 slots], tile t in segment t ^ (d & 1))
//     with the 8-byte chunks of each row XOR-swizzled by the row's low bits, so the transpose reads
//     (ds_read_b64_tr_b16) of four consecutive rows hit disjoint banks; V tiles are [64 slots][hd] with the 8-byte chunks of a slot rotated: hd 80 (160-byte
//     pitch) moves even slots by 4 chunks, hd 64 (128-byte pitch) slots 2, 3 (mod 4) by 8, so that the
//     4 slots x 8 chunks of a half wave's transpose read fall on 64 distinct banks. hd 80: the O^T rows
//     80..95 are discarded (their lanes re-read block 0). The softmax denominator is summed on the VALU;
//   * q rows and table rows are [row][hd] with the 16-byte chunks of a row rotated (hd 80: by one for
//     rows 8..15 of every 16; hd 64: by (row / 2) mod 8), so that the 16-byte reads of 16 rows at one
//     column fall on 64 distinct banks.
// Padding keys (columns >= W, rows >= H) and padding table rows read valid data of the same tensor:
// the keys' bias is -inf (P = 0), and the table rows' products are never scattered.
// Limits (checked by the dispatcher): 13 <= H <= 16 (4 key tiles), W <= 16 and even, hd 80 or 64,
// scale > 0.
#include "lds_dma.hpp"
#include "relpos_geom.hpp"

namespace samhip {

namespace win {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTiles = 4;          // key tiles per unit
constexpr int kRing = 3;           // tile buffers
constexpr int kQRows = kWaves * 32;  // q rows of a half unit
constexpr int kTRows = 64;         // table rows in LDS: Th at [0, 32), Tw at [32, 64)
constexpr int kRhsRows = 18;       // per-wave bias scratch rows: -1 (junk), 0..15, 16 (junk)
constexpr float kSlack = 8.0f;

template <int HD> struct Shape {
  static constexpr int kKS = HD / 16;            // k-steps of S^T = K Q^T
  static constexpr int kMBO = (HD + 31) / 32;    // 32-row blocks of O^T (hd 80: rows 80..95 are not stored)
  static constexpr int kTile = HD * 64;          // elements of a kT tile [d][64] and of a V tile [64][hd]
  static constexpr int kUnits = HD / 8;          // 1 KB DMA units of a kT or V tile (and of the table)
  static constexpr int kKDma = (kUnits + kWaves - 1) / kWaves;  // per wave: hd 80: 3 (2 repeats), hd 64: 2
  static constexpr int kVDma = kKDma;
  static constexpr int kTbDma = kKDma;
  static constexpr int kTDma = kKDma + kVDma;    // DMAs per wave per tile
  static constexpr int kQDma = kQRows * HD * 2 / 1024 / kWaves;  // 1 KB units of q per wave: 5 or 4
  static constexpr int kChunks = HD / 4;         // 8-byte chunks of a V slot
  static constexpr int kQChunks = HD / 8;        // 16-byte chunks of a q or table row
  // Two layouts.
  // * kRes (hd 80): the unit's whole kT is resident, [d][4 tiles][64 slots] at a 512-byte row pitch,
  //   requested in the prologue by DMAs that each cover two whole rows of the unit's kT (two
  //   contiguous 392-byte runs); only V goes through the ring (buffer b at kVOff + b kTile). The q rows
  //   fill V buffers 1 and 2 until the prologue has read them; the table has its own area. 80 KB, two
  //   workgroups per CU.
  // * otherwise (hd 64): buffer b is a kT tile at 2 b kTile and a V tile right after it; the q rows
  //   fill buffer 1 and the table the kT half of buffer 2 until the prologue has read them. 48 KB,
  //   three workgroups per CU.
  // In both, a wave's bias scratch then overlays its own 32 q rows, which it alone reads (into
  // registers) before it scatters, and the same rows stage its output once the last tile is in
  // buffer 0.
  static constexpr bool kRes = HD == 80;
  static constexpr int kSlots = kRes ? 256 : 64;   // kT row length in LDS (elements)
  static constexpr int kBuf = kRes ? kTile : 2 * kTile;   // ring buffer stride
  static constexpr int kVOff = kRes ? HD * 256 : kTile;   // V of ring buffer 0
  static constexpr int kQOff = kRes ? kVOff + kTile : kBuf;
  static constexpr int kTbOff = kRes ? kVOff + 3 * kTile : 2 * kBuf;
  static constexpr int kKAll = kRes ? HD * 512 / 1024 / kWaves : 0;  // resident kT: DMAs per wave
  static constexpr size_t kLdsBytes = kRes ? (size_t)(kTbOff + kTRows * HD) * 2 : (size_t)kRing * kBuf * 2;
  static constexpr int kPerCU = kRes ? 2 : 3;       // workgroups per CU
  static_assert(HD == 80 || HD == 64, "head dims");
  static_assert(kRhsRows * 32 * sizeof(float) <= 32 * HD * 2, "the scratch fits in a wave's q rows");
  static_assert(kPerCU * kLdsBytes <= 160 * 1024, "workgroups per CU");
  static_assert(kQRows * HD * 2 % (1024 * kWaves) == 0, "DMA split");
  static_assert(kTile * 2 <= kKDma * kWaves * 1024 && kTRows * HD * 2 <= kTbDma * kWaves * 1024, "units");
  static_assert(kQRows * HD <= (kRes ? 2 * kTile : kBuf) && kTRows * HD <= kTile, "staging fits");
  static_assert(!kRes || HD * 512 % (1024 * kWaves) == 0, "resident kT DMA split");
  // V chunk rotation: 8-byte chunk c of slot r is stored at (c + vrot(r)) % kChunks
  static constexpr int vrot(int r) { return HD == 80 ? ((r & 1) ? 0 : 4) : (((r >> 1) & 1) ? 8 : 0); }
  // q / table row rotation: 16-byte chunk c of LDS row r is stored at (c + qrot(r)) % kQChunks
  static constexpr int qrot(int r) { return HD == 80 ? ((r >> 3) & 1) : ((r >> 1) & 7); }
  // DMA unit of part i0 (parts past the last unit repeat the first ones)
  static constexpr int unit(int i0) { return i0 < kUnits ? i0 : i0 - kUnits; }
};

// Chunk swizzle of kT rows: 8-byte chunk c of row d is stored at c ^ kswz(d & 3).
__host__ __device__ constexpr int kswz(int r) { return 2 * (r & 1) + 8 * (r >> 1); }

}  // namespace win

__device__ __forceinline__ int win_xcd_block(int i, int total) {
  const int per = total >> 3, rem = total & 7, x = i & 7, j = i >> 3;
  return x * per + (x < rem ? x : rem) + j;
}

// HW > 0: the grid is HW x HW, a compile-time constant (the SAM windows, 14 x 14), so that the index
// arithmetic of the DMAs, the bias scatter and the stores folds; HW == 0 takes H and W at run time.
template <typename T, int HD, int HW>
__global__ __launch_bounds__(win::kThreads, 2) void attn_relpos_win_kernel(const T* __restrict__ q,
                                                                       const T* __restrict__ kt,
                                                                       const T* __restrict__ v,
                                                                       const T* __restrict__ table,
                                                                       T* __restrict__ out, int H_, int W_,
                                                                       float scale, int nunits, int n8) {
  const int H = HW ? HW : H_, W = HW ? HW : W_;
  using namespace win;
  typedef Shape<HD> S;
  constexpr int kKS = S::kKS, kMBO = S::kMBO, kBuf = S::kBuf, kTDma = S::kTDma;
  typedef KeyGeom<kPair> KG;
  typedef typename Vec<T>::x8 X8;
  constexpr bool kSplitP = __is_same(T, bf16);

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* kring = reinterpret_cast<T*>(smem);
  T* tb = kring + S::kTbOff;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: DMA destinations derive from it
  // the bias scratch, wave-private, over this wave's q rows in buffer 1 (prologue only)
  float* rhs = reinterpret_cast<float*>(kring + S::kQOff + wave * 32 * HD);
  const unsigned lds0 = lds_addr(smem);

  const int N = H * W;
  const int lane = threadIdx.x & 63;
  const int n = lane & 31, hh = lane >> 5;
  const int g = lane >> 4, gi = lane & 15;
  const long unit_elems = (long)N * HD;
  // Work order. n8 > 0: all first halves (workgroups [0, n8)), then all second halves; n8 is the unit
  // count rounded up to a multiple of 8, so both halves of a unit run on the same XCD (workgroup i
  // runs on XCD i % 8). n8 == 0: the halves of a unit are adjacent, in contiguous ranges per XCD.
  long u;
  int half;
  if (n8 > 0) {
    half = blockIdx.x >= (unsigned)n8;
    u = (long)blockIdx.x - half * n8;
  } else {
    const int blk = win_xcd_block(blockIdx.x, gridDim.x);
    u = blk >> 1;
    half = blk & 1;
  }
  if (u >= nunits) return;  // padding workgroup (n8 > 0): nothing issued, no barrier reached
  const int q0 = half * kQRows;  // first query of this half unit
  const int qidx = q0 + wave * 32 + n;
  const bool qvalid = qidx < N;
  // qidx < 256 and W <= 16: (qidx + 0.5) / W lies at least 0.5 / W from an integer, far beyond the
  // error of the approximate reciprocal and product, so truncation gives the exact quotient
  const int qdiv = (int)(((float)qidx + 0.5f) * __builtin_amdgcn_rcpf((float)W));
  const int qi = qvalid ? qdiv : 0, qj = qvalid ? qidx - qdiv * W : 0;
  const float sc = scale * kLog2e;
  // kT and V go through buffer descriptors of the unit's kT and V, so a lane's DMA offset is the same
  // for every tile (the tile's start is a wave-uniform soffset): slots past a grid row's W columns and
  // rows past H read other keys of the unit (their bias is -inf, so P = 0) or, past the unit's end, 0
  const i32x4 krsrc = buffer_rsrc(kt + u * unit_elems, (unsigned)(sizeof(T) * unit_elems));
  const i32x4 vrsrc = buffer_rsrc(v + u * unit_elems, (unsigned)(sizeof(T) * unit_elems));
  constexpr int kKD = S::kRes ? S::kKAll : S::kKDma;
  unsigned kdof[kKD], vdof[S::kVDma];
#pragma unroll
  for (int p = 0; p < kKD; ++p) {
    // kT, 16 bytes (8 slots) a lane: the swizzle keeps 16-byte pairs of 8-byte chunks together, so they
    // are the 8 consecutive slots from slot 4c = one grid row's columns kap .. kap+7 (kap = 0 or 8).
    // Resident: unit i covers rows 2i, 2i+1, a lane row 2i + lane/32, segment (lane/8)%4, which holds
    // tile t = segment ^ (d & 1). Ring: unit i covers rows 8i .. 8i+7 of the tile, a lane row
    // 8i + lane/8 (the tile is the DMA's soffset); hd 80 would repeat units 0, 1 as 10, 11.
    const int i = S::kRes ? wave * S::kKAll + p : S::unit(wave + kWaves * p);
    const int d = S::kRes ? 2 * i + (lane >> 5) : 8 * i + (lane >> 3);
    const int t = S::kRes ? ((lane >> 3) & 3) ^ (d & 1) : 0;
    const int c = (2 * (lane & 7)) ^ kswz(d & 3);
    kdof[p] = (unsigned)(sizeof(T) * (d * N + (4 * t + (c >> 2)) * W + 4 * (c & 3)));
  }
#pragma unroll
  for (int p = 0; p < S::kVDma; ++p) {
    // V: unit j covers elements [512 j, 512 j + 512) of the [64 slots][hd] tile, a lane 8 columns
    // (two chunks, the rotation moves them together) of one slot; hd 80: units 10, 11 repeat 0, 1
    const int j = S::unit(wave + kWaves * p);
    const int e = j * 512 + 8 * lane;
    const int slot = e / HD, ch = (e % HD) >> 2;
    const int col = 4 * ((ch + S::kChunks - S::vrot(slot)) % S::kChunks);
    vdof[p] = (unsigned)(sizeof(T) * (((slot >> 4) * W + (slot & 15)) * HD + col));
  }

  // This wave's DMAs of tile t (grid rows 4t .. 4t+3) into ring buffer buf: V, and kT unless it is
  // resident (kTDma of them, or kVDma)
  constexpr int kStepDma = S::kRes ? S::kVDma : kTDma;
  auto tile_dma = [&](int t, int buf) {
    const unsigned kso = (unsigned)(sizeof(T) * 4 * t * W), vso = kso * HD;
    if constexpr (!S::kRes) {
#pragma unroll
      for (int p = 0; p < S::kKDma; ++p)
        bdma16s(krsrc, kdof[p], kso, lds0 + (buf * kBuf + S::unit(wave + kWaves * p) * 512) * 2);
    }
#pragma unroll
    for (int p = 0; p < S::kVDma; ++p)
      bdma16s(vrsrc, vdof[p], vso, lds0 + (S::kVOff + buf * kBuf + S::unit(wave + kWaves * p) * 512) * 2);
  };

  // ---- 1. the half unit's q rows, the table and tile 0, all requested at once
  {
    const char* base = reinterpret_cast<const char*>(q + u * unit_elems);
#pragma unroll
    for (int p = 0; p < S::kQDma; ++p) {
      const int i = wave * S::kQDma + p;  // unit i covers q-image elements [512 i, 512 i + 512)
      const int e = i * 512 + 8 * lane;
      const int row = e / HD, ch = (e % HD) >> 3;
      const int col = 8 * ((ch + S::kQChunks - S::qrot(row)) % S::kQChunks);
      const int src = q0 + row;  // queries past the end read query 0
      dma16(base, (unsigned)(sizeof(T) * ((src < N ? src : 0) * HD + col)), lds0 + (S::kQOff + i * 512) * 2);
    }
  }
  {
    // LDS row r < 32 is Th row r, row 32 + r is Tw row r (rows past the end read row 0); hd 80: units
    // 10, 11 repeat units 0, 1
    const char* base = reinterpret_cast<const char*>(table);
#pragma unroll
    for (int p = 0; p < S::kTbDma; ++p) {
      const int i = S::unit(wave + kWaves * p);
      const int e = i * 512 + 8 * lane;
      const int r = e / HD, ch = (e % HD) >> 3;
      const int col = 8 * ((ch + S::kQChunks - S::qrot(r)) % S::kQChunks);
      const int src = r < 32 ? (r < 2 * H - 1 ? r : 0) : (r - 32 < 2 * W - 1 ? 2 * H - 1 + r - 32 : 0);
      dma16(base, (unsigned)(sizeof(T) * (src * HD + col)), lds0 + (S::kTbOff + i * 512) * 2);
    }
  }
  if constexpr (S::kRes) {
#pragma unroll
    for (int p = 0; p < S::kKAll; ++p) bdma16s(krsrc, kdof[p], 0u, lds0 + (wave * S::kKAll + p) * 1024);
  }
  tile_dma(0, 0);

  // per-lane constant parts of the transpose-read addresses
  // kT (A operand of S^T): source lane (4*s + c) of group g reads row 8*(g>>1) + s (+16*k, +4), the 4
  // slots slot(mb, 16*(g&1) + 4*c); the row's low bits are s, so the swizzle is lane constant
  // Resident kT: rows at a 512-byte pitch, tile t in segment t ^ (d & 1) (d & 1 is lane constant), so
  // koff[0] serves even tiles (+ 64 t) and koff[1] odd ones; rows d and d + 1 still lie 32 banks
  // apart, as in a 128-byte-pitch tile.
  int koff[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int d = 8 * (g >> 1) + (gi >> 2);
    const int slot = KG::slot(mb, 16 * (g & 1) + 4 * (gi & 3));
    const int base = d * S::kSlots + (((slot >> 2) ^ kswz(d & 3)) << 2);
    koff[0][mb] = S::kRes ? base + 64 * (d & 1) : base;
    koff[1][mb] = S::kRes ? base - 64 * (d & 1) : base;
  }
  // V^T (A operand of O^T): source lane (4*s + c) reads the slot of key 16*(w4&1) + 8*r + 4*(g>>1) + s of
  // block w4>>1, columns 32*ob + 16*(g&1) + 4*c .. +3 (logical chunk 8*ob + 4*(g&1) + c). hd 80: block
  // 1 is 8 chunks after block 0 (no wrap: c + vrot <= 11); block 2 has its own offsets (the rotation
  // wraps), and its lanes of the discarded rows 80..95 read what the data lanes 16 below them read, so
  // the half wave touches no further banks; hd 64 keeps an offset per block.
  constexpr int kVB = HD == 80 ? 2 : kMBO;
  int voff[kVB][4][2];
#pragma unroll
  for (int ob = 0; ob < kVB; ++ob)
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int ms = 16 * (w4 & 1) + 8 * r + 4 * (g >> 1) + (gi >> 2);
        const int slot = KG::slot(w4 >> 1, ms);
        const int c = HD == 80 && ob == 1 ? 16 + (gi & 3) : 8 * ob + 4 * (g & 1) + (gi & 3);
        voff[ob][w4][r] = slot * HD + 4 * ((c + S::vrot(slot)) % S::kChunks);
      }
  auto wave_sync = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // ---- 2. the bias (q and the table have landed; tile 0 may still be in flight)
  wait_vm<S::kRes ? S::kKAll + S::kVDma : kTDma>();  // q and the table (kT, tile 0 may be in flight)
  __syncthreads();
  // this lane's q fragments (B operand of S^T = K Q^T): Q[query][16*s + 8*hh + j]
  X8 qf[kKS];
#pragma unroll
  for (int s = 0; s < kKS; ++s)
    qf[s] = *reinterpret_cast<const X8*>(kring + S::kQOff + (wave * 32 + n) * HD +
                                         8 * ((2 * s + hh + S::qrot(n)) % S::kQChunks));
  f32x16 cinit;
  float rh[kTiles][2];
  {
    f32x16 gh = f32x16{}, gw = f32x16{};
#pragma unroll
    for (int s = 0; s < kKS; ++s) {
      const int col = 8 * ((2 * s + hh + S::qrot(n)) % S::kQChunks);  // rows n and 32 + n rotate alike
      const X8 ah = *reinterpret_cast<const X8*>(tb + n * HD + col);
      const X8 aw = *reinterpret_cast<const X8*>(tb + (32 + n) * HD + col);
      gh = mma32(ah, qf[s], gh);
      gw = mma32(aw, qf[s], gw);
    }
    // Scatter along the diagonal band: accumulator element e of this lane is table row rr = re + 4 hh
    // (re = 8 (e >> 2) + (e & 3)), which belongs to key column (row) b - rr with b = qj + W - 1
    // (qi + H - 1). The column is clamped into [-1, 16] and scratch row c + 1 takes it: the valid
    // columns 0..W-1 keep their row, a table row past 2W - 2 always lands on column -1, and columns
    // W..15 and 16 are never read as valid. So each element costs a subtract, a clamp and an address.
    float* rb = rhs + 32 + n;  // scratch row 0 = column -1
    // Rw: a lane's key columns are e = 0..15 in every 32-key block, so cinit[e] = Rw[e] / sc
    {
      const int b = qj + W - 1 - 4 * hh;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int c = min(max(b - (8 * (e >> 2) + (e & 3)), -1), 16);
        rb[c * 32] = gw[e] * kLog2e;
      }
    }
    wave_sync();
    const float inv_sc = 1.f / sc;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float x = rb[e * 32];
      cinit[e] = e < W ? x * inv_sc : -INFINITY;
    }
    wave_sync();
    {
      const int b = qi + H - 1 - 4 * hh;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int c = min(max(b - (8 * (e >> 2) + (e & 3)), -1), 16);
        rb[c * 32] = gh[e] * kLog2e;
      }
    }
    wave_sync();
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const int row = 4 * t + 2 * mb + hh;  // < 16
        const float x = rb[row * 32];
        rh[t][mb] = row < H ? x : -INFINITY;
      }
  }
  __syncthreads();  // everyone has read q and the table: buffers 1 and 2 are free
  tile_dma(1, 1);
  tile_dma(2, 2);

  // ---- 3. key loop: tile t as soon as its DMAs have landed
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[kMBO];
#pragma unroll
  for (int ob = 0; ob < kMBO; ++ob) o[ob] = f32x16{};
  // Tile t from buffer buf. NB = 1 when the tile's second 32-key block (grid rows 4t+2, 4t+3) lies
  // wholly below the grid: its products, exponentials and P.V are skipped.
  auto tile = [&](int t, int buf, auto nb_c) {
    constexpr int NB = decltype(nb_c)::value;
    f32x16 s[2];
    const T* kbuf = S::kRes ? kring + 64 * t : kring + buf * kBuf;
#pragma unroll
    for (int mb = 0; mb < NB; ++mb) {
#pragma unroll
      for (int k = 0; k < kKS; ++k) {
        const T* p = kbuf + koff[t & 1][mb] + 16 * k * S::kSlots;
        const X8 a = join8<T>(lds_read_tr16(p), lds_read_tr16(p + 4 * S::kSlots));
        s[mb] = mma32(a, qf[k], k == 0 ? cinit : s[mb]);
      }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < NB; ++mb) {
      float mm = s[mb][0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mm = max_nc(mm, s[mb][e]);
      mt = max_nc(mt, fmaf(mm, sc, rh[t][mb]));
    }
    mt = max_with_partner32(mt);
    if (wave_any(mt > m_run + kSlack)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = exp2_fast(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int ob = 0; ob < kMBO; ++ob) o[ob] *= alpha;
      m_run = m_new;
    }
    float c[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) c[mb] = rh[t][mb] - m_run;
    X8 b[4], blo[4];
    float lsum = 0.f;
#pragma unroll
    for (int w4 = 0; w4 < 2 * NB; ++w4) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = exp2_fast(fmaf(s[w4 >> 1][8 * (w4 & 1) + e], sc, c[w4 >> 1]));
        if (kSplitP) lsum += pv[e];  // bf16: P.V takes hi + lo, P itself to ~16 bits
      }
      b[w4] = pack8(pv, (X8*)nullptr);
      if constexpr (!kSplitP) {
        // f16: the denominator sums P as the P.V product sees it (rounded), so that numerator and
        // denominator weigh each key alike: v_dot2 of the packed P with ones, accumulated in f32
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int e = 0; e < 8; e += 2)
          lsum = __builtin_amdgcn_fdot2(h2{b[w4][e], b[w4][e + 1]}, h2{(f16)1.f, (f16)1.f}, lsum, false);
      }
      if (kSplitP) {
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] -= to_f32(b[w4][e]);
        blo[w4] = pack8(pv, (X8*)nullptr);
      }
    }
    l_run += lsum;
    const T* vbuf = kring + S::kVOff + buf * kBuf;
#pragma unroll
    for (int w4 = 0; w4 < 2 * NB; ++w4) {
#pragma unroll
      for (int ob = 0; ob < kMBO; ++ob) {
        const int vo = HD == 80 && ob == 1 ? 32 : 0, vb = HD == 80 ? ob >> 1 : ob;
        const X8 a = join8<T>(lds_read_tr16(vbuf + voff[vb][w4][0] + vo), lds_read_tr16(vbuf + voff[vb][w4][1] + vo));
        o[ob] = mma32(a, b[w4], o[ob]);
        if (kSplitP) o[ob] = mma32(a, blo[w4], o[ob]);
      }
    }
  };
  // tile t is in buffer t % 3; tile 3 goes into buffer 0 once every wave is done with tile 0
  // A wave whose 32 queries all lie past the end of the grid (the last block of the second half)
  // skips the key loop; it still moves its share of the tiles and takes part in every barrier.
  const bool active = q0 + wave * 32 < N;
  using Two = std::integral_constant<int, 2>;
  wait_vm<2 * kStepDma>();  // tile 0 (tiles 1, 2 may be in flight)
  __syncthreads();
  if (active) tile(0, 0, Two());
  wait_vm<kStepDma>();  // tile 1 (tile 2 may be in flight)
  __syncthreads();
  tile_dma(3, 0);
  if (active) tile(1, 1, Two());
  wait_vm<kStepDma>();  // tile 2 (tile 3 may be in flight)
  __syncthreads();
  if (active) tile(2, 2, Two());
  wait_vm<0>();  // tile 3
  __syncthreads();
  if (active) {
    if (4 * 3 + 2 < H)
      tile(3, 0, Two());
    else
      tile(3, 0, std::integral_constant<int, 1>());
  }

  // ---- 4. normalise and store: lane holds O^T[32*ob + 8*a + 4*hh + b][query n]. The wave's 32 output
  // rows are consecutive in memory, so they go through LDS (its own q rows in buffer 1, free since the
  // barrier before tile 3) as the [32][hd] image of that range and leave as contiguous 1 KB stores of
  // 16-byte pieces, non-temporal: whole lines that nothing in the launch reads again (ViT-H window
  // layer 19.9 -> 19.0 us; the global kernel's 8-byte row pieces lose with the same hint). At hd 64 (128-byte rows) the 16-byte chunk c of row r sits at chunk c ^ (r & 7), so
  // the 32 rows a store instruction covers spread over the banks.
  if (active) {
    const float inv = 1.f / sum_with_partner32(l_run);
    T* stage = kring + S::kQOff + wave * 32 * HD;
#pragma unroll
    for (int ob = 0; ob < kMBO; ++ob)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        if (32 * ob + 8 * a < HD) {
          typename Vec<T>::x4 w4;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) w4[bb] = from_f32<T>(o[ob][4 * a + bb] * inv);
          *reinterpret_cast<typename Vec<T>::x4*>(stage + n * HD + 8 * (HD == 64 ? (4 * ob + a) ^ (n & 7) : 4 * ob + a) + 4 * hh) = w4;
        }
      }
    wave_sync();
    const int q0w = q0 + wave * 32;
    const int nbytes = min(32, N - q0w) * HD * (int)sizeof(T);  // valid rows only
    char* dst = reinterpret_cast<char*>(out + u * unit_elems + (long)q0w * HD);
    const char* src = reinterpret_cast<const char*>(stage);
#pragma unroll
    for (int i = 0; i < 32 * HD * (int)sizeof(T) / 1024; ++i) {
      const int b = 1024 * i + 16 * lane;
      const int sb = HD == 64 ? (b & ~127) + 16 * (((b >> 4) & 7) ^ ((b >> 7) & 7)) : b;
      if (b < nbytes) __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(src + sb), reinterpret_cast<u32x4*>(dst + b));
    }
  }
}

// ---------------------------------------------------------------------------------------------- launch

template <typename T, int HD>
static hipError_t launch_win(const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                             int h, int w, float scale, hipStream_t stream) {
  const bool sam = h == 14 && w == 14;
  auto kern = sam ? attn_relpos_win_kernel<T, HD, 14> : attn_relpos_win_kernel<T, HD, 0>;
  constexpr size_t lds = win::Shape<HD>::kLdsBytes;
  static std::atomic<unsigned long long> lds_done_all[2];
  std::atomic<unsigned long long>& lds_done = lds_done_all[sam];
  if (const hipError_t e = lds_opt_in(lds_done, (const void*)kern, (int)lds); e != hipSuccess) return e;
  // When the grid fits in two rounds of the chip's workgroup slots, the second round should hold the
  // lighter second halves (68 of 196 queries at 14x14), so all first halves go first. Larger grids
  // keep the halves of a unit adjacent, so that the second half reads K and V from L2.
  const long slots = (long)device_cu_count() * win::Shape<HD>::kPerCU;
  const int n8 = bh <= slots ? (bh + 7) / 8 * 8 : 0;
  const unsigned grid = n8 > 0 ? (unsigned)(2 * n8) : (unsigned)(2 * bh);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(win::kThreads), lds, stream, (const T*)q, (const T*)kt, (const T*)v,
                     (const T*)table, (T*)out, h, w, scale, bh, n8);
  return hipGetLastError();
}

// The SAM windows (13 <= H <= 16 so a unit is exactly 4 key tiles, W <= 16 even, hd 80 or 64,
// scale > 0); returns false (nothing launched) for shapes it does not take.
bool attn_relpos_window(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out, int bh,
                        int hd, int h, int w, float scale, hipStream_t stream, hipError_t* err) {
  if ((hd != 80 && hd != 64) || h < 13 || h > 16 || w > 16 || w % 2 != 0 || !(scale > 0.f)) return false;
  if (hd == 80)
    *err = dtype == kF16 ? launch_win<f16, 80>(q, kt, v, table, out, bh, h, w, scale, stream)
                         : launch_win<bf16, 80>(q, kt, v, table, out, bh, h, w, scale, stream);
  else
    *err = dtype == kF16 ? launch_win<f16, 64>(q, kt, v, table, out, bh, h, w, scale, stream)
                         : launch_win<bf16, 64>(q, kt, v, table, out, bh, h, w, scale, stream);
  return true;
}

}  // namespace samhip

