// qkv projection output -> q, kT, v with the bias added, for gfx950 (the producer of the fused
// attention's input layout):
//
//   y [T, 3*C] (T = windows * n tokens, C = nh * hd; columns ordered (qkv, head, d)) + bias [3*C]
//   -> out [3, BH*n*hd]: q [BH, n, hd], kT [BH, hd, n], v [BH, n, hd], BH = windows * nh
//
// as the reference's qkv_split (kernels.rs:872-894; sam.cu:111-128; CPU twin kernels.rs:228-264). Every
// output element is from_T(to_f32(y) + to_f32(bias)), the reference's arithmetic, so results are
// bit-identical to it.
//
// One workgroup per (window, token tile, head), the tiles of a window balanced (196 tokens: 4 x 49).
// A thread owns one token of the tile and every fourth 16-byte vector of its head's row (all of them
// requested before the first store, for more bytes in flight), so the index arithmetic has no division: q and v rows are copied with 16-byte accesses on both sides; the k part
// goes through an LDS tile so that kT is written as rows of consecutive tokens (up to 128 bytes in
// f16) rather than 2-byte scatters. Bound by HBM: y is read once, out written once.
//
// Grid mode (gw > 0): y holds the tokens of the unpadded [B, gh, gw] grid, and the windows are cut from
// it here, as the reference's window_partition (sam1/encoder.rs:129-137) does before its qkv linear:
// window w = (b, wi, wj) over the grid zero-padded to multiples of ws, token (ti, tj) of it at grid
// (wi*ws + ti, wj*ws + tj). A padding token's projection is 0, so its q, k and v are the bias alone
// (from_T(0 + bias), as the reference computes them). The qkv linear then runs on the gh*gw grid
// tokens instead of the padded windows' ones.
//
// window_merge is the step after the attention: ctx [B*nW*nh, ws*ws, hd] in window order -> out
// [B, gh, gw, nh*hd], heads merged (sam1/encoder.rs:83) and the windows put back on the grid without
// their padding (window_unpartition, sam1/encoder.rs:140-143), four 16-byte vectors per thread, all loaded
// before the first is stored.
#include "common.hpp"

namespace samhip {

constexpr int kQkvTok = 64;     // tokens per tile at most
constexpr int kQkvLanes = 4;    // threads per token row
constexpr int kQkvThreads = kQkvTok * kQkvLanes;

// VE elements per vector access (16 bytes, or 1 when hd is not a multiple of 8); NV (VE == 8): a bound on the
// vectors per thread and part, ceil(hd / 8 / kQkvLanes), so that every load of the thread is issued before the
// first store (NV = 0: one vector at a time)
template <typename T, int VE, int NV>
__global__ __launch_bounds__(kQkvThreads) void qkv_split_kernel(const T* __restrict__ y, const T* __restrict__ bias,
                                                               T* __restrict__ out, int n, int nh, int hd, int tiles,
                                                               int tt, long plane, int gh, int gw, int ws) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* kt_tile = reinterpret_cast<float*>(smem);  // [hd][kQkvTok + 1]
  typedef typename Vec<T>::x8 V8;
  const int C = nh * hd;
  // workgroup i runs on XCD i % 8: give each XCD a contiguous range of (window, tile, head), so the heads
  // of a token tile, whose row slices share cache lines at their edges, meet in one L2
  const int nblk = gridDim.x, xcd = blockIdx.x & 7, per = nblk >> 3, rem = nblk & 7;
  const long lin = (long)xcd * per + (xcd < rem ? xcd : rem) + (blockIdx.x >> 3);
  const int head = (int)(lin % nh);
  const int tile = (int)((lin / nh) % tiles);
  const long win = lin / ((long)nh * tiles);
  const int n0 = tile * tt;
  const int ntok = min(tt, n - n0);
  const long bh = win * nh + head;
  const int vpr = hd / VE;  // vectors per token row of one head
  const int tok = threadIdx.x / kQkvLanes, lane = threadIdx.x % kQkvLanes;
  // the token's row of y: window order, or its place on the grid (-1: a padding token)
  long t = win * n + n0 + tok;
  if (gw > 0) {
    const int nww = (gw + ws - 1) / ws, nwin = ((gh + ws - 1) / ws) * nww;
    const long wb = win / nwin;
    const int wr = (int)(win - wb * nwin), wi = wr / nww, wj = wr - wi * nww;
    const int i = n0 + tok, ti = i / ws, tj = i - ti * ws, r = wi * ws + ti, c = wj * ws + tj;
    t = r < gh && c < gw ? (wb * gh + r) * gw + c : -1;
  }
  if (NV > 0 && tok < ntok) {
    // the token's q, k and v vectors of this head, all requested before any is used
    const T* yrow = y + (t < 0 ? 0 : t) * 3L * C + head * hd;
    V8 a[3][NV > 0 ? NV : 1];
#pragma unroll
    for (int which = 0; which < 3; ++which)
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int v = lane + j * kQkvLanes;
        a[which][j] = t < 0 || v >= vpr ? V8{} : *reinterpret_cast<const V8*>(yrow + which * C + v * 8);
      }
#pragma unroll
    for (int which = 0; which < 3; ++which) {
      const T* bsrc = bias + which * C + head * hd;
      T* dst = out + which * plane + (bh * n + n0 + tok) * hd;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int v = lane + j * kQkvLanes;
        if (v >= vpr) break;
        const V8 bb = *reinterpret_cast<const V8*>(bsrc + v * 8);
        float vals[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vals[e] = to_f32(a[which][j][e]) + to_f32(bb[e]);
        if (which == 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) kt_tile[(v * 8 + e) * (kQkvTok + 1) + tok] = vals[e];
        } else {
          V8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = from_f32<T>(vals[e]);
          *reinterpret_cast<V8*>(dst + v * 8) = o;
        }
      }
    }
  } else if (tok < ntok) {
    const T* yrow = y + (t < 0 ? 0 : t) * 3L * C + head * hd;
#pragma unroll
    for (int which = 0; which < 3; ++which) {
      const T* src = yrow + which * C;
      const T* bsrc = bias + which * C + head * hd;
      T* dst = out + which * plane + (bh * n + n0 + tok) * hd;
      for (int v = lane; v < vpr; v += kQkvLanes) {
        const int d0 = v * VE;
        float vals[VE];
        if constexpr (VE == 8) {
          const V8 a = t < 0 ? V8{} : *reinterpret_cast<const V8*>(src + d0);
          const V8 bb = *reinterpret_cast<const V8*>(bsrc + d0);
#pragma unroll
          for (int e = 0; e < 8; ++e) vals[e] = to_f32(a[e]) + to_f32(bb[e]);
        } else {
          vals[0] = (t < 0 ? 0.f : to_f32(src[d0])) + to_f32(bsrc[d0]);
        }
        if (which == 1) {
#pragma unroll
          for (int e = 0; e < VE; ++e) kt_tile[(d0 + e) * (kQkvTok + 1) + tok] = vals[e];
        } else if constexpr (VE == 8) {
          V8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = from_f32<T>(vals[e]);
          *reinterpret_cast<V8*>(dst + d0) = o;
        } else {
          dst[d0] = from_f32<T>(vals[0]);
        }
      }
    }
  }
  __syncthreads();
  // kT rows: kt[bh][d][n0 .. n0 + ntok), a wave writing one row of up to 64 consecutive tokens
  T* kdst = out + plane + bh * (long)hd * n + n0;
  const int wtok = threadIdx.x % kQkvTok, wrow = threadIdx.x / kQkvTok;
  if (wtok < ntok)
    for (int d = wrow; d < hd; d += kQkvThreads / kQkvTok)
      kdst[(long)d * n + wtok] = from_f32<T>(kt_tile[d * (kQkvTok + 1) + wtok]);
}

template <typename T>
static hipError_t launch_qkv(const void* y, const void* bias, void* out, long tokens, int n, int nh, int hd,
                             hipStream_t stream, int gh = 0, int gw = 0, int ws = 0) {
  const long windows = tokens / n;
  const int tiles = (n + kQkvTok - 1) / kQkvTok;
  const int tt = (n + tiles - 1) / tiles;  // balanced tiles of at most kQkvTok tokens
  const long blocks = windows * tiles * nh;
  const long plane = tokens * nh * (long)hd;
  const size_t lds = (size_t)hd * (kQkvTok + 1) * sizeof(float);
  const int nv = (hd / 8 + kQkvLanes - 1) / kQkvLanes;  // vectors per thread and part (hd % 8 == 0)
  if (hd % 8 == 0 && nv <= 2)
    hipLaunchKernelGGL((qkv_split_kernel<T, 8, 2>), dim3((unsigned)blocks), dim3(kQkvThreads), lds, stream,
                       (const T*)y, (const T*)bias, (T*)out, n, nh, hd, tiles, tt, plane, gh, gw, ws);
  else if (hd % 8 == 0 && nv == 3)
    hipLaunchKernelGGL((qkv_split_kernel<T, 8, 3>), dim3((unsigned)blocks), dim3(kQkvThreads), lds, stream,
                       (const T*)y, (const T*)bias, (T*)out, n, nh, hd, tiles, tt, plane, gh, gw, ws);
  else if (hd % 8 == 0 && nv == 4)
    hipLaunchKernelGGL((qkv_split_kernel<T, 8, 4>), dim3((unsigned)blocks), dim3(kQkvThreads), lds, stream,
                       (const T*)y, (const T*)bias, (T*)out, n, nh, hd, tiles, tt, plane, gh, gw, ws);
  else if (hd % 8 == 0)
    hipLaunchKernelGGL((qkv_split_kernel<T, 8, 0>), dim3((unsigned)blocks), dim3(kQkvThreads), lds, stream,
                       (const T*)y, (const T*)bias, (T*)out, n, nh, hd, tiles, tt, plane, gh, gw, ws);
  else
    hipLaunchKernelGGL((qkv_split_kernel<T, 1, 0>), dim3((unsigned)blocks), dim3(kQkvThreads), lds, stream,
                       (const T*)y, (const T*)bias, (T*)out, n, nh, hd, tiles, tt, plane, gh, gw, ws);
  return hipGetLastError();
}

// Checked by the caller: tokens % n == 0, hd <= 256, 3*nh*hd*tokens < 2^40, blocks < 2^31.
hipError_t qkv_split(int dtype, const void* y, const void* bias, void* out, long tokens, int n, int nh, int hd,
                     hipStream_t stream) {
  if (dtype == kF32) return launch_qkv<float>(y, bias, out, tokens, n, nh, hd, stream);
  if (dtype == kF16) return launch_qkv<f16>(y, bias, out, tokens, n, nh, hd, stream);
  return launch_qkv<bf16>(y, bias, out, tokens, n, nh, hd, stream);
}

// Checked by the caller: batch, gh, gw, ws, nh >= 1, hd <= 256; tokens = windows * ws * ws with the
// padded grid's windows; the sizes fit as in qkv_split.
hipError_t qkv_split_grid(int dtype, const void* y, const void* bias, void* out, int batch, int gh, int gw, int ws,
                          int nh, int hd, hipStream_t stream) {
  const long tokens = (long)batch * ((gh + ws - 1) / ws) * ((gw + ws - 1) / ws) * ws * ws;
  const int n = ws * ws;
  if (dtype == kF32) return launch_qkv<float>(y, bias, out, tokens, n, nh, hd, stream, gh, gw, ws);
  if (dtype == kF16) return launch_qkv<f16>(y, bias, out, tokens, n, nh, hd, stream, gh, gw, ws);
  return launch_qkv<bf16>(y, bias, out, tokens, n, nh, hd, stream, gh, gw, ws);
}

constexpr int kMergeVecs = 4;  // output vectors per thread, a block's width apart

template <typename T, int VE>
__global__ __launch_bounds__(256) void window_merge_kernel(const T* __restrict__ ctx, T* __restrict__ out, int gh,
                                                          int gw, int ws, int nh, int hd, long nvec) {
  typedef T TV __attribute__((ext_vector_type(VE)));
  const int C = nh * hd;
  const int nww = (gw + ws - 1) / ws, nwh = (gh + ws - 1) / ws;
  const long i0 = (long)blockIdx.x * (256 * kMergeVecs) + threadIdx.x;
  // every load of the thread is requested before the first store
  TV v[kMergeVecs];
#pragma unroll
  for (int k = 0; k < kMergeVecs; ++k) {
    const long i = i0 + 256L * k;
    if (i >= nvec) break;
    const long e = i * VE;  // output element: ((b*gh + r)*gw + c)*C + h*hd + d
    const long tokc = e / C;
    const int col = (int)(e - tokc * C), h = col / hd, d = col - h * hd;
    const long bg = tokc / gw;
    const int c = (int)(tokc - bg * gw);
    const long b = bg / gh;
    const int r = (int)(bg - b * gh);
    const long win = (b * nwh + r / ws) * nww + c / ws;
    const int tok = (r % ws) * ws + c % ws;
    v[k] = *reinterpret_cast<const TV*>(ctx + ((win * nh + h) * ws * ws + tok) * hd + d);
  }
#pragma unroll
  for (int k = 0; k < kMergeVecs; ++k) {
    const long i = i0 + 256L * k;
    if (i >= nvec) break;
    *reinterpret_cast<TV*>(out + i * VE) = v[k];
  }
}

template <typename T>
static hipError_t launch_merge(const void* ctx, void* out, int batch, int gh, int gw, int ws, int nh, int hd,
                               hipStream_t stream) {
  const long elems = (long)batch * gh * gw * nh * hd;
  const int ve = hd % (16 / (int)sizeof(T)) == 0 ? 16 / (int)sizeof(T) : (hd % 2 == 0 ? 2 : 1);
  const long nvec = elems / ve;
  const unsigned blocks = (unsigned)((nvec + 256 * kMergeVecs - 1) / (256 * kMergeVecs));
  if (ve == 16 / (int)sizeof(T))
    hipLaunchKernelGGL((window_merge_kernel<T, 16 / sizeof(T)>), dim3(blocks), dim3(256), 0, stream, (const T*)ctx,
                       (T*)out, gh, gw, ws, nh, hd, nvec);
  else if (ve == 2)
    hipLaunchKernelGGL((window_merge_kernel<T, 2>), dim3(blocks), dim3(256), 0, stream, (const T*)ctx, (T*)out, gh,
                       gw, ws, nh, hd, nvec);
  else
    hipLaunchKernelGGL((window_merge_kernel<T, 1>), dim3(blocks), dim3(256), 0, stream, (const T*)ctx, (T*)out, gh,
                       gw, ws, nh, hd, nvec);
  return hipGetLastError();
}

// Checked by the caller: batch, gh, gw, ws, nh, hd >= 1, 16-byte aligned pointers, sizes below 2^40.
hipError_t window_merge(int dtype, const void* ctx, void* out, int batch, int gh, int gw, int ws, int nh, int hd,
                        hipStream_t stream) {
  if (dtype == kF32) return launch_merge<float>(ctx, out, batch, gh, gw, ws, nh, hd, stream);
  if (dtype == kF16) return launch_merge<f16>(ctx, out, batch, gh, gw, ws, nh, hd, stream);
  return launch_merge<bf16>(ctx, out, batch, gh, gw, ws, nh, hd, stream);
}

}  // namespace samhip
