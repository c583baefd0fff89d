// SAM image preprocessing for gfx950: antialiased triangle-filter resize of an RGB u8 image [h, w, 3]
// to nh x nw, (x - mean[c]) / std[c], zero padded into [3, size, size] (f32, f16 or bf16).
//
// The arithmetic of the reference's CPU path (image_proc.rs:57-96, the same filter as the GPU kernel
// sam.cu:162-204 and PIL's bilinear resize), step for step in f32 with no FMA contraction, so f32
// output matches it bit for bit: the tap span from truncating casts, the weight sums in tap order,
// r = sum_xx w(xx) * px per input row, acc += wy * r, then (acc / (wsx * wsy) - mean) / std (a
// division by std, as the CPU path does; the reference GPU kernel multiplies by 1/std instead).
//
// One thread per output pixel, all three channels; a workgroup covers 4 output rows x 64 columns. The
// filter weights depend on the column (horizontal) or the row (vertical) only, so the workgroup computes
// each column's and each row's taps once into LDS, and every thread then runs the reference's per-pixel
// loops (r = sum_xx w(xx) * px per input row, acc += wy * r) on those stored values. Pixels outside
// nh x nw write zeros. The input bytes are gathered with byte loads, shared by adjacent threads through
// the L1 and L2.
#include "common.hpp"

namespace samhip {

namespace prep {
constexpr int kCols = 64, kRows = 4;  // output pixels of a workgroup
constexpr int kThreads = kCols * kRows;
constexpr int kMaxTaps = 64;  // filter taps per output pixel and axis
}  // namespace prep

__device__ __forceinline__ float prep_tri(float x) {
  x = fabsf(x);
  return x < 1.f ? 1.f - x : 0.f;
}

template <typename T>
__global__ __launch_bounds__(prep::kThreads) void preprocess_kernel(const unsigned char* __restrict__ img,
                                                                    T* __restrict__ out, int h, int w, int nh,
                                                                    int nw, int size, float sx, float sy, float fx,
                                                                    float fy, int xtaps, int ytaps, float m0,
                                                                    float m1, float m2, float s0, float s1,
                                                                    float s2) {
#pragma clang fp contract(off)
  using namespace prep;
  extern __shared__ float lds[];
  float* wxs = lds;                                          // [xtaps][kCols]
  float* wys = wxs + xtaps * kCols;                          // [kRows][ytaps]
  int* xspan = reinterpret_cast<int*>(wys + kRows * ytaps);  // [kCols][2]: x0, x1
  int* yspan = xspan + 2 * kCols;                            // [kRows][2]: y0, y1
  const int tid = threadIdx.x, c = tid % kCols, t = tid / kCols;
  const int xb = blockIdx.x * kCols, yb = blockIdx.y * kRows;

  // horizontal taps of the workgroup's columns (one thread per column)
  if (t == 0) {
    const int x = xb + c;
    long x0 = 0, x1 = 0;
    if (x < nw) {
      const float cx = ((float)x + 0.5f) * sx;
      x0 = max((long)(cx - fx + 0.5f), 0L);
      x1 = min((long)(cx + fx + 0.5f), (long)w);
      for (long xx = x0; xx < x1; ++xx) wxs[(xx - x0) * kCols + c] = prep_tri(((float)xx + 0.5f - cx) / fx);
    }
    xspan[2 * c] = (int)x0;
    xspan[2 * c + 1] = (int)x1;
  }
  // vertical taps of the workgroup's rows (one thread per row and tap)
  for (int i = tid; i < kRows * ytaps; i += kThreads) {
    const int r = i / ytaps, k = i - r * ytaps, y = yb + r;
    long y0 = 0, y1 = 0;
    if (y < nh) {
      const float cy = ((float)y + 0.5f) * sy;
      y0 = max((long)(cy - fy + 0.5f), 0L);
      y1 = min((long)(cy + fy + 0.5f), (long)h);
      if (y0 + k < y1) wys[i] = prep_tri(((float)(y0 + k) + 0.5f - cy) / fy);
    }
    if (k == 0) {
      yspan[2 * r] = (int)y0;
      yspan[2 * r + 1] = (int)y1;
    }
  }
  __syncthreads();

  const int x = xb + c, y = yb + t;
  if (x >= size || y >= size) return;
  const long plane = (long)size * size;
  T* o = out + (long)y * size + x;
  if (x >= nw || y >= nh) {
    o[0] = from_f32<T>(0.f);
    o[plane] = from_f32<T>(0.f);
    o[2 * plane] = from_f32<T>(0.f);
    return;
  }
  const int x0 = xspan[2 * c], nx = xspan[2 * c + 1] - x0;
  const int y0 = yspan[2 * t], ny = yspan[2 * t + 1] - y0;
  const float* wx = wxs + c;
  const float* wy = wys + t * ytaps;
  float wsx = 0.f, wsy = 0.f;
  for (int j = 0; j < nx; ++j) wsx += wx[j * kCols];
  for (int k = 0; k < ny; ++k) wsy += wy[k];
  float a0 = 0.f, a1 = 0.f, a2 = 0.f;
  for (int k = 0; k < ny; ++k) {
    const unsigned char* p = img + ((long)(y0 + k) * w + x0) * 3;
    float r0 = 0.f, r1 = 0.f, r2 = 0.f;
    for (int j = 0; j < nx; ++j) {
      const float wt = wx[j * kCols];
      r0 += wt * (float)p[3 * j];
      r1 += wt * (float)p[3 * j + 1];
      r2 += wt * (float)p[3 * j + 2];
    }
    const float wk = wy[k];
    a0 += wk * r0;
    a1 += wk * r1;
    a2 += wk * r2;
  }
  const float ws = wsx * wsy;
  o[0] = from_f32<T>((a0 / ws - m0) / s0);
  o[plane] = from_f32<T>((a1 / ws - m1) / s1);
  o[2 * plane] = from_f32<T>((a2 / ws - m2) / s2);
}

// Filter taps per output pixel never exceed this bound on either axis:
// x1 - x0 <= (cx + fx + 0.5) - (cx - fx + 0.5) + 1.
int preprocess_max_taps(int n, int nout) {
  const float s = (float)n / (float)nout;
  const float f = s > 1.f ? s : 1.f;
  return (int)(2.f * f) + 2;
}

template <typename T>
static hipError_t launch_pre(const unsigned char* img, void* out, int h, int w, int nh, int nw, int size,
                             const float* mean, const float* stdv, hipStream_t stream) {
  using namespace prep;
  const float sx = (float)w / (float)nw, sy = (float)h / (float)nh;
  const float fx = sx > 1.f ? sx : 1.f, fy = sy > 1.f ? sy : 1.f;
  const int xtaps = preprocess_max_taps(w, nw), ytaps = preprocess_max_taps(h, nh);
  const size_t lds = ((size_t)xtaps * kCols + (size_t)kRows * ytaps + 2 * (kCols + kRows)) * sizeof(float);
  static std::atomic<unsigned long long> lds_done{0};  // opt-in to more than the default dynamic LDS
  {
    const int most = (kMaxTaps * (kCols + kRows) + 2 * (kCols + kRows)) * (int)sizeof(float);
    const hipError_t e = lds_opt_in(lds_done, (const void*)preprocess_kernel<T>, most);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((unsigned)((size + kCols - 1) / kCols), (unsigned)((size + kRows - 1) / kRows));
  hipLaunchKernelGGL(preprocess_kernel<T>, grid, dim3(kThreads), lds, stream, img, (T*)out, h, w, nh, nw, size, sx, sy,
                     fx, fy, xtaps, ytaps, mean[0], mean[1], mean[2], stdv[0], stdv[1], stdv[2]);
  return hipGetLastError();
}

// Checked by the caller: 1 <= nh, nw <= size, preprocess_max_taps(w, nw) <= 64, preprocess_max_taps(h, nh) <= 64.
hipError_t preprocess(int dtype, const void* img, void* out, int h, int w, int nh, int nw, int size, const float* mean,
                      const float* stdv, hipStream_t stream) {
  const unsigned char* src = reinterpret_cast<const unsigned char*>(img);
  if (dtype == kF32) return launch_pre<float>(src, out, h, w, nh, nw, size, mean, stdv, stream);
  if (dtype == kF16) return launch_pre<f16>(src, out, h, w, nh, nw, size, mean, stdv, stream);
  return launch_pre<bf16>(src, out, h, w, nh, nw, size, mean, stdv, stream);
}

}  // namespace samhip
