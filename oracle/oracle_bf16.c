/*
 * oracle_bf16.c - the reference's default CPU attention path (bf16 operands on AVX-512 BF16), restated
 * in C. Test infrastructure: the CPU baseline of the benchmark and a checked second CPU path for the
 * tests; the product never links it.
 *
 * The reference takes this path whenever the CPU has AVX-512F and AVX-512 BF16 and cpu_gemm is enabled
 * (cpu_gemm.rs:11-32); it is the default on such machines. Restated pieces, with their sources:
 *   - bf16_bits: f32 -> bf16 bits, round to nearest even (cpu_gemm.rs:38-45);
 *   - PackedB: a [K, N] matrix as panels of NR = 32 columns of (k even, k odd) bf16 pairs
 *     (cpu_gemm.rs:48-82);
 *   - block: c[rows, N] = a[rows, K] @ B, the A rows converted to bf16 (vcvtneps2bf16 by 16s, bf16_bits
 *     for the tail, zero padded to an even K and to MR = 8 rows), an MR x NR microkernel of vdpbf16ps
 *     with one broadcast (a[2q], a[2q+1]) pair per row (cpu_gemm.rs:129-178);
 *   - Bf16Matmul: row blocks of MC = 64 in parallel (cpu_gemm.rs:100-126);
 *   - softmax_row: x*scale + Rh (one fma) + Rw, masked 16-lane vectors, a max reduction, exp_ps, a
 *     16-lane sum then _mm512_reduce_add_ps, times 1/sum (cpu_gemm.rs:229-270);
 *   - exp_ps: 2^(x log2 e) with a degree-6 polynomial on the rounded fraction and vscalefps
 *     (cpu_gemm.rs:272-286; the reference's own coefficients);
 *   - rel_bias: sequential f32 dot products, no fused multiply-add (cpu_gemm.rs:292-303);
 *   - softmax_scaled: softmax(s * scale) on the same vector pattern (cpu_gemm.rs:321-354);
 *   - flash_attention: [B, L, H, D] attention, K^T and V packed once per (batch, head), 32-row query
 *     tiles (cpu_gemm.rs:361-417);
 *   - TiledAttention's bf16 branch: kT and V packed per head, per 32-row tile q @ kT on the bf16
 *     kernel, rel_bias and softmax_row per row, then P @ V on the bf16 kernel (kernels.rs:139-179).
 * Rust does not contract a * b + c into an fma, so this file is compiled with -ffp-contract=off; the
 * fmas are the reference's explicit _mm512_fmadd_ps.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "sam_oracle.h"

#define NR 32
#define MR 8
#define MC 64
#define ATT_TILE 32
#define BF16_FN __attribute__((target("avx512f,avx512bf16")))

static int threads_or_all(int n) { return n > 0 ? n : omp_get_max_threads(); }

int oracle_bf16_available(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bf16");
}

/* cpu_gemm.rs:38-45 */
static uint16_t bf16_bits(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  if (isnan(x)) return (uint16_t)((b >> 16) | 0x40);
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

void oracle_bf16_round(const float* x, uint16_t* out, long n) {
  for (long i = 0; i < n; ++i) out[i] = bf16_bits(x[i]);
}

typedef struct {
  int k, n, kp;
  uint32_t* data; /* panels * kp * NR pairs */
} PackedB;

/* cpu_gemm.rs:64-82: w row-major [k, n] */
static PackedB packed_from(const float* w, int k, int n, long ld) {
  PackedB b;
  b.k = k;
  b.n = n;
  b.kp = (k + 1) / 2;
  const int panels = (n + NR - 1) / NR;
  b.data = (uint32_t*)calloc((size_t)panels * b.kp * NR, sizeof(uint32_t));
  for (int p = 0; p < panels; ++p)
    for (int q = 0; q < b.kp; ++q)
      for (int c = 0; c < NR; ++c) {
        const int col = p * NR + c;
        if (col >= n) continue;
        const uint32_t lo = bf16_bits(w[(long)(2 * q) * ld + col]);
        const uint32_t hi = 2 * q + 1 < k ? bf16_bits(w[(long)(2 * q + 1) * ld + col]) : 0;
        b.data[((long)p * b.kp + q) * NR + c] = lo | (hi << 16);
      }
  return b;
}

/* cpu_gemm.rs:129-178: c[rows, n] = a[rows, k] @ b, one block of rows */
BF16_FN static void block(const PackedB* b, const float* a, int rows, float* c) {
  const int k = b->k, n = b->n, kp = b->kp, kpad = 2 * kp;
  const int padded_rows = (rows + MR - 1) / MR * MR;
  uint16_t* ab = (uint16_t*)calloc((size_t)padded_rows * kpad, sizeof(uint16_t));
  for (int r = 0; r < rows; ++r) {
    const float* src = a + (long)r * k;
    uint16_t* dst = ab + (long)r * kpad;
    int i = 0;
    for (; i + 16 <= k; i += 16) {
      const __m256bh h = _mm512_cvtneps_pbh(_mm512_loadu_ps(src + i));
      _mm256_storeu_si256((__m256i*)(dst + i), (__m256i)h);
    }
    for (; i < k; ++i) dst[i] = bf16_bits(src[i]);
  }
  const int panels = (n + NR - 1) / NR;
  float tmp[MR * NR];
  for (int p = 0; p < panels; ++p) {
    const uint32_t* bp = b->data + (long)p * kp * NR;
    const int cols = NR < n - p * NR ? NR : n - p * NR;
    for (int r0 = 0; r0 < padded_rows; r0 += MR) {
      const uint16_t* ap = ab + (long)r0 * kpad;
      __m512 acc[MR][2];
      for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = _mm512_setzero_ps();
      for (int q = 0; q < kp; ++q) {
        const __m512bh b0 = (__m512bh)_mm512_loadu_si512((const void*)(bp + (long)q * NR));
        const __m512bh b1 = (__m512bh)_mm512_loadu_si512((const void*)(bp + (long)q * NR + 16));
        for (int r = 0; r < MR; ++r) {
          uint32_t pair;
          memcpy(&pair, ap + (long)r * kpad + 2 * q, 4);
          const __m512bh av = (__m512bh)_mm512_set1_epi32((int)pair);
          acc[r][0] = _mm512_dpbf16_ps(acc[r][0], av, b0);
          acc[r][1] = _mm512_dpbf16_ps(acc[r][1], av, b1);
        }
      }
      const int live = rows - r0 < MR ? (rows - r0 > 0 ? rows - r0 : 0) : MR;
      for (int r = 0; r < live; ++r) {
        _mm512_storeu_ps(tmp + r * NR, acc[r][0]);
        _mm512_storeu_ps(tmp + r * NR + 16, acc[r][1]);
        memcpy(c + (long)(r0 + r) * n + p * NR, tmp + r * NR, sizeof(float) * cols);
      }
    }
  }
  free(ab);
}

/* cpu_gemm.rs:100-126: x [m, k] @ w [k, n] on the bf16 kernel, row blocks of MC in parallel */
void oracle_bf16_matmul(const float* x, const float* w, float* c, int m, int k, int n, int nthreads) {
  PackedB b = packed_from(w, k, n, n);
  const int blocks = (m + MC - 1) / MC;
#pragma omp parallel for schedule(static) num_threads(threads_or_all(nthreads))
  for (int blk = 0; blk < blocks; ++blk) {
    const int r0 = blk * MC, rows = MC < m - r0 ? MC : m - r0;
    block(&b, x + (long)r0 * k, rows, c + (long)r0 * n);
  }
  free(b.data);
}

/* cpu_gemm.rs:272-286 */
BF16_FN static inline __m512 exp_ps(__m512 x) {
  const __m512 t = _mm512_max_ps(_mm512_mul_ps(x, _mm512_set1_ps(1.44269504088896340736f)), _mm512_set1_ps(-126.0f));
  const __m512 n = _mm512_roundscale_ps(t, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  const __m512 r = _mm512_sub_ps(t, n);
  static const float cs[6] = {0.00133335581f, 0.00961812911f, 0.0555041087f, 0.240226507f, 0.693147181f, 1.0f};
  __m512 p = _mm512_set1_ps(0.000154035303f);
  for (int i = 0; i < 6; ++i) p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(cs[i]));
  return _mm512_scalef_ps(p, n);
}

BF16_FN void oracle_bf16_exp(const float* x, float* y, long n) {
  long i = 0;
  for (; i + 16 <= n; i += 16) _mm512_storeu_ps(y + i, exp_ps(_mm512_loadu_ps(x + i)));
  for (; i < n; ++i) {
    float buf[16] = {0};
    buf[0] = x[i];
    float out[16];
    _mm512_storeu_ps(out, exp_ps(_mm512_loadu_ps(buf)));
    y[i] = out[0];
  }
}

static inline __mmask16 tail_mask(int left) { return left >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << left) - 1); }

/* cpu_gemm.rs:229-270 */
BF16_FN static void softmax_row(float* s, const float* rh, const float* rw, int h, int w, float scale) {
  const int n = h * w;
  const __m512 vscale = _mm512_set1_ps(scale);
  __m512 vmax = _mm512_set1_ps(-INFINITY);
  for (int kh = 0; kh < h; ++kh) {
    const __m512 add = _mm512_set1_ps(rh[kh]);
    for (int kw = 0; kw < w; kw += 16) {
      const __mmask16 m = tail_mask(w - kw);
      float* p = s + (long)kh * w + kw;
      const __m512 x = _mm512_maskz_loadu_ps(m, p);
      const __m512 b = _mm512_maskz_loadu_ps(m, rw + kw);
      const __m512 v = _mm512_add_ps(_mm512_fmadd_ps(x, vscale, add), b);
      _mm512_mask_storeu_ps(p, m, v);
      vmax = _mm512_mask_max_ps(vmax, m, vmax, v);
    }
  }
  const __m512 vm = _mm512_set1_ps(_mm512_reduce_max_ps(vmax));
  __m512 vsum = _mm512_setzero_ps();
  for (int i = 0; i < n; i += 16) {
    const __mmask16 m = tail_mask(n - i);
    const __m512 e = exp_ps(_mm512_sub_ps(_mm512_maskz_loadu_ps(m, s + i), vm));
    _mm512_mask_storeu_ps(s + i, m, e);
    vsum = _mm512_mask_add_ps(vsum, m, vsum, e);
  }
  const __m512 inv = _mm512_set1_ps(1.0f / _mm512_reduce_add_ps(vsum));
  for (int i = 0; i < n; i += 16) {
    const __mmask16 m = tail_mask(n - i);
    _mm512_mask_storeu_ps(s + i, m, _mm512_mul_ps(_mm512_maskz_loadu_ps(m, s + i), inv));
  }
}

/* cpu_gemm.rs:321-354 */
BF16_FN static void softmax_scaled(float* s, int n, float scale) {
  const __m512 vscale = _mm512_set1_ps(scale);
  __m512 vmax = _mm512_set1_ps(-INFINITY);
  for (int i = 0; i < n; i += 16) {
    const __mmask16 m = tail_mask(n - i);
    const __m512 v = _mm512_mul_ps(_mm512_maskz_loadu_ps(m, s + i), vscale);
    _mm512_mask_storeu_ps(s + i, m, v);
    vmax = _mm512_mask_max_ps(vmax, m, vmax, v);
  }
  const __m512 vm = _mm512_set1_ps(_mm512_reduce_max_ps(vmax));
  __m512 vsum = _mm512_setzero_ps();
  for (int i = 0; i < n; i += 16) {
    const __mmask16 m = tail_mask(n - i);
    const __m512 e = exp_ps(_mm512_sub_ps(_mm512_maskz_loadu_ps(m, s + i), vm));
    _mm512_mask_storeu_ps(s + i, m, e);
    vsum = _mm512_mask_add_ps(vsum, m, vsum, e);
  }
  const __m512 inv = _mm512_set1_ps(1.0f / _mm512_reduce_add_ps(vsum));
  for (int i = 0; i < n; i += 16) {
    const __mmask16 m = tail_mask(n - i);
    _mm512_mask_storeu_ps(s + i, m, _mm512_mul_ps(_mm512_maskz_loadu_ps(m, s + i), inv));
  }
}

/* cpu_gemm.rs:292-303: sequential dot products (no fma) */
static void rel_bias(const float* q, const float* th, const float* tw, int h, int w, int hd, int i, int j, float* rh,
                     float* rw) {
  for (int kh = 0; kh < h; ++kh) {
    const float* t = th + (long)(i + h - 1 - kh) * hd;
    float s = 0.0f;
    for (int c = 0; c < hd; ++c) s += t[c] * q[c];
    rh[kh] = s;
  }
  for (int kw = 0; kw < w; ++kw) {
    const float* t = tw + (long)(j + w - 1 - kw) * hd;
    float s = 0.0f;
    for (int c = 0; c < hd; ++c) s += t[c] * q[c];
    rw[kw] = s;
  }
}

/* kernels.rs:139-179 (TiledAttention, bf16 branch): q [bh, n, hd], kt [bh, hd, n], v [bh, n, hd] */
void oracle_bf16_attention_relpos(const float* q, const float* kt, const float* v, const float* table, float* out,
                                  long bh, int h, int w, int hd, float scale, int nthreads) {
  const int n = h * w, tiles = (n + ATT_TILE - 1) / ATT_TILE;
  const float* th = table;
  const float* tw = table + (long)(2 * h - 1) * hd;
  PackedB* kp = (PackedB*)malloc(sizeof(PackedB) * bh);
  PackedB* vp = (PackedB*)malloc(sizeof(PackedB) * bh);
  const int nt = threads_or_all(nthreads);
#pragma omp parallel for schedule(static) num_threads(nt)
  for (long b = 0; b < bh; ++b) {
    kp[b] = packed_from(kt + b * (long)hd * n, hd, n, n);
    vp[b] = packed_from(v + b * (long)n * hd, n, hd, hd);
  }
#pragma omp parallel num_threads(nt)
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)ATT_TILE * n);
    float* rh = (float*)malloc(sizeof(float) * h);
    float* rw = (float*)malloc(sizeof(float) * w);
#pragma omp for schedule(dynamic)
    for (long task = 0; task < bh * tiles; ++task) {
      const long b = task / tiles;
      const int t = (int)(task % tiles);
      const int r0 = t * ATT_TILE, rows = ATT_TILE < n - r0 ? ATT_TILE : n - r0;
      const float* qb = q + (b * n + r0) * (long)hd;
      block(&kp[b], qb, rows, sc);
      for (int r = 0; r < rows; ++r) {
        const int row = r0 + r, i = row / w, j = row % w;
        rel_bias(qb + (long)r * hd, th, tw, h, w, hd, i, j, rh, rw);
        softmax_row(sc + (long)r * n, rh, rw, h, w, scale);
      }
      block(&vp[b], sc, rows, out + (b * n + r0) * (long)hd);
    }
    free(sc);
    free(rh);
    free(rw);
  }
  for (long b = 0; b < bh; ++b) {
    free(kp[b].data);
    free(vp[b].data);
  }
  free(kp);
  free(vp);
}

/* cpu_gemm.rs:361-417: q [b, lq, h, d], k/v [b, lk, h, d] -> out [b, lq, h, d] */
void oracle_bf16_flash_attention(const float* q, const float* k, const float* v, float* out, int b, int lq, int lk,
                                 int h, int d, float scale, int nthreads) {
  const long row = (long)h * d;
  const int nt = threads_or_all(nthreads);
  PackedB* kp = (PackedB*)malloc(sizeof(PackedB) * (size_t)b * h);
  PackedB* vp = (PackedB*)malloc(sizeof(PackedB) * (size_t)b * h);
#pragma omp parallel for schedule(static) num_threads(nt)
  for (long bh = 0; bh < (long)b * h; ++bh) {
    const long bi = bh / h, hi = bh % h;
    float* ktm = (float*)malloc(sizeof(float) * (size_t)d * lk);
    float* vm = (float*)malloc(sizeof(float) * (size_t)lk * d);
    for (int j = 0; j < lk; ++j) {
      const long src = (bi * lk + j) * row + hi * d;
      for (int c = 0; c < d; ++c) ktm[(long)c * lk + j] = k[src + c];
      memcpy(vm + (long)j * d, v + src, sizeof(float) * d);
    }
    kp[bh] = packed_from(ktm, d, lk, lk);
    vp[bh] = packed_from(vm, lk, d, d);
    free(ktm);
    free(vm);
  }
  const int tiles = (lq + ATT_TILE - 1) / ATT_TILE;
#pragma omp parallel num_threads(nt)
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)ATT_TILE * lk);
    float* qt = (float*)malloc(sizeof(float) * (size_t)ATT_TILE * d);
    float* ot = (float*)malloc(sizeof(float) * (size_t)ATT_TILE * d);
#pragma omp for schedule(dynamic)
    for (long task = 0; task < (long)b * h * tiles; ++task) {
      const long bh = task / tiles, bi = bh / h, hi = bh % h;
      const int t = (int)(task % tiles);
      const int r0 = t * ATT_TILE, rows = ATT_TILE < lq - r0 ? ATT_TILE : lq - r0;
      for (int r = 0; r < rows; ++r)
        memcpy(qt + (long)r * d, q + (bi * lq + r0 + r) * row + hi * d, sizeof(float) * d);
      block(&kp[bh], qt, rows, sc);
      for (int r = 0; r < rows; ++r) softmax_scaled(sc + (long)r * lk, lk, scale);
      block(&vp[bh], sc, rows, ot);
      for (int r = 0; r < rows; ++r)
        memcpy(out + (bi * lq + r0 + r) * row + hi * d, ot + (long)r * d, sizeof(float) * d);
    }
    free(sc);
    free(qt);
    free(ot);
  }
  for (long i = 0; i < (long)b * h; ++i) {
    free(kp[i].data);
    free(vp[i].data);
  }
  free(kp);
  free(vp);
}
