/*
 * CPU oracle: plain-C restatement of the reference CPU path for the fused-attention hot path.
 * Test infrastructure only (checker and CPU baseline); the product never links it.
 *
 * Compiled with -ffp-contract=off so that `x*scale + rh + rw` rounds after every operation, as the
 * reference's Rust does (Rust never contracts to FMA). The tile GEMMs live in oracle_gemm.c.
 */
#include "sam_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* oracle_gemm.c */
void oracle_gemm_rows(const float* a, const float* b, float* c, int rows, int k, int n);

static int threads_or_all(int nthreads) {
#ifdef _OPENMP
  return nthreads > 0 ? nthreads : omp_get_max_threads();
#else
  (void)nthreads;
  return 1;
#endif
}

/* Sequential f32 dot product, in the order `tab.iter().zip(q).map(|(a, b)| a * b).sum()` uses
 * (kernels.rs:77, 190). */
static float dot_seq(const float* a, const float* b, int n) {
  float acc = 0.0f;
  for (int c = 0; c < n; ++c) acc += a[c] * b[c];
  return acc;
}

/* kernels.rs:75-83 / 187-196: rh[kh] = q . th[i + h-1 - kh], rw[kw] = q . tw[j + w-1 - kw]. */
static void rel_bias_row(const float* qr, const float* th, const float* tw, int h, int w, int hd, int i, int j,
                         float* rh, float* rw) {
  for (int kh = 0; kh < h; ++kh) rh[kh] = dot_seq(th + (long)(i + h - 1 - kh) * hd, qr, hd);
  for (int kw = 0; kw < w; ++kw) rw[kw] = dot_seq(tw + (long)(j + w - 1 - kw) * hd, qr, hd);
}

/* kernels.rs:84-101 / 197-214: x = s*scale + rh[kh] + rw[kw]; max; exp(x - max); sum; x *= 1/sum. */
static void softmax_relpos_row(const float* s, float* o, const float* rh, const float* rw, int h, int w,
                               float scale) {
  const int n = h * w;
  float mx = -INFINITY;
  for (int kh = 0; kh < h; ++kh) {
    for (int kw = 0; kw < w; ++kw) {
      float v = s[kh * w + kw] * scale;
      v = v + rh[kh];
      v = v + rw[kw];
      o[kh * w + kw] = v;
      mx = fmaxf(mx, v);
    }
  }
  float sum = 0.0f;
  for (int k = 0; k < n; ++k) {
    o[k] = expf(o[k] - mx);
    sum += o[k];
  }
  const float inv = 1.0f / sum;
  for (int k = 0; k < n; ++k) o[k] *= inv;
}

void oracle_relpos_softmax(const float* s, const float* q, const float* table, float* out, long bh, int h, int w,
                           int hd, float scale, int nthreads) {
  const int n = h * w;
  const float* th = table;
  const float* tw = table + (long)(2 * h - 1) * hd;
  const long rows = bh * n;
#pragma omp parallel num_threads(threads_or_all(nthreads))
  {
    float* rh = (float*)malloc(sizeof(float) * (size_t)h);
    float* rw = (float*)malloc(sizeof(float) * (size_t)w);
#pragma omp for schedule(static)
    for (long row = 0; row < rows; ++row) {
      const int rem = (int)(row % n), i = rem / w, j = rem % w;
      rel_bias_row(q + row * hd, th, tw, h, w, hd, i, j, rh, rw);
      softmax_relpos_row(s + row * n, out + row * n, rh, rw, h, w, scale);
    }
    free(rh);
    free(rw);
  }
}

/* kernels.rs:116 (TILE) and 157-221: one task per (head, 32-row query tile). */
#define ORACLE_TILE 32

void oracle_attention_relpos(const float* q, const float* kt, const float* v, const float* table, float* out, long bh,
                             int h, int w, int hd, float scale, int nthreads) {
  const int n = h * w;
  const float* th = table;
  const float* tw = table + (long)(2 * h - 1) * hd;
  const long tiles = (n + ORACLE_TILE - 1) / ORACLE_TILE;
  const long tasks = bh * tiles;
#pragma omp parallel num_threads(threads_or_all(nthreads))
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)ORACLE_TILE * n);
    float* rh = (float*)malloc(sizeof(float) * (size_t)h);
    float* rw = (float*)malloc(sizeof(float) * (size_t)w);
#pragma omp for schedule(dynamic, 1)
    for (long task = 0; task < tasks; ++task) {
      const long b = task / tiles, t = task % tiles;
      const int r0 = (int)(t * ORACLE_TILE);
      const int rows = n - r0 < ORACLE_TILE ? n - r0 : ORACLE_TILE;
      const float* qb = q + (b * n + r0) * (long)hd;
      const float* ktb = kt + b * (long)hd * n;
      const float* vb = v + b * (long)n * hd;
      float* o = out + (b * n + r0) * (long)hd;
      /* scores[rows, n] = q_tile[rows, hd] @ kt[hd, n]   (kernels.rs:181-185) */
      oracle_gemm_rows(qb, ktb, sc, rows, hd, n);
      for (int r = 0; r < rows; ++r) {
        const int row = r0 + r, i = row / w, j = row % w;
        rel_bias_row(qb + (long)r * hd, th, tw, h, w, hd, i, j, rh, rw);
        softmax_relpos_row(sc + (long)r * n, sc + (long)r * n, rh, rw, h, w, scale);
      }
      /* out_tile[rows, hd] = probs[rows, n] @ v[n, hd]   (kernels.rs:216-220) */
      oracle_gemm_rows(sc, vb, o, rows, n, hd);
    }
    free(sc);
    free(rh);
    free(rw);
  }
}

void oracle_qkv_split(const float* y, const float* bias, float* out, long tokens, int n, int nh, int hd, int nthreads) {
  const long c = (long)nh * hd;
  const long plane = tokens * c;
#pragma omp parallel for schedule(static) num_threads(threads_or_all(nthreads))
  for (long t = 0; t < tokens; ++t) {
    const long win = t / n, tok = t % n;
    for (int which = 0; which < 3; ++which) {
      for (int head = 0; head < nh; ++head) {
        const long bhi = win * nh + head;
        for (int d = 0; d < hd; ++d) {
          const long col = which * c + (long)head * hd + d;
          const long dst = which == 1 ? (bhi * hd + d) * n + tok : (bhi * n + tok) * hd + d;
          out[which * plane + dst] = y[t * 3 * c + col] + bias[col];
        }
      }
    }
  }
}

/* kernels.rs:321-362 (cpu::QkvRope; the GPU op sam.cu:210-235 has the same data flow). Per token t, with
 * (x0, x1) = y + bias of a pair in f32: q and k pairs become (x0*cs - x1*sn, x1*cs + x0*sn) with
 * cs, sn the table's even column 2j of row t % n (kernels.rs:348), each product and the difference
 * rounded (this file is built without FMA contraction); v pairs stay x0, x1. out is [3, tokens, c]. */
void oracle_qkv_rope(const float* y, const float* bias, const float* cos_t, const float* sin_t, float* out,
                     long tokens, int n, int nh, int hd, int nthreads) {
  const long c = (long)nh * hd;
#pragma omp parallel for schedule(static) num_threads(threads_or_all(nthreads))
  for (long t = 0; t < tokens; ++t) {
    const long tok = t % n;
    for (int which = 0; which < 3; ++which) {
      const float* src = y + t * 3 * c + which * c;
      const float* b = bias + which * c;
      float* dst = out + which * tokens * c + t * c;
      for (int h = 0; h < nh; ++h) {
        for (int j = 0; j < hd / 2; ++j) {
          const long i = (long)h * hd + 2 * j;
          const float x0 = src[i] + b[i], x1 = src[i + 1] + b[i + 1];
          if (which < 2) {
            const float cs = cos_t[tok * hd + 2 * j], sn = sin_t[tok * hd + 2 * j];
            dst[i] = x0 * cs - x1 * sn;
            dst[i + 1] = x1 * cs + x0 * sn;
          } else {
            dst[i] = x0;
            dst[i + 1] = x1;
          }
        }
      }
    }
  }
}

/* x.floor() as i64 in Rust (kernels.rs:799-800): NaN gives 0 and out-of-range values saturate. The clamp
   to +-2^62 leaves every comparison with a level's size as it is and keeps x0 + 1 from overflowing. */
static long floor_as_index(float xf) {
  if (xf != xf) return 0;
  if (xf >= 4.6e18f) return 1L << 62;
  if (xf <= -4.6e18f) return -(1L << 62);
  return (long)xf;
}

void oracle_deform_attn(const float* value, const float* loc, const float* attn, float* out, int b, int s, int q, int h,
                        int d, int l, int p, const int* shapes, int nthreads) {
  long starts[64];
  long acc = 0;
  for (int li = 0; li < l; ++li) {
    starts[li] = acc;
    acc += (long)shapes[2 * li] * shapes[2 * li + 1];
  }
  const long bq_total = (long)b * q;
#pragma omp parallel for schedule(static) num_threads(threads_or_all(nthreads))
  for (long bq = 0; bq < bq_total; ++bq) {
    const long bi = bq / q;
    float* o = out + bq * (long)h * d;
    memset(o, 0, sizeof(float) * (size_t)h * d);
    for (int hi = 0; hi < h; ++hi) {
      float* a = o + (long)hi * d;
      for (int li = 0; li < l; ++li) {
        const int hl = shapes[2 * li], wl = shapes[2 * li + 1];
        for (int pi = 0; pi < p; ++pi) {
          const long base = ((bq * h + hi) * l + li) * p + pi;
          const float wgt = attn[base];
          const float x = loc[base * 2] * (float)wl - 0.5f;
          const float y = loc[base * 2 + 1] * (float)hl - 0.5f;
          const float xf = floorf(x), yf = floorf(y);
          const long x0 = floor_as_index(xf), y0 = floor_as_index(yf);
          const float fx = x - xf, fy = y - yf;
          for (int c = 0; c < 4; ++c) {
            const long xx = x0 + (c & 1), yy = y0 + (c >> 1);
            if (xx < 0 || xx >= wl || yy < 0 || yy >= hl) continue;
            /* kernels.rs:805: w * wx * wy, left to right */
            float wt = wgt * ((c & 1) ? fx : 1.0f - fx);
            wt = wt * ((c >> 1) ? fy : 1.0f - fy);
            const float* src = value + ((bi * s + starts[li] + yy * wl + xx) * h + hi) * (long)d;
            for (int e = 0; e < d; ++e) a[e] += wt * src[e];
          }
        }
      }
    }
  }
}

/* candle's softmax_last_dim on CPU: max, exp(x - max), sum, x / sum. */
static void softmax_div(float* x, int n) {
  float mx = -INFINITY;
  for (int k = 0; k < n; ++k) mx = fmaxf(mx, x[k]);
  float sum = 0.0f;
  for (int k = 0; k < n; ++k) {
    x[k] = expf(x[k] - mx);
    sum += x[k];
  }
  for (int k = 0; k < n; ++k) x[k] = x[k] / sum;
}

/* Deform::forward between its input projections and deform_attn (dino/mod.rs:166-178):
 *   attn = softmax over the l*p points of each (b, q, h) of the logits [b,q,h,l,p] (:167);
 *   loc from the offsets off [b,q,h,l,p,2] and the reference points refs [b,q,l,ncoord]:
 *     ncoord 2 (encoder, :169-173): loc = ref + off / (W_l, H_l);
 *     ncoord 4 (decoder, :174-178): loc = xy + ((off * (1/p)) * wh) * 0.5, where candle's `off / p`
 *       is Tensor::affine(1/p, 0) (x * mul + add) and `.affine(0.5, 0.0)` is x * 0.5 + 0.
 * Every step is one f32 rounding, left to right, as the candle ops compute them. The candle ops run in
 * the query's dtype, so with round_dt 1 (f16) or 2 (bf16) each step's result, the softmax output and
 * the level sizes (`norm`, converted with to_dtype at :170) are also rounded to that dtype. */
static float round_bf16_scalar(float x);
static float round_to_f16(float x);
static float round_dt_scalar(float x, int dt) {
  return dt == 1 ? round_to_f16(x) : dt == 2 ? round_bf16_scalar(x) : x;
}

void oracle_deform_prep(const float* off, const float* logits, const float* refs, float* loc, float* attn, int b,
                        int q, int h, int l, int p, int ncoord, const int* shapes, int round_dt, int nthreads) {
  const long pairs = (long)b * q * h;
  const int npt = l * p;
  const float inv_p = (float)(1.0 / (double)p);
#define R(x) round_dt_scalar((x), round_dt)
#pragma omp parallel for schedule(static) num_threads(threads_or_all(nthreads))
  for (long pr = 0; pr < pairs; ++pr) {
    const long bq = pr / h;
    float* a = attn + pr * npt;
    for (int j = 0; j < npt; ++j) a[j] = logits[pr * npt + j];
    softmax_div(a, npt);
    for (int j = 0; j < npt; ++j) a[j] = R(a[j]);
    for (int j = 0; j < npt; ++j) {
      const int li = j / p;
      const float* r = refs + (bq * l + li) * ncoord;
      const float ox = off[(pr * npt + j) * 2], oy = off[(pr * npt + j) * 2 + 1];
      float* o = loc + (pr * npt + j) * 2;
      if (ncoord == 2) {
        o[0] = R(r[0] + R(ox / R((float)shapes[2 * li + 1])));
        o[1] = R(r[1] + R(oy / R((float)shapes[2 * li])));
      } else {
        const float tx = R(ox * inv_p + 0.0f), ty = R(oy * inv_p + 0.0f);
        const float ux = R(tx * r[2]), uy = R(ty * r[3]);
        o[0] = R(r[0] + R(ux * 0.5f + 0.0f));
        o[1] = R(r[1] + R(uy * 0.5f + 0.0f));
      }
    }
  }
#undef R
}

void oracle_sdpa(const float* q, const float* k, const float* v, float* out, int b, int h, int lq, int lk, int d,
                 int nthreads) {
  const float scale = powf((float)d, -0.5f);
  const long heads = (long)b * h;
  const long tiles = (lq + ORACLE_TILE - 1) / ORACLE_TILE;
#pragma omp parallel num_threads(threads_or_all(nthreads))
  {
    float* kt = (float*)malloc(sizeof(float) * (size_t)d * lk);
    float* sc = (float*)malloc(sizeof(float) * (size_t)ORACLE_TILE * lk);
    long cur = -1;
#pragma omp for schedule(static)
    for (long task = 0; task < heads * tiles; ++task) {
      const long bh = task / tiles, t = task % tiles;
      const float* kb = k + bh * (long)lk * d;
      if (bh != cur) { /* k.transpose(2, 3).contiguous() (nn.rs:28) */
        for (int j = 0; j < lk; ++j)
          for (int c = 0; c < d; ++c) kt[(long)c * lk + j] = kb[(long)j * d + c];
        cur = bh;
      }
      const int r0 = (int)(t * ORACLE_TILE);
      const int rows = lq - r0 < ORACLE_TILE ? lq - r0 : ORACLE_TILE;
      oracle_gemm_rows(q + (bh * lq + r0) * (long)d, kt, sc, rows, d, lk);
      for (int r = 0; r < rows; ++r) {
        float* row = sc + (long)r * lk;
        for (int j = 0; j < lk; ++j) row[j] = row[j] * scale; /* (q k^T) * scale (nn.rs:28) */
        softmax_div(row, lk);
      }
      oracle_gemm_rows(sc, v + bh * (long)lk * d, out + (bh * lq + r0) * (long)d, rows, lk, d);
    }
    free(kt);
    free(sc);
  }
}

/* sam3/nn.rs:26-34 with Some(mask): s = (q k^T) * scale, then s.broadcast_add(mask) (:29-32), softmax
 * over the keys, times v. The mask is read through element strides sm (batch, head, query, key); a
 * stride of 0 broadcasts. A row whose keys are all -inf comes out NaN, as candle's softmax gives. */
void oracle_sdpa_mask(const float* q, const float* k, const float* v, const float* mask, const long* sm, float* out,
                      int b, int h, int lq, int lk, int d, int nthreads) {
  const float scale = powf((float)d, -0.5f);
  const long heads = (long)b * h;
  const long tiles = (lq + ORACLE_TILE - 1) / ORACLE_TILE;
#pragma omp parallel num_threads(threads_or_all(nthreads))
  {
    float* kt = (float*)malloc(sizeof(float) * (size_t)d * lk);
    float* sc = (float*)malloc(sizeof(float) * (size_t)ORACLE_TILE * lk);
    long cur = -1;
#pragma omp for schedule(static)
    for (long task = 0; task < heads * tiles; ++task) {
      const long bh = task / tiles, t = task % tiles;
      const long bi = bh / h, hi = bh % h;
      const float* kb = k + bh * (long)lk * d;
      if (bh != cur) {
        for (int j = 0; j < lk; ++j)
          for (int c = 0; c < d; ++c) kt[(long)c * lk + j] = kb[(long)j * d + c];
        cur = bh;
      }
      const int r0 = (int)(t * ORACLE_TILE);
      const int rows = lq - r0 < ORACLE_TILE ? lq - r0 : ORACLE_TILE;
      oracle_gemm_rows(q + (bh * lq + r0) * (long)d, kt, sc, rows, d, lk);
      for (int r = 0; r < rows; ++r) {
        float* row = sc + (long)r * lk;
        const float* mrow = mask + bi * sm[0] + hi * sm[1] + (long)(r0 + r) * sm[2];
        for (int j = 0; j < lk; ++j) row[j] = row[j] * scale + mrow[(long)j * sm[3]];
        softmax_div(row, lk);
      }
      oracle_gemm_rows(sc, v + bh * (long)lk * d, out + (bh * lq + r0) * (long)d, rows, lk, d);
    }
    free(kt);
    free(sc);
  }
}

void oracle_mha_blhd(const float* q, const float* k, const float* v, float* out, int b, int lq, int lk, int h, int d,
                     float scale, int nthreads) {
  const long e = (long)h * d;
  const long tasks = (long)b * lq * h;
#pragma omp parallel num_threads(threads_or_all(nthreads))
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)lk);
#pragma omp for schedule(static)
    for (long task = 0; task < tasks; ++task) {
      const long bi = task / ((long)lq * h);
      const long qi = (task / h) % lq, head = task % h;
      const float* qv = q + (bi * lq + qi) * e + head * d;
      float* o = out + (bi * lq + qi) * e + head * d;
      float mx = -INFINITY;
      for (int j = 0; j < lk; ++j) {
        const float* kv = k + (bi * lk + j) * e + head * d;
        const float s = dot_seq(qv, kv, d) * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
      }
      float sum = 0.0f;
      for (int j = 0; j < lk; ++j) {
        sc[j] = expf(sc[j] - mx);
        sum += sc[j];
      }
      const float inv = 1.0f / sum;
      for (int c = 0; c < d; ++c) o[c] = 0.0f;
      for (int j = 0; j < lk; ++j) {
        const float pj = sc[j] * inv;
        const float* vv = v + (bi * lk + j) * e + head * d;
        for (int c = 0; c < d; ++c) o[c] += pj * vv[c];
      }
    }
    free(sc);
  }
}

void oracle_rope_tables(int side, float scale, int hd, float theta, float* cos_out, float* sin_out) {
  const int sp = hd / 2;
  float inv[1024];
  for (int i = 0; i < sp / 2; ++i) inv[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)sp);
  for (int r = 0; r < side; ++r) {
    for (int c = 0; c < side; ++c) {
      const long t = (long)r * side + c;
      for (int j = 0; j < sp; ++j) {
        const float pos = j < sp / 2 ? (float)c * scale : (float)r * scale;
        const float f = j < sp / 2 ? inv[j] : inv[j - sp / 2];
        const float a = pos * f;
        for (int kk = 0; kk < 2; ++kk) { /* repeat_interleave(2) */
          cos_out[t * hd + 2 * j + kk] = cosf(a);
          sin_out[t * hd + 2 * j + kk] = sinf(a);
        }
      }
    }
  }
}

void oracle_rope(const float* x, const float* cos_t, const float* sin_t, float* out, long l, int d) {
  for (long t = 0; t < l; ++t) {
    const float* xr = x + t * d;
    for (int c = 0; c < d; c += 2) {
      const float x0 = xr[c], x1 = xr[c + 1];
      /* x*cos + rot*sin with rot = [-x1, x0] (video.rs:110-112) */
      float a = x0 * cos_t[t * d + c];
      float b = -x1 * sin_t[t * d + c];
      out[t * d + c] = a + b;
      a = x1 * cos_t[t * d + c + 1];
      b = x0 * sin_t[t * d + c + 1];
      out[t * d + c + 1] = a + b;
    }
  }
}

void oracle_rope_attention(const float* q, const float* k, const float* v, const float* cos_t, const float* sin_t,
                           int trows, float* out, int lq, int mk, int d, int n_exclude, int nthreads) {
  float* qr = (float*)malloc(sizeof(float) * (size_t)lq * d);
  float* kr = (float*)malloc(sizeof(float) * (size_t)mk * d);
  oracle_rope(q, cos_t, sin_t, qr, lq, d);
  const int rot = mk - n_exclude;
  for (int r0 = 0; r0 < rot; r0 += trows) { /* tables tiled `rot / trows` times (video.rs:137-139) */
    const int len = rot - r0 < trows ? rot - r0 : trows;
    oracle_rope(k + (long)r0 * d, cos_t, sin_t, kr + (long)r0 * d, len, d);
  }
  memcpy(kr + (long)rot * d, k + (long)rot * d, sizeof(float) * (size_t)n_exclude * d);
  oracle_sdpa(qr, kr, v, out, 1, 1, lq, mk, d, nthreads);
  free(qr);
  free(kr);
}

/* image_proc.rs:57-96 (resize_normalize): PIL-style antialiased triangle filter. */
static float tri_weight(float x) {
  x = fabsf(x);
  return x < 1.0f ? 1.0f - x : 0.0f;
}

/* image_proc.rs:57-96: one task per (channel, output row); rows >= nh and columns >= nw stay 0. Every
 * step rounds in f32 in the reference's order (this file is built without FMA contraction): the tap
 * span from truncating casts, the weight sums in tap order, r = sum_xx w(xx) * px row by row,
 * acc += wy * r, then (acc / (wsx * wsy) - mean) / std. */
void oracle_preprocess(const uint8_t* img, int h, int w, int nh, int nw, int size, const float* mean,
                       const float* std_dev, float* out, int nthreads) {
  const float sx = (float)w / (float)nw, sy = (float)h / (float)nh;
  const float fx = sx > 1.0f ? sx : 1.0f, fy = sy > 1.0f ? sy : 1.0f;
  memset(out, 0, sizeof(float) * 3 * (size_t)size * size);
  const long rows = 3L * size;
#pragma omp parallel for schedule(dynamic, 8) num_threads(threads_or_all(nthreads))
  for (long i = 0; i < rows; ++i) {
    const int c = (int)(i / size), y = (int)(i % size);
    if (y >= nh) continue;
    float* row = out + i * size;
    const float cy = ((float)y + 0.5f) * sy;
    long y0 = (long)(cy - fy + 0.5f);
    if (y0 < 0) y0 = 0;
    long y1 = (long)(cy + fy + 0.5f);
    if (y1 > h) y1 = h;
    float wsy = 0.0f;
    for (long yy = y0; yy < y1; ++yy) wsy += tri_weight(((float)yy + 0.5f - cy) / fy);
    for (int x = 0; x < nw && x < size; ++x) {
      const float cx = ((float)x + 0.5f) * sx;
      long x0 = (long)(cx - fx + 0.5f);
      if (x0 < 0) x0 = 0;
      long x1 = (long)(cx + fx + 0.5f);
      if (x1 > w) x1 = w;
      float wsx = 0.0f;
      for (long xx = x0; xx < x1; ++xx) wsx += tri_weight(((float)xx + 0.5f - cx) / fx);
      float acc = 0.0f;
      for (long yy = y0; yy < y1; ++yy) {
        float r = 0.0f;
        for (long xx = x0; xx < x1; ++xx)
          r += tri_weight(((float)xx + 0.5f - cx) / fx) * (float)img[(yy * w + xx) * 3 + c];
        acc += tri_weight(((float)yy + 0.5f - cy) / fy) * r;
      }
      row[x] = (acc / (wsx * wsy) - mean[c]) / std_dev[c];
    }
  }
}

/* kernels.rs:618-640 (cpu::BiasResidual): out[i] = res[i] + y[i] + b[i % c], left to right in f32. */
void oracle_bias_residual(const float* res, const float* y, const float* b, float* out, long total, int c) {
  for (long i = 0; i < total; ++i) out[i] = res[i] + y[i] + b[i % c];
}

/* kernels.rs:642-663 (cpu::BiasGelu): x = y[i] + b[i % c]; out = 0.5 * x * (1 + erf(x * FRAC_1_SQRT_2)).
 * The reference calls the `libm` crate's erff (a port of musl's); this calls the C library's erff.
 * Both are faithful to within an ulp, so the two can differ in the last bit of an element. */
void oracle_bias_gelu(const float* y, const float* b, float* out, long total, int c) {
  for (long i = 0; i < total; ++i) {
    const float x = y[i] + b[i % c];
    out[i] = 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
  }
}

/* IEEE binary16 round-to-nearest-even, returned as f32 (gcc has no _Float16 on x86 here). */
static float round_to_f16(float x) {
  if (isnan(x)) return x;
  const float ax = fabsf(x);
  if (ax >= 65520.0f) return copysignf(INFINITY, x); /* halfway between 65504 and 2^16 rounds up */
  float quantum;
  if (ax < 6.103515625e-05f) {
    quantum = 5.9604644775390625e-08f; /* subnormal spacing 2^-24 */
  } else {
    int e;
    frexpf(ax, &e); /* ax in [2^(e-1), 2^e): 11 significant bits -> spacing 2^(e-11) */
    quantum = ldexpf(1.0f, e - 11);
  }
  return copysignf(nearbyintf(ax / quantum) * quantum, x);
}

void oracle_round_f16(float* x, long n) {
  for (long i = 0; i < n; ++i) x[i] = round_to_f16(x[i]);
}

/* bfloat16 round-to-nearest-even (NaN stays NaN), returned as f32. */
static float round_bf16_scalar(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  if (isnan(x)) {
    b = (b | 0x00400000u) & 0xffff0000u;
  } else {
    b = (b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u;
  }
  memcpy(&x, &b, 4);
  return x;
}

void oracle_round_bf16(float* x, long n) {
  for (long i = 0; i < n; ++i) x[i] = round_bf16_scalar(x[i]);
}

static uint64_t splitmix64(uint64_t* st) {
  uint64_t z = (*st += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void oracle_randn(unsigned long long seed, float* out, long n, float mean, float std) {
  uint64_t st = seed;
  for (long i = 0; i < n; i += 2) {
    /* two uniforms in (0, 1]: 53-bit mantissas */
    const double u1 = ((double)(splitmix64(&st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(splitmix64(&st) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double a = 6.283185307179586 * u2;
    out[i] = (float)(mean + std * r * cos(a));
    if (i + 1 < n) out[i + 1] = (float)(mean + std * r * sin(a));
  }
}
