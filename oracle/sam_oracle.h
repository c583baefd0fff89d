/*
 * CPU oracle for the fused-attention hot path: a plain-C restatement of the reference's
 * CPU algorithms (sam-rs `src/kernels.rs`, `src/sam3/nn.rs`, `src/sam3/video.rs`, `src/sam3/vision.rs`), used ONLY as the checker.
 *
 * This is test infrastructure. Only the test suite, the smoke check and the CPU-baseline leg of the
 * benchmark load it, and never as the thing that is measured or shipped. The product path
 * (libsam_hip.so) does not link, call or fall back to anything here.
 *
 * All arrays are contiguous, row-major f32 (the reference's CPU ops take f32; its bf16 path rounds
 * operands to bf16 inside its GEMMs, restated in oracle_bf16.c). `nthreads` <= 0
 * means "all OpenMP threads". Every function cites the reference lines it restates.
 *
 * Parity pins (see tests/test_oracle.py): each function is checked against an independent float64
 * formulation (textbook SAM decomposed rel-pos, torch grid_sample, torch sdpa, complex-number RoPE,
 * PIL's float-mode bilinear resize),
 * closed forms and brute force on tiny inputs; none is left unpinned.
 */
#ifndef SAM_ORACLE_H
#define SAM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kernels.rs:62-105 (cpu::RelposSoftmax). s [bh, n, n], q [bh, n, hd], table [(2h-1)+(2w-1), hd]
 * -> out [bh, n, n] with n = h*w. */
void oracle_relpos_softmax(const float* s, const float* q, const float* table, float* out, long bh, int h, int w,
                           int hd, float scale, int nthreads);

/* kernels.rs:131-224, exact-f32 branch 181-220 (cpu::TiledAttention with cpu_gemm disabled).
 * q [bh, n, hd], kt [bh, hd, n], v [bh, n, hd], table as above -> out [bh, n, hd]. */
void oracle_attention_relpos(const float* q, const float* kt, const float* v, const float* table, float* out, long bh,
                             int h, int w, int hd, float scale, int nthreads);

/* kernels.rs:239-263 (cpu::QkvSplit). y [tokens, 3*nh*hd], bias [3*nh*hd] -> out [3, bh*n*hd] holding
 * q [bh,n,hd], kT [bh,hd,n], v [bh,n,hd] back to back, bh = tokens/n*nh. */
void oracle_qkv_split(const float* y, const float* bias, float* out, long tokens, int n, int nh, int hd, int nthreads);

/* kernels.rs:321-362 (cpu::QkvRope). y [tokens, 3*nh*hd], bias [3*nh*hd], cos/sin [n, hd] -> out
 * [3, tokens, nh*hd]: bias added, q and k pairs rotated by row t % n of the tables (even columns). */
void oracle_qkv_rope(const float* y, const float* bias, const float* cos_t, const float* sin_t, float* out,
                     long tokens, int n, int nh, int hd, int nthreads);

/* kernels.rs:776-818 (cpu::DeformAttn). value [b,s,h,d], loc [b,q,h,l,p,2], attn [b,q,h,l,p],
 * shapes = l (height,width) pairs -> out [b,q,h*d]. */
void oracle_deform_attn(const float* value, const float* loc, const float* attn, float* out, int b, int s, int q, int h,
                        int d, int l, int p, const int* shapes, int nthreads);

/* dino/mod.rs:166-178 (Deform::forward after its input projections): softmax of logits [b,q,h,l,p]
 * over l*p -> attn; offsets off [b,q,h,l,p,2] and refs [b,q,l,ncoord] (ncoord 2: encoder, 4: decoder)
 * -> loc [b,q,h,l,p,2]; shapes = l (height,width) pairs. */
void oracle_deform_prep(const float* off, const float* logits, const float* refs, float* loc, float* attn, int b,
                        int q, int h, int l, int p, int ncoord, const int* shapes, int round_dt, int nthreads);

/* sam3/nn.rs:26-34 (sdpa, mask = None) on [b, h, l, d] tensors: softmax(q k^T * d^-0.5) v. */
void oracle_sdpa(const float* q, const float* k, const float* v, float* out, int b, int h, int lq, int lk, int d,
                 int nthreads);

/* kernels.rs:502-548 (cpu::Mha) semantics on the [B, L, H, D] layout that flash attention takes
 * (kernels.rs:416-434): one task per (batch, query, head), scale = d^-0.5. */
void oracle_mha_blhd(const float* q, const float* k, const float* v, float* out, int b, int lq, int lk, int h, int d,
                     float scale, int nthreads);

/* sam3/vision.rs:26-46 (rope_tables_hd): cos/sin [side*side, hd]. */
void oracle_rope_tables(int side, float scale, int hd, float theta, float* cos_out, float* sin_out);

/* sam3/video.rs:106-113 (rope): x [l, d] -> x*cos + rot(x)*sin, rot([x0,x1]) = [-x1, x0]; cos/sin [l, d]. */
void oracle_rope(const float* x, const float* cos_t, const float* sin_t, float* out, long l, int d);

/* sam3/video.rs:129-145 (RopeAttn::forward after the projections): q [lq, d] rotated with the
 * tables, the first mk - n_exclude keys rotated with the tables tiled to their length, the last
 * n_exclude keys left as they are, then sdpa with one head. cos/sin have `trows` rows. */
void oracle_rope_attention(const float* q, const float* k, const float* v, const float* cos_t, const float* sin_t,
                           int trows, float* out, int lq, int mk, int d, int n_exclude, int nthreads);

/* image_proc.rs:57-96 (resize_normalize; the CPU side of image_proc::prepare / prepare_square,
 * image_proc.rs:21-53): antialiased triangle-filter resize of img (u8 [h, w, 3]) to nh x nw, then
 * (x - mean[c]) / std[c], zero padded into out [3, size, size]. */
void oracle_preprocess(const unsigned char* img, int h, int w, int nh, int nw, int size, const float* mean,
                       const float* std_dev, float* out, int nthreads);

/* kernels.rs:618-640 (cpu::BiasResidual): out = res + y + b[i % c]. */
void oracle_bias_residual(const float* res, const float* y, const float* b, float* out, long total, int c);

/* kernels.rs:642-663 (cpu::BiasGelu): out = gelu_erf(y + b[i % c]). */
void oracle_bias_gelu(const float* y, const float* b, float* out, long total, int c);

/* Round-to-nearest-even conversions used to pre-round inputs to the kernel dtype
 * (the reference test does the same, tests/kernels.rs:28-31). */
void oracle_round_f16(float* x, long n);
void oracle_round_bf16(float* x, long n);

/* SplitMix64 + Box-Muller normal generator: the one seeded source of synthetic inputs. */
void oracle_randn(unsigned long long seed, float* out, long n, float mean, float std);

#ifdef __cplusplus
}
#endif
/* The reference's default CPU path on AVX-512 BF16 machines (cpu_gemm.rs, kernels.rs:139-179), in
 * oracle_bf16.c. Call only when oracle_bf16_available() is nonzero. */
int oracle_bf16_available(void);
void oracle_bf16_round(const float* x, uint16_t* out, long n);
void oracle_bf16_exp(const float* x, float* y, long n);
void oracle_bf16_matmul(const float* x, const float* w, float* c, int m, int k, int n, int nthreads);
void oracle_bf16_attention_relpos(const float* q, const float* kt, const float* v, const float* table, float* out,
                                  long bh, int h, int w, int hd, float scale, int nthreads);
void oracle_bf16_flash_attention(const float* q, const float* k, const float* v, float* out, int b, int lq, int lk,
                                 int h, int d, float scale, int nthreads);

#endif
