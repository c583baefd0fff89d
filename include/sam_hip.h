/*
 * sam_hip.h - C ABI of libsam_hip.so, the MI355X (gfx950) fused-attention hot path of sam-rs.
 *
 * Each entry point replaces one GPU path of the reference's `src/kernels.rs` (file:line cited per
 * function). Conventions, shared by all entry points:
 *   - plain device pointers (hipMalloc'd or any HIP-visible device memory), 16-byte aligned,
 *     contiguous row-major in the layouts the reference uses; the caller allocates every buffer;
 *   - dtype: 0 = f32, 1 = f16, 2 = bf16 (the three the reference's `by_dtype!` accepts,
 *     kernels.rs:1086-1095); every tensor argument of one call has that dtype;
 *   - stream: a hipStream_t passed as void* (NULL = the default stream); launches are asynchronous,
 *     exactly as the reference's are on candle's CUDA stream;
 *   - return 0 on success, nonzero on error; sam_hip_last_error() then returns a message (per thread);
 *   - no global mutable state beyond each kernel's once-per-device LDS opt-in (an atomic flag word)
 *     and the workspace array of sam_hip_flash_attn_noalloc; safe to call from many threads (except
 *     that overlapping sam_hip_flash_attn_noalloc calls on one GPU share that array).
 */
#ifndef SAM_HIP_H
#define SAM_HIP_H

#ifdef __cplusplus
extern "C" {
#endif

enum sam_hip_status {
  SAM_HIP_OK = 0,
  SAM_HIP_EINVAL = 1,      /* a null pointer or an inconsistent size */
  SAM_HIP_EDTYPE = 2,      /* dtype not in {0, 1, 2} or not supported by this entry point */
  SAM_HIP_EUNSUPPORTED = 3, /* a shape beyond this kernel's limits (message says which) */
  SAM_HIP_EHIP = 4,        /* the HIP runtime reported an error at launch */
  SAM_HIP_EDISABLED = 5    /* the HIP path is switched off (sam_hip_set_enabled); nothing was done */
};

/*
 * Process-wide switch of the HIP path, the counterpart of the reference's cpu_gemm::set_enabled /
 * cpu_gemm::enabled (cpu_gemm.rs:11, 25-32), which main.rs:117-125 turns off for --f32. On by default;
 * off from load time when the environment variable SAM_HIP_DISABLE is set to anything but "" or "0".
 * While it is off, every compute entry point (all but the size queries, sam_hip_last_error,
 * sam_hip_abi_version and these two) returns SAM_HIP_EDISABLED before reading any argument or
 * touching a device, and the caller takes the reference's own path: the Rust binding maps that code
 * to Ok(None) in the Option-returning ops and to the tensor path elsewhere. Takes effect for calls
 * that start after it returns; safe to call from any thread.
 */
void sam_hip_set_enabled(int on);
int sam_hip_enabled(void);

/*
 * Fused SAM ViT attention with the decomposed relative-position bias:
 *   out[b, r, :] = softmax_k(scale * q[b,r].kt[b,:,k] + q[b,r].Th[i-kh+h-1] + q[b,r].Tw[j-kw+w-1]) . v[b,k,:]
 * with r = i*w + j, k = kh*w + kw, Th = table rows [0, 2h-1), Tw = rows [2h-1, 2h-1 + 2w-1).
 *   q [bh, h*w, hd], kt [bh, hd, h*w] (the key matrix transposed, as qkv_split writes it),
 *   v [bh, h*w, hd], table [(2h-1) + (2w-1), hd], out [bh, h*w, hd].
 * Replaces, in one kernel, the reference's GPU sequence bmm(q, kT) -> relpos_softmax -> bmm(P, v)
 * (sam1/encoder.rs:79-82; kernels.rs:12-43, 919-924, 1108-1149) and is the GPU counterpart of
 * attention_relpos_cpu (kernels.rs:899-906).
 * Limits: f16/bf16 1 <= h, w <= 128, hd % 8 == 0 and hd <= 128; f32 1 <= h, w <= 64, hd % 4 == 0 and
 * hd <= 128. Which kernel runs (f16/bf16) is chosen for speed only; every shape within the limits gets
 * the same result to the same tolerance. Dedicated kernels take SAM's two shapes at hd 64 and 80:
 * windows with 13 <= h <= 16 and an even w <= 16, and the 64-column global grid (w == 64, h <= 64) when
 * 2^-6 <= scale * log2(e) <= 4 (SAM's hd^-0.5 * log2(e) is 0.16-0.18). Every other shape or scale up to
 * 64 x 64 runs on the general kernel, and grids past 64 rows or columns on a kernel that walks them in
 * 64-column passes, each at a lower speed. The reference's own GPU sequence stops at h*w <= 8192 (the
 * relpos_softmax row limit); here the scores stay on chip, so every h, w <= 128 runs. In f32, hd 64 has
 * its own window kernel (w <= 16, h <= 16, h*w <= 256) and global kernel (w == 64); other f32 shapes run
 * on the general f32 kernel.
 */
int sam_hip_attn_relpos(const void* q, const void* kt, const void* v, const void* table, void* out, int dtype,
                        int bh, int h, int w, int hd, float scale, void* stream);

/*
 * Softmax over materialised scores with the decomposed relative-position bias:
 *   out[b, r, k] = softmax_k(scale * s[b, r, k] + q[b,r].Th[i-kh+h-1] + q[b,r].Tw[j-kw+w-1])
 *   s [bh, h*w, h*w], q [bh, h*w, hd], table as above -> out [bh, h*w, h*w]; rows = bh*h*w.
 * The literal drop-in for kernels::relpos_softmax (kernels.rs:12-43; GPU op kernels.rs:1108-1149,
 * sam.cu:44-96) for callers that hold the score matrix. Limits: h, w <= 128 (rows of up to 16384
 * keys), hd <= 256. The reference's GPU kernel stops at h*w <= 8192 (kernels.rs:1078-1083) and takes
 * its tensor path past it (kernels.rs:20-42); a binding that keeps that split bit for bit keeps its
 * guard, one that wants the GPU past 8192 keys drops it (same formula, f32 arithmetic as below 8192).
 */
int sam_hip_relpos_softmax(const void* s, const void* q, const void* table, void* out, int dtype, long rows, int h,
                           int w, int hd, float scale, void* stream);

/*
 * qkv projection output to the attention layout, bias added:
 *   y [tokens, 3*nh*hd] (columns (qkv, head, d)), bias [3*nh*hd] -> out [3, bh*n*hd] holding
 *   q [bh, n, hd], kT [bh, hd, n], v [bh, n, hd] back to back, bh = tokens/n * nh.
 * Replaces kernels::qkv_split (kernels.rs:872-894; GPU op sam.cu:111-128). Each element is
 * round(y + bias) as the reference computes it. Limits: tokens % n == 0, hd <= 256.
 */
int sam_hip_qkv_split(const void* y, const void* bias, void* out, int dtype, long tokens, int n, int nh, int hd,
                      void* stream);

/*
 * qkv_split on the unpadded token grid, with the window partition in it:
 *   y [batch*gh*gw, 3*nh*hd] (the qkv projection of the grid tokens, row (b*gh + r)*gw + c), bias as
 *   above -> out [3, bh*n*hd] as sam_hip_qkv_split writes it for the windows of the grid zero-padded to
 *   multiples of ws: n = ws*ws, bh = batch * ceil(gh/ws) * ceil(gw/ws) * nh, window (b, wi, wj) in that
 *   order, token (ti, tj) of it at grid (wi*ws + ti, wj*ws + tj).
 * The reference partitions the normalised tokens first (sam1/encoder.rs:129-137) and runs the qkv
 * linear on the padded windows, so a padding token's projection is 0 and its q, k and v are the bias
 * alone; this entry point writes exactly that, so the linear can run on the gh*gw grid tokens only.
 * No reference entry point of its own: the composition of window_partition and kernels::qkv_split
 * (kernels.rs:872-894). Limits: hd <= 256, ws <= 256, gh, gw <= 4096; 16-byte aligned pointers.
 */
int sam_hip_qkv_split_grid(const void* y, const void* bias, void* out, int dtype, int batch, int gh, int gw, int ws,
                           int nh, int hd, void* stream);

/*
 * The attention output back on the grid: ctx [bh, ws*ws, hd] in the window order of
 * sam_hip_qkv_split_grid -> out [batch, gh, gw, nh*hd], heads merged (the transpose and reshape of
 * sam1/encoder.rs:83) and the windows put back without their padding (window_unpartition,
 * sam1/encoder.rs:140-143). A copy: out holds ctx's values. No reference entry point of its own.
 * Limits: ws <= 256, gh, gw <= 4096; 16-byte aligned pointers.
 */
int sam_hip_window_merge(const void* ctx, void* out, int dtype, int batch, int gh, int gw, int ws, int nh, int hd,
                         void* stream);

/*
 * Multi-scale deformable attention (Grounding DINO), forward:
 *   out[b, q, h*d + c] = sum_{l,p} attn[b,q,h,l,p] * bilinear(value_l[b,:,h,c], (x*W_l - 0.5, y*H_l - 0.5))
 * with (x, y) = loc[b,q,h,l,p,:], zero padding outside each level.
 *   value [b, s, h, d] (levels concatenated), loc [b, q, h, l, p, 2], attn [b, q, h, l, p] -> out [b, q, h*d].
 *   shapes: host array of 2*l ints, (height, width) of each level; their pixels must add up to s.
 * Replaces kernels::deform_attn (kernels.rs:824-835) on the GPU (cuda::DeformAttn, kernels.rs:1162-1194;
 * sam.cu:305-350). Limits: l <= 4 (the reference's GPU error, kernels.rs:1175-1177), l*p <= 64,
 * b*s*h*d < 2^31.
 */
int sam_hip_deform_attn(const void* value, const void* loc, const void* attn, void* out, int dtype, int b, int s,
                        int q, int h, int d, int l, int p, const int* shapes, void* stream);

/*
 * Grounding DINO's Deform::forward between its input projections and its output projection
 * (dino/mod.rs:161-181 without the four Linear layers), in one launch:
 *   attn = softmax over the l*p points of each (b, q, h) of logits [b, q, h, l, p]          (:167)
 *   loc  = refs[b,q,l,0:2] + offsets / (W_l, H_l)                       ncoord 2, encoder (:169-173)
 *   loc  = refs[b,q,l,0:2] + ((offsets * (1/p)) * refs[b,q,l,2:4]) * 0.5  ncoord 4, decoder (:174-178)
 *   out  = deform_attn(value, loc, attn, shapes)                                             (:179)
 * with offsets [b, q, h, l, p, 2] (the sampling_offsets projection reshaped), refs [b, q, l, ncoord].
 * loc and attn are formed per point in f32 and never stored. Limits and alignment as
 * sam_hip_deform_attn; ncoord is 2 or 4.
 */
int sam_hip_deform_core(const void* value, const void* offsets, const void* logits, const void* refs, void* out,
                        int dtype, int b, int s, int q, int h, int d, int l, int p, int ncoord, const int* shapes,
                        void* stream);

/*
 * SAM image preprocessing: antialiased triangle-filter resize (PIL's bilinear) of an RGB u8 image
 * img [h, w, 3] to nh x nw, then (x - mean[c]) / std_dev[c], zero padded at the bottom and right into
 * out [3, size, size] of `dtype`. mean and std_dev are host arrays of 3 floats.
 * Replaces kernels::preprocess (kernels.rs:1063-1070; cuda::Preprocess, kernels.rs:1396-1430;
 * sam.cu:162-204), the GPU side of image_proc::prepare / prepare_square (image_proc.rs:21-53), with
 * the arithmetic of their CPU side image_proc::resize_normalize (image_proc.rs:57-96): f32 output
 * equals it bit for bit, f16 / bf16 output is that value rounded to nearest even.
 * Limits: 1 <= nh, nw <= size; std_dev[c] != 0; at most 64 filter taps per output pixel and axis
 * (w / nw and h / nh at most 31); fewer than 2^31 input and output elements.
 */
int sam_hip_preprocess(const void* img, void* out, int dtype, int h, int w, int nh, int nw, int size,
                       const float* mean, const float* std_dev, void* stream);

/*
 * out = res + y + bias[i % c] over `total` elements (bias broadcast over the last dimension, c of them),
 * computed in f32 as (res + y) + bias and rounded once to `dtype`.
 * Replaces kernels::bias_residual (kernels.rs:1040-1049; cuda::BiasResidual, kernels.rs:1229-1258,
 * sam.cu:129-134; CPU cpu::BiasResidual, kernels.rs:618-640). Requires total % c == 0; total == 0 is a
 * no-op. out may alias res or y.
 */
int sam_hip_bias_residual(const void* res, const void* y, const void* bias, void* out, int dtype, long total, int c,
                          void* stream);

/*
 * out = gelu_erf(y + bias[i % c]) = 0.5 x (1 + erf(x / sqrt(2))) with x = y + bias[i % c], in f32, rounded
 * once to `dtype`. Replaces kernels::bias_gelu (kernels.rs:1051-1061; cuda::BiasGelu,
 * kernels.rs:1260-1290, sam.cu:136-141; CPU cpu::BiasGelu, kernels.rs:642-663). Requires
 * total % c == 0. out may alias y.
 */
int sam_hip_bias_gelu(const void* y, const void* bias, void* out, int dtype, long total, int c, void* stream);

/*
 * bias_residual followed by LayerNorm over each row, in one pass: for rows of c elements,
 *   out[r, :]    = res[r, :] + y[r, :] + bias          (as sam_hip_bias_residual, rounded to dtype)
 *   ln_out[r, :] = (out[r, :] - mean) / sqrt(var + eps) * ln_w + ln_b   (biased variance, f32)
 * with mean and var taken over the rounded out row. The reference runs the two as separate steps of
 * its encoder block, kernels::bias_residual (kernels.rs:1040-1049) and candle_nn::LayerNorm
 * (sam1/encoder.rs:118-124: the residual after the attention, then norm2; the residual after the MLP,
 * then the next block's norm1); no single reference kernel corresponds to the pair. c must be a
 * multiple of the 16-byte vector width (4 f32, 8 f16/bf16) and at most 512 vectors (2048 f32, 4096
 * f16/bf16), every pointer 16-byte aligned; otherwise SAM_HIP_EUNSUPPORTED. out may alias res or y;
 * ln_out must not alias any input.
 */
int sam_hip_bias_residual_ln(const void* res, const void* y, const void* bias, const void* ln_w, const void* ln_b,
                             void* out, void* ln_out, int dtype, long rows, int c, float eps, void* stream);

/*
 * Flash attention without a mask, f32 / f16 / bf16, on [b, l, h, d] operands given by (batch, row, head)
 * element strides (NULL = contiguous [b, l, h, d]; the head dimension is always contiguous):
 *   out[b, i, h, :] = softmax_j(scale * q[b,i,h,:] . k[b,j,h,:]) . v[b, :, h, :]
 * Replaces the reference's GPU flash attention candle_flash_attn::flash_attn(q, k, v, scale, false)
 * (sam2/hiera.rs:143-151, sam3/nn.rs:65-71, sam3/vision.rs:116-121), kernels::flash_attn_cpu
 * (kernels.rs:910-915, cpu_gemm.rs:361-417) and sam3::nn::sdpa with mask None (sam3/nn.rs:26-34; pass
 * [b, h, l, d] tensors as strides (h*l*d, d, l*d)). Lq != Lk is allowed.
 * Optional RoPE, as SAM 2 memory attention applies it before sdpa (RopeAttn::forward,
 * sam3/video.rs:106-141): the first n_rope_q queries and the first n_rope_k keys are rotated with the
 * f32 tables rope_cos / rope_sin [rope_rows, d] (table row = index % rope_rows), the other rows are
 * used as they are; n_rope_q = n_rope_k = 0 disables it (the tables may then be NULL).
 * Workspace: sam_hip_flash_attn_workspace_size() bytes of device memory (16-byte aligned), for the
 * key-split partial results, when n_rope_k > 0 the rotated keys and queries, and when d == 256 V as
 * transposed key tiles; it may be NULL when that size is 0. The size depends on the current device's
 * CU count: query it on the device that runs the call.
 * f32 is the reference's f32 GPU path (with --dtype f32 every attention runs as sdpa in candle's f32
 * matmuls): exact f32 arithmetic in natural units, to 1e-5 relative of the exact result.
 * Limits: d % 8 == 0, d <= 256; scale >= 0; pointers and strides 16-byte aligned; out must not
 * overlap k, v or the workspace.
 */
long sam_hip_flash_attn_workspace_size(int dtype, int b, int lq, int lk, int h, int d, int n_rope_k);
int sam_hip_flash_attn(const void* q, const void* k, const void* v, void* out, int dtype, int b, int lq, int lk,
                       int h, int d, const long* strides_q, const long* strides_k, const long* strides_v,
                       const long* strides_o, float scale, const float* rope_cos, const float* rope_sin,
                       int rope_rows, int n_rope_q, int n_rope_k, void* workspace, long workspace_bytes,
                       void* stream);

/*
 * sam3::nn::sdpa with an additive mask (sam3/nn.rs:26-34, Some(mask)), f32 / f16 / bf16:
 *   out[b, i, h, :] = softmax_j(scale * q[b,i,h,:] . k[b,j,h,:] + mask[b, h, i, j]) . v[b, :, h, :]
 * the GPU counterpart for its masked callers: the key-padding text mask of SAM 3's DETR encoder and
 * decoder (sam3/detr.rs:55, 191, 272; additive [1, 1, 1, L], 0 or -inf) and TinyViT's attention
 * biases (sam1/tinyvit.rs:216; [1, heads, N, N]). The mask has the element type of q and is read through 4 element strides (batch,
 * head, query, key); a stride of 0 broadcasts that dimension. A query whose keys are all -inf gets NaN,
 * as the reference's softmax gives. Operands, strides, workspace (sam_hip_flash_attn_workspace_size
 * with n_rope_k = 0) and limits as sam_hip_flash_attn; no RoPE; the mask is aligned to its element size.
 */
int sam_hip_sdpa_mask(const void* q, const void* k, const void* v, const void* mask, void* out, int dtype, int b,
                      int lq, int lk, int h, int d, const long* strides_q, const long* strides_k,
                      const long* strides_v, const long* strides_mask, const long* strides_o, float scale,
                      void* workspace, long workspace_bytes, void* stream);

/*
 * sam_hip_flash_attn without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart
 * in the reference: its GPU flash attention allocates internally. The workspace comes from a fixed
 * array of SAM_HIP_FLASH_NOALLOC_MAX_BYTES bytes that the library holds on every GPU it runs on until
 * the process ends; a call whose sam_hip_flash_attn_workspace_size exceeds it fails with
 * SAM_HIP_EUNSUPPORTED. Its key-split plan assumes at most 256 CUs whatever the device has (the split
 * count, and so the workspace, grows with the CU count), so a call's need does not depend on the
 * device: SAM 2.1 memory attention needs 65.3 MB. The call itself
 * allocates nothing. All calls on one GPU share that array: calls on one stream are ordered and safe,
 * calls that overlap on one GPU (several streams or threads) race. Arguments and limits otherwise as
 * sam_hip_flash_attn.
 */
#define SAM_HIP_FLASH_NOALLOC_MAX_BYTES (64L << 20)
int sam_hip_flash_attn_noalloc(const void* q, const void* k, const void* v, void* out, int dtype, int b, int lq,
                               int lk, int h, int d, const long* strides_q, const long* strides_k,
                               const long* strides_v, const long* strides_o, float scale, const float* rope_cos,
                               const float* rope_sin, int rope_rows, int n_rope_q, int n_rope_k, void* stream);

/*
 * 2-D axial RoPE on rows of a [b, l, h, d] tensor (strides as for flash attention, NULL = contiguous):
 *   out[.., r, .., 2i]   = x[2i] * cos[t, 2i] - x[2i+1] * sin[t, 2i]
 *   out[.., r, .., 2i+1] = x[2i+1] * cos[t, 2i+1] + x[2i] * sin[t, 2i+1]   (r < n_rot, t = r % rope_rows)
 * in f32, each product and the sum rounded, then converted to dtype; rows r >= n_rot are copied.
 * Replaces the reference's rope (sam3/video.rs:106-113) and its key tiling / pointer exclusion
 * (sam3/video.rs:133-141); the tables are those of rope_tables_hd (sam3/vision.rs:26-46), f32.
 * Limits: d % 8 == 0 (f16/bf16) or d % 4 == 0 (f32); pointers and strides 16-byte aligned.
 */
int sam_hip_rope(const void* x, const float* rope_cos, const float* rope_sin, void* out, int dtype, int b, int l,
                 int h, int d, const long* strides_x, const long* strides_out, int rope_rows, int n_rot,
                 void* stream);

/*
 * SAM 3 ViT's qkv step: the fused qkv projection's output with the bias added and 2-D RoPE on q and k,
 * packed for the attention:
 *   y [tokens, 3*nh*hd] (columns (qkv, head, d)), bias [3*nh*hd], rope_cos/rope_sin f32 [n, hd]
 *   -> out [3, tokens, nh, hd]; for a q or k pair (x0, x1) = (y + bias)[2i, 2i+1] of token t,
 *   out = (x0*c - x1*s, x1*c + x0*s) with c, s = cos/sin[t % n, 2i] (the even column serves both);
 *   v rows are y + bias.
 * In f32, y + bias unrounded, each product and the difference (sum) rounded, converted to dtype once.
 * Replaces kernels::qkv_rope (kernels.rs:1013-1037; GPU op kernels.rs:1330-1362, sam.cu:210-235; CPU
 * twin kernels.rs:321-362); the tables are those of rope_tables_hd (sam3/vision.rs:26-46).
 * Limits: hd even; 3*nh*hd < 2^31; pointers 16-byte aligned. hd % 8 == 0 runs the vector kernel.
 */
int sam_hip_qkv_rope(const void* y, const void* bias, const float* rope_cos, const float* rope_sin, void* out,
                     int dtype, long tokens, int n, int nh, int hd, void* stream);

/* Message describing the last error returned on this thread ("" if none). */
const char* sam_hip_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int sam_hip_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
