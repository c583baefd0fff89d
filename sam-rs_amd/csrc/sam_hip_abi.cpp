// extern "C" entry points of libsam_hip.so (declared in include/sam_hip.h): argument checks with the
// reference's error behaviour, dtype dispatch, and the kernel launches.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "../../include/sam_hip.h"
#include "flash_attn.hpp"

namespace samhip {
hipError_t attn_relpos_half(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out,
                            int bh, int hd, int h, int w, float scale, hipStream_t stream);
hipError_t attn_relpos_f32(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                           int h, int w, float scale, hipStream_t stream);
hipError_t deform_attn(int dtype, const void* value, const void* loc, const void* attn, void* out, int b, int s,
                       int q, int h, int d, int l, int p, const int* shapes, hipStream_t stream);
hipError_t deform_core(int dtype, const void* value, const void* offsets, const void* logits, const void* refs,
                       int ncoord, void* out, int b, int s, int q, int h, int d, int l, int p, const int* shapes,
                       hipStream_t stream);
hipError_t relpos_softmax(int dtype, const void* s, const void* q, const void* tab, void* out, long rows, int h, int w,
                          int hd, float scale, hipStream_t stream);
hipError_t qkv_split(int dtype, const void* y, const void* bias, void* out, long tokens, int n, int nh, int hd,
                     hipStream_t stream);
hipError_t qkv_split_grid(int dtype, const void* y, const void* bias, void* out, int batch, int gh, int gw, int ws,
                          int nh, int hd, hipStream_t stream);
hipError_t window_merge(int dtype, const void* ctx, void* out, int batch, int gh, int gw, int ws, int nh, int hd,
                        hipStream_t stream);
hipError_t qkv_rope(int dtype, const void* y, const void* bias, const float* cos_t, const float* sin_t, void* out,
                    long tokens, int n, int nh, int hd, hipStream_t stream);
hipError_t preprocess(int dtype, const void* img, void* out, int h, int w, int nh, int nw, int size, const float* mean,
                      const float* stdv, hipStream_t stream);
int preprocess_max_taps(int n, int nout);
hipError_t bias_residual(int dtype, const void* res, const void* y, const void* b, void* out, long total, int c,
                         hipStream_t stream);
hipError_t bias_gelu(int dtype, const void* y, const void* b, void* out, long total, int c, hipStream_t stream);
hipError_t bias_residual_ln(int dtype, const void* res, const void* y, const void* b, const void* lw, const void* lb,
                            void* out, void* ln, long rows, int c, float eps, hipStream_t stream);
}  // namespace samhip

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return SAM_HIP_OK;
}

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SAM_HIP_EHIP, "%s: HIP error %s", what, hipGetErrorString(e));
  return ok();
}

// The reference's dtype dispatch (kernels.rs:1086-1095) accepts exactly f16, bf16 and f32.
bool dtype_ok(int dtype) { return dtype == 0 || dtype == 1 || dtype == 2; }

// The process-wide switch of sam_hip_set_enabled, the counterpart of the reference's cpu_gemm::ENABLED
// (cpu_gemm.rs:11, 25-32): on unless the environment variable SAM_HIP_DISABLE is set to anything but
// "" or "0" when the library is loaded; sam_hip_set_enabled changes it at any time.
bool initially_enabled() {
  const char* e = std::getenv("SAM_HIP_DISABLE");
  return !(e && e[0] && !(e[0] == '0' && e[1] == 0));
}
std::atomic<bool> g_enabled{initially_enabled()};

// Every compute entry point starts here: when the switch is off it returns SAM_HIP_EDISABLED before
// looking at any argument, and no device call is made.
#define SAM_HIP_REQUIRE_ENABLED(what)                                                                       \
  do {                                                                                                      \
    if (!g_enabled.load(std::memory_order_relaxed))                                                         \
      return fail(SAM_HIP_EDISABLED, "%s: the HIP path is switched off (sam_hip_set_enabled(0) or "        \
                  "SAM_HIP_DISABLE); take the reference path", what);                                       \
  } while (0)

// The kernels move their operands in 16-byte vectors (and by 16-byte LDS DMA), which the header's
// alignment rule guarantees; a pointer that breaks it is rejected rather than read.
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

namespace samhip {
// Sets this thread's sam_hip_last_error message (for entry points defined in other files).
int report_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
}  // namespace samhip

extern "C" {

int sam_hip_abi_version(void) { return 5; }

void sam_hip_set_enabled(int on) { g_enabled.store(on != 0, std::memory_order_relaxed); }

int sam_hip_enabled(void) { return g_enabled.load(std::memory_order_relaxed) ? 1 : 0; }

const char* sam_hip_last_error(void) { return g_last_error.c_str(); }

int sam_hip_attn_relpos(const void* q, const void* kt, const void* v, const void* table, void* out, int dtype, int bh,
                        int h, int w, int hd, float scale, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("attn-relpos");
  if (!q || !kt || !v || !table || !out) return fail(SAM_HIP_EINVAL, "attn-relpos: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (bh <= 0 || h <= 0 || w <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "attn-relpos: sizes must be positive (bh=%d h=%d w=%d hd=%d)", bh, h, w, hd);
  if (h > 128 || w > 128 || (dtype == 0 && (h > 64 || w > 64)))
    return fail(SAM_HIP_EUNSUPPORTED, "attn-relpos: the fused kernels support grids up to %s, got %dx%d",
                dtype == 0 ? "64x64 in f32" : "128x128", h, w);
  if ((long)bh * h * w >= (1L << 31))  // the launch grids count workgroups of 32 to 256 queries in 32 bits
    return fail(SAM_HIP_EUNSUPPORTED, "attn-relpos: bh*h*w = %ld queries is beyond 2^31", (long)bh * h * w);
  const int align = dtype == 0 ? 4 : 8;
  if (hd % align != 0 || hd > 128)
    return fail(SAM_HIP_EUNSUPPORTED, "attn-relpos: head dim must be a multiple of %d and at most 128, got %d", align,
                hd);
  if (!aligned16(q) || !aligned16(kt) || !aligned16(v) || !aligned16(table) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "attn-relpos: q, kt, v, table and out must be 16-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = dtype == 0 ? samhip::attn_relpos_f32(q, kt, v, table, out, bh, hd, h, w, scale, s)
                            : samhip::attn_relpos_half(dtype, q, kt, v, table, out, bh, hd, h, w, scale, s);
  return check_launch(e, "attn-relpos");
}

namespace {
// The argument checks shared by sam_hip_deform_attn and sam_hip_deform_core (pointers checked by the callers).
int check_deform(const void* value, const void* out, int dtype, int b, int s, int q, int h, int d, int l, int p,
                 const int* shapes) {
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (b <= 0 || s <= 0 || q <= 0 || h <= 0 || d <= 0 || l <= 0 || p <= 0)
    return fail(SAM_HIP_EINVAL, "deform-attn: sizes must be positive (b=%d s=%d q=%d h=%d d=%d l=%d p=%d)", b, s, q, h,
                d, l, p);
  if (l > 4) return fail(SAM_HIP_EUNSUPPORTED, "deform-attn supports at most 4 levels, got %d", l);  // kernels.rs:1175
  if (l * p > 64) return fail(SAM_HIP_EUNSUPPORTED, "deform-attn: at most 64 sampling points per head, got %d", l * p);
  long total = 0;
  for (int i = 0; i < l; ++i) {
    if (shapes[2 * i] <= 0 || shapes[2 * i + 1] <= 0)
      return fail(SAM_HIP_EINVAL, "deform-attn: level %d has shape %dx%d", i, shapes[2 * i], shapes[2 * i + 1]);
    total += (long)shapes[2 * i] * shapes[2 * i + 1];
  }
  if (total != s)
    return fail(SAM_HIP_EINVAL, "deform-attn: the levels hold %ld pixels but value has %d", total, s);
  if ((long)b * s * h * d >= (1L << 31))
    return fail(SAM_HIP_EUNSUPPORTED, "deform-attn: value holds more than 2^31 elements");
  // value rows are gathered and out rows stored in 16-byte vectors; loc and attn are read per element
  if (!aligned16(value) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "deform-attn: value and out must be 16-byte aligned");
  return SAM_HIP_OK;
}
}  // namespace

int sam_hip_deform_attn(const void* value, const void* loc, const void* attn, void* out, int dtype, int b, int s,
                        int q, int h, int d, int l, int p, const int* shapes, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("deform-attn");
  if (!value || !loc || !attn || !out || !shapes) return fail(SAM_HIP_EINVAL, "deform-attn: null pointer argument");
  if (int rc = check_deform(value, out, dtype, b, s, q, h, d, l, p, shapes); rc != SAM_HIP_OK) return rc;
  hipError_t e = samhip::deform_attn(dtype, value, loc, attn, out, b, s, q, h, d, l, p, shapes,
                                     reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "deform-attn");
}

int sam_hip_deform_core(const void* value, const void* offsets, const void* logits, const void* refs, void* out,
                        int dtype, int b, int s, int q, int h, int d, int l, int p, int ncoord, const int* shapes,
                        void* stream) {
  SAM_HIP_REQUIRE_ENABLED("deform-core");
  if (!value || !offsets || !logits || !refs || !out || !shapes)
    return fail(SAM_HIP_EINVAL, "deform-core: null pointer argument");
  if (ncoord != 2 && ncoord != 4)
    return fail(SAM_HIP_EINVAL, "deform-core: reference points have 2 or 4 coordinates, got %d", ncoord);
  if (int rc = check_deform(value, out, dtype, b, s, q, h, d, l, p, shapes); rc != SAM_HIP_OK) return rc;
  hipError_t e = samhip::deform_core(dtype, value, offsets, logits, refs, ncoord, out, b, s, q, h, d, l, p, shapes,
                                     reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "deform-core");
}

int sam_hip_preprocess(const void* img, void* out, int dtype, int h, int w, int nh, int nw, int size,
                       const float* mean, const float* std_dev, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("preprocess");
  if (!img || !out || !mean || !std_dev) return fail(SAM_HIP_EINVAL, "preprocess: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (h <= 0 || w <= 0 || size <= 0)
    return fail(SAM_HIP_EINVAL, "preprocess: sizes must be positive (h=%d w=%d size=%d)", h, w, size);
  if (nh < 1 || nw < 1 || nh > size || nw > size)
    return fail(SAM_HIP_EINVAL, "preprocess: resized %dx%d does not fit in %dx%d", nh, nw, size, size);
  if ((long)h * w * 3 >= (1L << 31) || 3L * size * size >= (1L << 31))
    return fail(SAM_HIP_EUNSUPPORTED, "preprocess: more than 2^31 input or output elements");
  for (int c = 0; c < 3; ++c)
    if (!(std_dev[c] != 0.f)) return fail(SAM_HIP_EINVAL, "preprocess: std[%d] is zero", c);
  if (samhip::preprocess_max_taps(w, nw) > 64)
    return fail(SAM_HIP_EUNSUPPORTED, "preprocess: shrinking %d columns to %d needs more than 64 filter taps", w, nw);
  if (samhip::preprocess_max_taps(h, nh) > 64)
    return fail(SAM_HIP_EUNSUPPORTED, "preprocess: shrinking %d rows to %d needs more than 64 filter taps", h, nh);
  hipError_t e = samhip::preprocess(dtype, img, out, h, w, nh, nw, size, mean, std_dev,
                                    reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "preprocess");
}

int sam_hip_bias_residual(const void* res, const void* y, const void* bias, void* out, int dtype, long total, int c,
                          void* stream) {
  SAM_HIP_REQUIRE_ENABLED("bias-residual");
  if (!res || !y || !bias || !out) return fail(SAM_HIP_EINVAL, "bias-residual: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (total < 0 || c <= 0 || total % c != 0)
    return fail(SAM_HIP_EINVAL, "bias-residual: %ld elements do not hold whole rows of the %d-element bias", total, c);
  hipError_t e = samhip::bias_residual(dtype, res, y, bias, out, total, c, reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "bias-residual");
}

int sam_hip_bias_residual_ln(const void* res, const void* y, const void* bias, const void* ln_w, const void* ln_b,
                             void* out, void* ln_out, int dtype, long rows, int c, float eps, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("bias-residual-ln");
  if (!res || !y || !bias || !ln_w || !ln_b || !out || !ln_out)
    return fail(SAM_HIP_EINVAL, "bias-residual-ln: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  const int vec = dtype == 0 ? 4 : 8;  // elements per 16-byte vector (f32: 4)
  if (rows < 0 || c <= 0 || !(eps >= 0.f))
    return fail(SAM_HIP_EINVAL, "bias-residual-ln: rows %ld, c %d, eps %g", rows, c, (double)eps);
  if (c % vec != 0 || c > 512 * vec)
    return fail(SAM_HIP_EUNSUPPORTED, "bias-residual-ln: the row length %d must be a multiple of %d and at most %d", c,
                vec, 512 * vec);
  // elements below 2^40; one wave per row, four rows per workgroup, fewer than 2^31 workgroups
  if (rows > (1L << 40) / c || rows > 4L * 0x7fffffffL)
    return fail(SAM_HIP_EUNSUPPORTED, "bias-residual-ln: %ld rows of %d are too many", rows, c);
  if (!aligned16(res) || !aligned16(y) || !aligned16(bias) || !aligned16(ln_w) || !aligned16(ln_b) ||
      !aligned16(out) || !aligned16(ln_out))
    return fail(SAM_HIP_EUNSUPPORTED, "bias-residual-ln: every pointer must be 16-byte aligned");
  hipError_t e = samhip::bias_residual_ln(dtype, res, y, bias, ln_w, ln_b, out, ln_out, rows, c, eps,
                                          reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "bias-residual-ln");
}

int sam_hip_bias_gelu(const void* y, const void* bias, void* out, int dtype, long total, int c, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("bias-gelu");
  if (!y || !bias || !out) return fail(SAM_HIP_EINVAL, "bias-gelu: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (total < 0 || c <= 0 || total % c != 0)
    return fail(SAM_HIP_EINVAL, "bias-gelu: %ld elements do not hold whole rows of the %d-element bias", total, c);
  hipError_t e = samhip::bias_gelu(dtype, y, bias, out, total, c, reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "bias-gelu");
}

int sam_hip_relpos_softmax(const void* s, const void* q, const void* table, void* out, int dtype, long rows, int h,
                           int w, int hd, float scale, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("relpos-softmax");
  if (!s || !q || !table || !out) return fail(SAM_HIP_EINVAL, "relpos-softmax: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (rows <= 0 || h <= 0 || w <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "relpos-softmax: sizes must be positive (rows=%ld h=%d w=%d hd=%d)", rows, h, w, hd);
  if (rows % ((long)h * w) != 0)
    return fail(SAM_HIP_EINVAL, "relpos-softmax: %ld rows is not a multiple of h*w = %d", rows, h * w);
  // Rows of up to 16384 keys: past 8192 (the reference's GPU kernel limit, kernels.rs:1078-1083, beyond
  // which it takes its tensor path) they run on the two-pass scalar kernel.
  if (h > 128 || w > 128 || hd > 256)
    return fail(SAM_HIP_EUNSUPPORTED, "relpos-softmax: h, w <= 128 and hd <= 256, got %d, %d, %d", h, w, hd);
  if (rows > 0x7fffffffL) return fail(SAM_HIP_EUNSUPPORTED, "relpos-softmax: more than 2^31 rows");
  if (!aligned16(s) || !aligned16(q) || !aligned16(table) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "relpos-softmax: s, q, table and out must be 16-byte aligned");
  hipError_t e = samhip::relpos_softmax(dtype, s, q, table, out, rows, h, w, hd, scale,
                                        reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "relpos-softmax");
}

int sam_hip_qkv_split(const void* y, const void* bias, void* out, int dtype, long tokens, int n, int nh, int hd,
                      void* stream) {
  SAM_HIP_REQUIRE_ENABLED("qkv-split");
  if (!y || !bias || !out) return fail(SAM_HIP_EINVAL, "qkv-split: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (tokens <= 0 || n <= 0 || nh <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "qkv-split: sizes must be positive (tokens=%ld n=%d nh=%d hd=%d)", tokens, n, nh, hd);
  if (tokens % n != 0) return fail(SAM_HIP_EINVAL, "qkv-split: %ld tokens is not a multiple of n = %d", tokens, n);
  if (hd > 256) return fail(SAM_HIP_EUNSUPPORTED, "qkv-split: head dim at most 256, got %d", hd);
  if (3L * nh * hd > 0x7fffffffL)  // the kernel's row arithmetic (the 3*nh*hd columns of y) is 32-bit
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-split: 3*nh*hd = %ld columns is beyond 2^31", 3L * nh * hd);
  const long blocks = tokens / n * ((n + 63) / 64) * nh;
  if (blocks > 0x7fffffffL) return fail(SAM_HIP_EUNSUPPORTED, "qkv-split: too many tokens");
  if (!aligned16(y) || !aligned16(bias) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-split: y, bias and out must be 16-byte aligned");
  hipError_t e = samhip::qkv_split(dtype, y, bias, out, tokens, n, nh, hd, reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "qkv-split");
}

int sam_hip_qkv_split_grid(const void* y, const void* bias, void* out, int dtype, int batch, int gh, int gw, int ws,
                           int nh, int hd, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("qkv-split-grid");
  if (!y || !bias || !out) return fail(SAM_HIP_EINVAL, "qkv-split-grid: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (batch <= 0 || gh <= 0 || gw <= 0 || ws <= 0 || nh <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "qkv-split-grid: sizes must be positive (batch=%d gh=%d gw=%d ws=%d nh=%d hd=%d)",
                batch, gh, gw, ws, nh, hd);
  if (hd > 256) return fail(SAM_HIP_EUNSUPPORTED, "qkv-split-grid: head dim at most 256, got %d", hd);
  if (gh > 4096 || gw > 4096 || ws > 256) return fail(SAM_HIP_EUNSUPPORTED, "qkv-split-grid: grid or window too large");
  const long windows = (long)batch * ((gh + ws - 1) / ws) * ((gw + ws - 1) / ws);
  const long n = (long)ws * ws;
  if (windows * ((n + 63) / 64) * nh > 0x7fffffffL || windows * n * 3L * nh * hd >= (1L << 40))
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-split-grid: too many tokens");
  // the kernel's row arithmetic (the 3*nh*hd columns of y) is 32-bit
  if (3L * nh * hd > 0x7fffffffL)
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-split-grid: 3*nh*hd = %ld columns is beyond 2^31", 3L * nh * hd);
  if (!aligned16(y) || !aligned16(bias) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-split-grid: y, bias and out must be 16-byte aligned");
  hipError_t e =
      samhip::qkv_split_grid(dtype, y, bias, out, batch, gh, gw, ws, nh, hd, reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "qkv-split-grid");
}

int sam_hip_window_merge(const void* ctx, void* out, int dtype, int batch, int gh, int gw, int ws, int nh, int hd,
                         void* stream) {
  SAM_HIP_REQUIRE_ENABLED("window-merge");
  if (!ctx || !out) return fail(SAM_HIP_EINVAL, "window-merge: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (batch <= 0 || gh <= 0 || gw <= 0 || ws <= 0 || nh <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "window-merge: sizes must be positive (batch=%d gh=%d gw=%d ws=%d nh=%d hd=%d)", batch,
                gh, gw, ws, nh, hd);
  if (gh > 4096 || gw > 4096 || ws > 256 || hd > 4096)
    return fail(SAM_HIP_EUNSUPPORTED, "window-merge: grid, window or head dim too large");
  const long windows = (long)batch * ((gh + ws - 1) / ws) * ((gw + ws - 1) / ws);
  if (windows * ws * ws * (long)nh * hd >= (1L << 38))
    return fail(SAM_HIP_EUNSUPPORTED, "window-merge: too many elements");
  // the kernel's row arithmetic (nh*hd columns of out) is 32-bit
  if ((long)nh * hd > 0x7fffffffL)
    return fail(SAM_HIP_EUNSUPPORTED, "window-merge: nh*hd = %ld columns is beyond 2^31", (long)nh * hd);
  if (!aligned16(ctx) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "window-merge: ctx and out must be 16-byte aligned");
  hipError_t e = samhip::window_merge(dtype, ctx, out, batch, gh, gw, ws, nh, hd, reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "window-merge");
}

}  // extern "C"

// ------------------------------------------------------------------------------------ flash attention

namespace {

void contiguous_strides(long* s, int l, int h, int d) {
  s[0] = (long)l * h * d;
  s[1] = (long)h * d;
  s[2] = d;
}

// Strides of a [b, l, h, d] operand: the caller's, or those of the contiguous layout when null.
int get_strides(const long* in, long* out, int l, int h, int d, int elem, const char* what) {
  if (in) {
    for (int i = 0; i < 3; ++i) out[i] = in[i];
  } else {
    contiguous_strides(out, l, h, d);
  }
  for (int i = 0; i < 3; ++i)
    if (out[i] < 0 || (out[i] * elem) % 16 != 0)
      return fail(SAM_HIP_EUNSUPPORTED, "flash-attn: %s strides must be non-negative multiples of 16 bytes", what);
  return SAM_HIP_OK;
}

int device_cus() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
  }
  return cus;
}

struct FlashPlan {
  int qblocks, nsplit, tps;
  size_t partial_bytes, krot_bytes, qrot_bytes, vt_bytes, total;
};

size_t round256(size_t n) { return (n + 255) / 256 * 256; }

// Workspace: key-split partials, then (when keys are rotated) the rotated keys and room for the rotated
// queries, both contiguous [b, l, h, d], then (head dim 256) V as transposed key tiles.
// cu_cap > 0 plans as if the device had at most that many CUs (fewer key splits, a smaller workspace).
FlashPlan plan_flash(int dtype, int b, int lq, int lk, int h, int d, int n_rope_k, int cu_cap) {
  FlashPlan pl;
  int cus = device_cus();
  if (cu_cap > 0 && cus > cu_cap) cus = cu_cap;
  samhip::flash_plan(dtype, b, h, lq, lk, d, cus, &pl.qblocks, &pl.nsplit, &pl.tps);
  pl.partial_bytes = round256(samhip::flash_partial_bytes(b, h, lq, d, pl.nsplit));
  const size_t elem = dtype == 0 ? 4 : 2;
  pl.krot_bytes = n_rope_k > 0 ? round256((size_t)b * lk * h * d * elem) : 0;
  pl.qrot_bytes = n_rope_k > 0 ? round256((size_t)b * lq * h * d * elem) : 0;
  pl.vt_bytes = dtype == 0 ? 0 : round256(samhip::flash256_vt_bytes(b, h, lk, d));
  pl.total = pl.partial_bytes + pl.krot_bytes + pl.qrot_bytes + pl.vt_bytes;
  return pl;
}

int check_flash_sizes(int dtype, int b, int lq, int lk, int h, int d) {
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (b <= 0 || lq <= 0 || lk <= 0 || h <= 0 || d <= 0)
    return fail(SAM_HIP_EINVAL, "flash-attn: sizes must be positive (b=%d lq=%d lk=%d h=%d d=%d)", b, lq, lk, h, d);
  if (d % 8 != 0 || d > 256)
    return fail(SAM_HIP_EUNSUPPORTED, "flash-attn: head dim must be a multiple of 8 and at most 256, got %d", d);
  if ((long)b * h * lq >= (1L << 31) || (long)lk * 64 >= (1L << 31))
    return fail(SAM_HIP_EUNSUPPORTED, "flash-attn: too many rows");
  return SAM_HIP_OK;
}

}  // namespace

extern "C" {

long sam_hip_flash_attn_workspace_size(int dtype, int b, int lq, int lk, int h, int d, int n_rope_k) {
  if (check_flash_sizes(dtype, b, lq, lk, h, d) != SAM_HIP_OK) return -1;
  return (long)plan_flash(dtype, b, lq, lk, h, d, n_rope_k, 0).total;
}

// sam_hip_flash_attn, and sam_hip_sdpa_mask when mask is not null (no RoPE then).
static int flash_entry(const void* q, const void* k, const void* v, void* out, int dtype, int b, int lq, int lk, int h,
                       int d, const long* strides_q, const long* strides_k, const long* strides_v,
                       const long* strides_o, float scale, const float* rope_cos, const float* rope_sin,
                       int rope_rows, int n_rope_q, int n_rope_k, void* workspace, long workspace_bytes,
                       void* stream, const void* mask, const long* strides_mask, int cu_cap) {
  SAM_HIP_REQUIRE_ENABLED(mask ? "sdpa-mask" : "flash-attn");
  if (!q || !k || !v || !out) return fail(SAM_HIP_EINVAL, "flash-attn: null pointer argument");
  int rc = check_flash_sizes(dtype, b, lq, lk, h, d);
  if (rc != SAM_HIP_OK) return rc;
  if (!(scale >= 0.f) || scale > 3.0e38f)
    return fail(SAM_HIP_EINVAL, "flash-attn: scale must be finite and non-negative, got %g", (double)scale);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "flash-attn: q, k, v and out must be 16-byte aligned");
  if (n_rope_q < 0 || n_rope_k < 0 || n_rope_q > lq || n_rope_k > lk)
    return fail(SAM_HIP_EINVAL, "flash-attn: rotated rows out of range (n_rope_q=%d of %d, n_rope_k=%d of %d)",
                n_rope_q, lq, n_rope_k, lk);
  if ((n_rope_q > 0 || n_rope_k > 0) && (!rope_cos || !rope_sin || rope_rows <= 0 || !aligned16(rope_cos) ||
                                         !aligned16(rope_sin)))
    return fail(SAM_HIP_EINVAL, "flash-attn: RoPE needs 16-byte aligned cos/sin tables with rope_rows > 0");
  const int elem = dtype == 0 ? 4 : 2;
  samhip::FlashParams p{};
  if ((rc = get_strides(strides_q, p.sq, lq, h, d, elem, "q")) != SAM_HIP_OK) return rc;
  if ((rc = get_strides(strides_k, p.sk, lk, h, d, elem, "k")) != SAM_HIP_OK) return rc;
  if ((rc = get_strides(strides_v, p.sv, lk, h, d, elem, "v")) != SAM_HIP_OK) return rc;
  if ((rc = get_strides(strides_o, p.so, lq, h, d, elem, "out")) != SAM_HIP_OK) return rc;
  if (mask) {
    if (!strides_mask) return fail(SAM_HIP_EINVAL, "sdpa-mask: the mask needs its 4 strides (batch, head, query, key)");
    for (int i = 0; i < 4; ++i) {
      if (strides_mask[i] < 0) return fail(SAM_HIP_EUNSUPPORTED, "sdpa-mask: mask strides must be non-negative");
      p.sm[i] = strides_mask[i];
    }
    if ((reinterpret_cast<size_t>(mask) & (size_t)(elem - 1)) != 0)
      return fail(SAM_HIP_EUNSUPPORTED, "sdpa-mask: the mask must be aligned to its element size");
    p.mask = mask;
  }
  const FlashPlan pl = plan_flash(dtype, b, lq, lk, h, d, n_rope_k, cu_cap);
  if (pl.total > 0 && (!workspace || workspace_bytes < (long)pl.total))
    return fail(SAM_HIP_EINVAL, "flash-attn: needs a workspace of %zu bytes (sam_hip_flash_attn_workspace_size), got %ld",
                pl.total, workspace ? workspace_bytes : 0L);
  if (workspace && !aligned16(workspace)) return fail(SAM_HIP_EINVAL, "flash-attn: workspace must be 16-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = out;
  bool ropeq = n_rope_q > 0;
  p.vt = pl.vt_bytes > 0 ? ws + pl.partial_bytes + pl.krot_bytes + pl.qrot_bytes : nullptr;
  if (n_rope_k > 0 && dtype == 0) {
    // f32: the keys go into the workspace rotated; the f32 kernel rotates the queries as it loads them
    void* kr = ws + pl.partial_bytes;
    long skr[3];
    contiguous_strides(skr, lk, h, d);
    hipError_t e = samhip::rope_rows(0, k, p.sk, kr, skr, b, lk, h, d, rope_cos, rope_sin, rope_rows, n_rope_k, s);
    if (e != hipSuccess) return check_launch(e, "flash-attn (rotation)");
    p.k = kr;
    for (int i = 0; i < 3; ++i) p.sk[i] = skr[i];
  } else if (n_rope_k > 0) {
    // keys, and the queries when they are rotated too, go into the workspace as contiguous [b, l, h, d]
    // copies, in one launch; the attention kernel then reads plain operands
    void* kr = ws + pl.partial_bytes;
    void* qr = ws + pl.partial_bytes + pl.krot_bytes;
    long skr[3], sqr[3];
    contiguous_strides(skr, lk, h, d);
    contiguous_strides(sqr, lq, h, d);
    const samhip::RopeJob jk = samhip::rope_job(k, p.sk, kr, skr, b, lk, h, d, n_rope_k);
    const samhip::RopeJob jq = samhip::rope_job(q, p.sq, qr, sqr, b, lq, h, d, n_rope_q);
    // head dim 256: V's transposed key tiles are written by the same launch
    const samhip::VtJob jv{v, {p.sv[0], p.sv[1], p.sv[2]}, b, h, lk, p.vt};
    hipError_t e = samhip::rope_rows2(dtype, jk, ropeq ? &jq : nullptr, d, rope_cos, rope_sin, rope_rows, s,
                                      p.vt ? &jv : nullptr);
    if (e != hipSuccess) return check_launch(e, "flash-attn (rotation)");
    p.vt_ready = p.vt != nullptr;
    p.k = kr;
    for (int i = 0; i < 3; ++i) p.sk[i] = skr[i];
    if (ropeq) {
      p.q = qr;
      for (int i = 0; i < 3; ++i) p.sq[i] = sqr[i];
      ropeq = false;
    }
  }
  p.b = b;
  p.h = h;
  p.lq = lq;
  p.lk = lk;
  p.d = d;
  p.sc = scale * 1.4426950408889634f;
  p.fscale = scale;
  p.qblocks = pl.qblocks;
  p.nsplit = pl.nsplit;
  p.tps = pl.tps;
  if (pl.nsplit > 1) {
    p.opart = reinterpret_cast<float*>(ws);
    p.ml = reinterpret_cast<float*>(ws + (size_t)pl.nsplit * b * h * lq * samhip::flash_padded_dim(d) * sizeof(float));
  }
  p.rcos = rope_cos;
  p.rsin = rope_sin;
  p.rrows = rope_rows;
  p.nrq = ropeq ? n_rope_q : 0;
  const hipError_t e = dtype == 0 ? samhip::flash_attn_f32(p, ropeq, s) : samhip::flash_attn_half(dtype, p, ropeq, s);
  return check_launch(e, mask ? "sdpa-mask" : "flash-attn");
}

int sam_hip_flash_attn(const void* q, const void* k, const void* v, void* out, int dtype, int b, int lq, int lk, int h,
                       int d, const long* strides_q, const long* strides_k, const long* strides_v,
                       const long* strides_o, float scale, const float* rope_cos, const float* rope_sin,
                       int rope_rows, int n_rope_q, int n_rope_k, void* workspace, long workspace_bytes,
                       void* stream) {
  return flash_entry(q, k, v, out, dtype, b, lq, lk, h, d, strides_q, strides_k, strides_v, strides_o, scale,
                     rope_cos, rope_sin, rope_rows, n_rope_q, n_rope_k, workspace, workspace_bytes, stream, nullptr,
                     nullptr, 0);
}

int sam_hip_sdpa_mask(const void* q, const void* k, const void* v, const void* mask, void* out, int dtype, int b,
                      int lq, int lk, int h, int d, const long* strides_q, const long* strides_k,
                      const long* strides_v, const long* strides_mask, const long* strides_o, float scale,
                      void* workspace, long workspace_bytes, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("sdpa-mask");
  if (!mask) return fail(SAM_HIP_EINVAL, "sdpa-mask: null mask (use sam_hip_flash_attn for mask None)");
  return flash_entry(q, k, v, out, dtype, b, lq, lk, h, d, strides_q, strides_k, strides_v, strides_o, scale, nullptr,
                     nullptr, 0, 0, 0, workspace, workspace_bytes, stream, mask, strides_mask, 0);
}

}  // extern "C"

namespace samhip {
// sam_hip_flash_attn_workspace_size and sam_hip_flash_attn with the key-split plan of a device of at
// most cu_cap CUs (sam_hip_flash_attn_noalloc, whose workspace has a fixed size).
long flash_workspace_size_capped(int dtype, int b, int lq, int lk, int h, int d, int n_rope_k, int cu_cap) {
  if (check_flash_sizes(dtype, b, lq, lk, h, d) != SAM_HIP_OK) return -1;
  return (long)plan_flash(dtype, b, lq, lk, h, d, n_rope_k, cu_cap).total;
}
int flash_attn_capped(const void* q, const void* k, const void* v, void* out, int dtype, int b, int lq, int lk, int h,
                      int d, const long* strides_q, const long* strides_k, const long* strides_v,
                      const long* strides_o, float scale, const float* rope_cos, const float* rope_sin, int rope_rows,
                      int n_rope_q, int n_rope_k, void* workspace, long workspace_bytes, void* stream, int cu_cap) {
  return flash_entry(q, k, v, out, dtype, b, lq, lk, h, d, strides_q, strides_k, strides_v, strides_o, scale,
                     rope_cos, rope_sin, rope_rows, n_rope_q, n_rope_k, workspace, workspace_bytes, stream, nullptr,
                     nullptr, cu_cap);
}
}  // namespace samhip

extern "C" {

int sam_hip_rope(const void* x, const float* cos_t, const float* sin_t, void* out, int dtype, int b, int l, int h,
                 int d, const long* strides_x, const long* strides_out, int rope_rows, int n_rot, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("rope");
  if (!x || !cos_t || !sin_t || !out) return fail(SAM_HIP_EINVAL, "rope: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (b <= 0 || l <= 0 || h <= 0 || d <= 0 || rope_rows <= 0)
    return fail(SAM_HIP_EINVAL, "rope: sizes must be positive (b=%d l=%d h=%d d=%d rope_rows=%d)", b, l, h, d,
                rope_rows);
  const int per = dtype == 0 ? 4 : 8;
  if (d % per != 0) return fail(SAM_HIP_EUNSUPPORTED, "rope: head dim must be a multiple of %d, got %d", per, d);
  if (n_rot < 0 || n_rot > l) return fail(SAM_HIP_EINVAL, "rope: n_rot=%d outside [0, %d]", n_rot, l);
  if (!aligned16(x) || !aligned16(out)) return fail(SAM_HIP_EUNSUPPORTED, "rope: x and out must be 16-byte aligned");
  const int elem = dtype == 0 ? 4 : 2;
  long sx[3], so[3];
  int rc;
  if ((rc = get_strides(strides_x, sx, l, h, d, elem, "x")) != SAM_HIP_OK) return rc;
  if ((rc = get_strides(strides_out, so, l, h, d, elem, "out")) != SAM_HIP_OK) return rc;
  if ((long)b * l * h * (d / per) >= (1L << 40)) return fail(SAM_HIP_EUNSUPPORTED, "rope: too many elements");
  return check_launch(samhip::rope_rows(dtype, x, sx, out, so, b, l, h, d, cos_t, sin_t, rope_rows, n_rot,
                                        reinterpret_cast<hipStream_t>(stream)),
                      "rope");
}

int sam_hip_qkv_rope(const void* y, const void* bias, const float* cos_t, const float* sin_t, void* out, int dtype,
                     long tokens, int n, int nh, int hd, void* stream) {
  SAM_HIP_REQUIRE_ENABLED("qkv-rope");
  if (!y || !bias || !cos_t || !sin_t || !out) return fail(SAM_HIP_EINVAL, "qkv-rope: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (tokens <= 0 || n <= 0 || nh <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "qkv-rope: sizes must be positive (tokens=%ld n=%d nh=%d hd=%d)", tokens, n, nh, hd);
  if (hd % 2 != 0) return fail(SAM_HIP_EINVAL, "qkv-rope: head dim must be even (RoPE rotates pairs), got %d", hd);
  if (3L * nh * hd > 0x7fffffffL)  // the kernels' column arithmetic is 32-bit
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-rope: 3*nh*hd = %ld columns is beyond 2^31", 3L * nh * hd);
  // the vector kernel (hd % 8 == 0) counts its threads, at most one per 8-column vector, in 32 bits; the
  // pair kernel's grid is 32-bit
  const long units = hd % 8 == 0 ? tokens * (3L * nh * hd / 8) : tokens * (3L * nh * hd / 2);
  if (units >= (hd % 8 == 0 ? (1L << 32) : (1L << 39)) || (long)n * hd >= (1L << 40))
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-rope: too many tokens (%ld)", tokens);
  if (!aligned16(y) || !aligned16(bias) || !aligned16(cos_t) || !aligned16(sin_t) || !aligned16(out))
    return fail(SAM_HIP_EUNSUPPORTED, "qkv-rope: y, bias, cos, sin and out must be 16-byte aligned");
  return check_launch(
      samhip::qkv_rope(dtype, y, bias, cos_t, sin_t, out, tokens, n, nh, hd, reinterpret_cast<hipStream_t>(stream)),
      "qkv-rope");
}

}  // extern "C"
