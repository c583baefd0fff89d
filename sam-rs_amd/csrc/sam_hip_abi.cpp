// extern "C" entry points of libsam_hip.so (declared in include/sam_hip.h): argument checks with the
// reference's error behaviour, dtype dispatch, and the kernel launches.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/sam_hip.h"

namespace samhip {
hipError_t attn_relpos_half(int dtype, const void* q, const void* kt, const void* v, const void* table, void* out,
                            int bh, int hd, int h, int w, float scale, hipStream_t stream);
hipError_t attn_relpos_f32(const void* q, const void* kt, const void* v, const void* table, void* out, int bh, int hd,
                           int h, int w, float scale, hipStream_t stream);
hipError_t deform_attn(int dtype, const void* value, const void* loc, const void* attn, void* out, int b, int s,
                       int q, int h, int d, int l, int p, const int* shapes, hipStream_t stream);
hipError_t relpos_softmax(int dtype, const void* s, const void* q, const void* tab, void* out, long rows, int h, int w,
                          int hd, float scale, hipStream_t stream);
hipError_t qkv_split(int dtype, const void* y, const void* bias, void* out, long tokens, int n, int nh, int hd,
                     hipStream_t stream);
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

}  // namespace

extern "C" {

int sam_hip_abi_version(void) { return 1; }

const char* sam_hip_last_error(void) { return g_last_error.c_str(); }

int sam_hip_attn_relpos(const void* q, const void* kt, const void* v, const void* table, void* out, int dtype, int bh,
                        int h, int w, int hd, float scale, void* stream) {
  if (!q || !kt || !v || !table || !out) return fail(SAM_HIP_EINVAL, "attn-relpos: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (bh <= 0 || h <= 0 || w <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "attn-relpos: sizes must be positive (bh=%d h=%d w=%d hd=%d)", bh, h, w, hd);
  if (h > 64 || w > 64)
    return fail(SAM_HIP_EUNSUPPORTED, "attn-relpos: the fused kernel supports grids up to 64x64, got %dx%d", h, w);
  const int align = dtype == 0 ? 4 : 8;
  if (hd % align != 0 || hd > 128)
    return fail(SAM_HIP_EUNSUPPORTED, "attn-relpos: head dim must be a multiple of %d and at most 128, got %d", align,
                hd);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = dtype == 0 ? samhip::attn_relpos_f32(q, kt, v, table, out, bh, hd, h, w, scale, s)
                            : samhip::attn_relpos_half(dtype, q, kt, v, table, out, bh, hd, h, w, scale, s);
  return check_launch(e, "attn-relpos");
}

int sam_hip_deform_attn(const void* value, const void* loc, const void* attn, void* out, int dtype, int b, int s,
                        int q, int h, int d, int l, int p, const int* shapes, void* stream) {
  if (!value || !loc || !attn || !out || !shapes) return fail(SAM_HIP_EINVAL, "deform-attn: null pointer argument");
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
  hipError_t e = samhip::deform_attn(dtype, value, loc, attn, out, b, s, q, h, d, l, p, shapes,
                                     reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "deform-attn");
}

int sam_hip_relpos_softmax(const void* s, const void* q, const void* table, void* out, int dtype, long rows, int h,
                           int w, int hd, float scale, void* stream) {
  if (!s || !q || !table || !out) return fail(SAM_HIP_EINVAL, "relpos-softmax: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (rows <= 0 || h <= 0 || w <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "relpos-softmax: sizes must be positive (rows=%ld h=%d w=%d hd=%d)", rows, h, w, hd);
  if (rows % ((long)h * w) != 0)
    return fail(SAM_HIP_EINVAL, "relpos-softmax: %ld rows is not a multiple of h*w = %d", rows, h * w);
  // the reference's GPU kernel keeps a row in registers up to 256 x 32 values (kernels.rs:1078-1083)
  if ((long)h * w > 8192)
    return fail(SAM_HIP_EUNSUPPORTED, "relpos-softmax: rows longer than 8192 (h*w = %d)", h * w);
  if (h > 128 || w > 128 || hd > 256)
    return fail(SAM_HIP_EUNSUPPORTED, "relpos-softmax: h, w <= 128 and hd <= 256, got %d, %d, %d", h, w, hd);
  if (rows > 0x7fffffffL) return fail(SAM_HIP_EUNSUPPORTED, "relpos-softmax: more than 2^31 rows");
  hipError_t e = samhip::relpos_softmax(dtype, s, q, table, out, rows, h, w, hd, scale,
                                        reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "relpos-softmax");
}

int sam_hip_qkv_split(const void* y, const void* bias, void* out, int dtype, long tokens, int n, int nh, int hd,
                      void* stream) {
  if (!y || !bias || !out) return fail(SAM_HIP_EINVAL, "qkv-split: null pointer argument");
  if (!dtype_ok(dtype)) return fail(SAM_HIP_EDTYPE, "unsupported dtype %d for a sam-rs HIP kernel", dtype);
  if (tokens <= 0 || n <= 0 || nh <= 0 || hd <= 0)
    return fail(SAM_HIP_EINVAL, "qkv-split: sizes must be positive (tokens=%ld n=%d nh=%d hd=%d)", tokens, n, nh, hd);
  if (tokens % n != 0) return fail(SAM_HIP_EINVAL, "qkv-split: %ld tokens is not a multiple of n = %d", tokens, n);
  if (hd > 256) return fail(SAM_HIP_EUNSUPPORTED, "qkv-split: head dim at most 256, got %d", hd);
  const long blocks = tokens / n * ((n + 63) / 64) * nh;
  if (blocks > 0x7fffffffL) return fail(SAM_HIP_EUNSUPPORTED, "qkv-split: too many tokens");
  hipError_t e = samhip::qkv_split(dtype, y, bias, out, tokens, n, nh, hd, reinterpret_cast<hipStream_t>(stream));
  return check_launch(e, "qkv-split");
}

}  // extern "C"
