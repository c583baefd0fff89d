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

}  // extern "C"
