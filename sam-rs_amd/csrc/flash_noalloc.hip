// sam_hip_flash_attn_noalloc: flash attention for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It is
// sam_hip_flash_attn with the workspace taken from a fixed device array of this library instead of
// from the caller.
//
// The array is a file-scope __device__ variable, so every GPU the library runs on holds its own copy
// from module load until the process ends. Host code never uses its name as an address (on the host
// the name is only a stand-in): the device address comes from hipGetSymbolAddress, once per device,
// with that device current, and is kept per device.
//
// Every call on one GPU shares that GPU's array. Calls on one stream run in order and are safe; calls
// that overlap on one GPU (other streams, other threads) race on it. Nothing in it has to start at
// zero: the key-split partial results and the rotated keys and queries are written in full before
// they are read, so no clearing pass runs.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <string>

#include "../../include/sam_hip.h"

namespace samhip {
int report_error(int code, const std::string& msg);  // sam_hip_abi.cpp: the message of sam_hip_last_error
// sam_hip_abi.cpp: the workspace query and the flash entry point with the key-split plan of at most
// cu_cap CUs
long flash_workspace_size_capped(int dtype, int b, int lq, int lk, int h, int d, int n_rope_k, int cu_cap);
int flash_attn_capped(const void* q, const void* k, const void* v, void* out, int dtype, int b, int lq, int lk, int h,
                      int d, const long* strides_q, const long* strides_k, const long* strides_v,
                      const long* strides_o, float scale, const float* rope_cos, const float* rope_sin, int rope_rows,
                      int n_rope_q, int n_rope_k, void* workspace, long workspace_bytes, void* stream, int cu_cap);
}  // namespace samhip

constexpr long kScratchBytes = SAM_HIP_FLASH_NOALLOC_MAX_BYTES;  // 64 MiB
// The key-split count grows with the CU count, and the partial results with it; planning as for at most
// 256 CUs (an MI355X) makes a call's workspace need independent of the device, so a call that fits on
// one device fits on all.
constexpr int kPlanCUs = 256;

static __device__ __attribute__((aligned(256))) unsigned char scratch[kScratchBytes];

namespace {

// Device address of this device's copy of scratch (nullptr and a message on failure).
void* scratch_on_current_device(std::string* why) {
  static std::atomic<void*> ptrs[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *why = std::string("hipGetDevice: ") + hipGetErrorString(e);
    return nullptr;
  }
  if (dev < 0 || dev >= 64) {
    *why = "device ordinal beyond 63";
    return nullptr;
  }
  void* p = ptrs[dev].load(std::memory_order_acquire);
  if (p) return p;
  // Two threads may both get here for one device; they store the same address.
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    *why = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
    return nullptr;
  }
  ptrs[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace

extern "C" int sam_hip_flash_attn_noalloc(const void* q, const void* k, const void* v, void* out, int dtype, int b,
                                          int lq, int lk, int h, int d, const long* strides_q, const long* strides_k,
                                          const long* strides_v, const long* strides_o, float scale,
                                          const float* rope_cos, const float* rope_sin, int rope_rows, int n_rope_q,
                                          int n_rope_k, void* stream) {
  // The switch and the size checks first (no device call): the plan of sam_hip_flash_attn on a device of
  // at most kPlanCUs CUs.
  const long need = samhip::flash_workspace_size_capped(dtype, b, lq, lk, h, d, n_rope_k, kPlanCUs);
  if (!sam_hip_enabled() || need < 0)  // reports the switch or the size error
    return samhip::flash_attn_capped(q, k, v, out, dtype, b, lq, lk, h, d, strides_q, strides_k, strides_v, strides_o,
                                     scale, rope_cos, rope_sin, rope_rows, n_rope_q, n_rope_k, nullptr, 0, stream,
                                     kPlanCUs);
  if (need > kScratchBytes) {
    char buf[256];
    snprintf(buf, sizeof buf,
             "flash-attn-noalloc: this call needs %ld bytes of workspace, beyond the library's fixed %ld-byte "
             "array; use sam_hip_flash_attn with a caller workspace",
             need, kScratchBytes);
    return samhip::report_error(SAM_HIP_EUNSUPPORTED, buf);
  }
  void* ws = nullptr;
  if (need > 0) {
    std::string why;
    ws = scratch_on_current_device(&why);
    if (!ws) return samhip::report_error(SAM_HIP_EHIP, "flash-attn-noalloc: " + why);
  }
  return samhip::flash_attn_capped(q, k, v, out, dtype, b, lq, lk, h, d, strides_q, strides_k, strides_v, strides_o,
                                   scale, rope_cos, rope_sin, rope_rows, n_rope_q, n_rope_k, ws,
                                   need > 0 ? kScratchBytes : 0, stream, kPlanCUs);
}
