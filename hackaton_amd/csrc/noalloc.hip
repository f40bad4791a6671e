// The attention backward for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc): va_bwd_noalloc takes the same
// inputs and outputs as va_bwd but no workspace. The per-query-head dK/dV partials that va_bwd
// keeps in its workspace live here in a file-scope device array, `scratch`, which every GPU the
// library runs on holds (kNoAllocScratchBytes each) until the process ends.
//
// On the host the name `scratch` is only a stand-in for the symbol: its device address is fetched
// once per device with hipGetSymbolAddress (with that device current, at the first call that runs
// on it) and only that address is ever passed to kernels. Every call on one GPU shares that GPU's
// array: calls that overlap on one GPU (two streams, or two threads) race on it. Nothing in it
// needs to start at zero: each call's kernels write every partial row of the rows its plan covers
// before the GQA sum reads it (rows the plan does not cover come back as whatever the last call
// left there, as with an uninitialised workspace in va_bwd).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../../include/varlen_attn.h"
#include "va_api_internal.h"
#include "va_kernels.h"

namespace {

// The partials of N * Hq <= 131072 rows at head_dim 128 (64 MiB), the row flags (4 N bytes) and
// the row statistics (8 N Hq bytes).
constexpr int64_t kNoAllocScratchBytes = int64_t(66) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::once_flag g_once[kMaxDevices];
void* g_scratch[kMaxDevices];     // device address of `scratch` on each device
hipError_t g_status[kMaxDevices];

// Device address of this device's scratch array (looked up once per device).
int scratch_of(int device, void** ptr) {
  if (device < 0 || device >= kMaxDevices)
    return va::fail(VA_EINVAL, "va_bwd_noalloc: device %d out of range", device);
  std::call_once(g_once[device], [device] {
    int current = -1;
    g_status[device] = hipGetDevice(&current);
    if (g_status[device] != hipSuccess) return;
    if (current != device && (g_status[device] = hipSetDevice(device)) != hipSuccess) return;
    void* p = nullptr;
    g_status[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch[device] = p;
    if (current != device) {
      const hipError_t e = hipSetDevice(current);
      if (g_status[device] == hipSuccess) g_status[device] = e;
    }
  });
  if (g_status[device] != hipSuccess || g_scratch[device] == nullptr)
    return va::fail((int)g_status[device], "va_bwd_noalloc: hipGetSymbolAddress(scratch): %s",
                    hipGetErrorString(g_status[device]));
  *ptr = g_scratch[device];
  return VA_OK;
}

}  // namespace

extern "C" int64_t va_bwd_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int va_bwd_noalloc(const void* dout, const void* q, const void* k, const void* v,
                              const void* out, const float* lse, const int32_t* items,
                              int64_t n_items, int64_t total_tokens, int32_t hq, int32_t hkv,
                              int32_t head_dim, float scale, int32_t dtype, void* dq, void* dk,
                              void* dv, void* stream) {
  if (dk == nullptr || dv == nullptr)
    return va::fail(VA_EINVAL, "va_bwd_noalloc: dk and dv are required (the partials stay in "
                               "the library's scratch memory)");
  int64_t offs[2], need = 0;
  int rc = va_bwd_workspace_layout(total_tokens, hq, hkv, head_dim, offs, &need);
  if (rc) return rc;
  if (hq == hkv || total_tokens == 0)  // no partials: dK/dV are written directly
    return va::bwd_checked(-1, dout, q, k, v, out, lse, items, n_items, total_tokens, hq, hkv,
                           head_dim, scale, dtype, dq, dk, dv, nullptr, 0, stream, nullptr);
  if (need > kNoAllocScratchBytes)
    return va::fail(VA_ECAPACITY,
                    "va_bwd_noalloc: total_tokens=%lld x Hq=%d needs %lld bytes of dK/dV "
                    "partials, the static scratch holds %lld (total_tokens * Hq <= %lld); use "
                    "va_bwd with a workspace",
                    (long long)total_tokens, hq, (long long)need, (long long)kNoAllocScratchBytes,
                    (long long)(kNoAllocScratchBytes / (2 * 2 * head_dim)));
  int device = -1;
  hipError_t e = hipStreamGetDevice((hipStream_t)stream, &device);
  if (e != hipSuccess)
    return va::fail((int)e, "va_bwd_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
  void* ws = nullptr;
  if ((rc = scratch_of(device, &ws))) return rc;
  return va::bwd_checked(-1, dout, q, k, v, out, lse, items, n_items, total_tokens, hq, hkv,
                         head_dim, scale, dtype, dq, dk, dv, ws, kNoAllocScratchBytes, stream,
                         nullptr);
}
