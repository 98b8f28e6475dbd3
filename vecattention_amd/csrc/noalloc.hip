// Allocation-free decode attention: va_decode_attn_noalloc.
//
// For callers that cannot call hipMalloc (code under HIP graph capture, tight
// serving loops, harnesses that forbid allocation).  It runs the same kernels
// as va_decode_attn; the partial softmax states that va_decode_attn keeps in
// the caller's workspace live here in `scratch`, a file-scope device array of
// kScratchBytes: every GPU the library runs on holds its own copy until the
// process ends.  Calls on one GPU share that copy, so calls that overlap on
// one GPU (different streams, no ordering between them) race; calls ordered on
// one stream do not.  The split kernel writes every partial the merge kernel
// reads, so nothing needs clearing between calls.
#include <mutex>

#include "../../include/vecattn.h"
#include "common.h"

namespace va {
int api_error(int code, const char* fmt, ...);
int decode_run(int dtype, const void* q, int64_t sqh, const void* k, int64_t skh, int64_t sks,
               const void* v, int64_t svh, int64_t svs, void* out, int64_t soh, int64_t Hq,
               int64_t Hk, int64_t L, int64_t D, float softmax_scale, int kernel,
               void* workspace, int64_t workspace_bytes, void* stream);
}  // namespace va

namespace {

constexpr int64_t kScratchBytes = int64_t(8) << 20;  // 8 MiB per GPU

// The partial states of va_decode_attn_noalloc.  Host code never passes this
// name to a kernel: its host-side symbol is not a device address.  The device
// address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) float scratch[kScratchBytes / 4];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_addr[kMaxDevices];  // device address of `scratch`, per device

// Device address of `scratch` on the current device, looked up on the first
// call on that device (with that device current) and kept.
int scratch_address(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return va::api_error(VA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return va::api_error(VA_ERR_UNSUPPORTED, "device %d: at most %d devices are supported", dev,
                         kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return va::api_error(VA_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                           hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return VA_OK;
}

}  // namespace

extern "C" {

int64_t va_decode_noalloc_scratch_bytes(void) { return kScratchBytes; }

int va_decode_attn_noalloc(int dtype, const void* q, int64_t sqh, const void* k, int64_t skh,
                           int64_t sks, const void* v, int64_t svh, int64_t svs, void* out,
                           int64_t soh, int64_t Hq, int64_t Hk, int64_t L, int64_t D,
                           float softmax_scale, int kernel, void* stream) {
  const int64_t need = va_decode_workspace_size(Hq, Hk, L, D);
  if (need < 0) return va::api_error(VA_ERR_ARG, "invalid decode sizes");
  if (need > kScratchBytes)
    return va::api_error(VA_ERR_UNSUPPORTED,
                         "allocation-free decode holds at most %lld bytes of partial states; "
                         "Hq=%lld, Hk=%lld, L=%lld, D=%lld need %lld (use va_decode_attn with a "
                         "workspace)",
                         (long long)kScratchBytes, (long long)Hq, (long long)Hk, (long long)L,
                         (long long)D, (long long)need);
  void* addr = nullptr;
  const int rc = scratch_address(&addr);
  if (rc) return rc;
  return va::decode_run(dtype, q, sqh, k, skh, sks, v, svh, svs, out, soh, Hq, Hk, L, D,
                        softmax_scale, kernel, addr, kScratchBytes, stream);
}

}  // extern "C"
