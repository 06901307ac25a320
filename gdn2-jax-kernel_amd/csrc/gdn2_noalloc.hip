// gdn2_fwd_noalloc: the inference forward (gdn2_fwd's kernels) with its
// workspace in a fixed device array of this library, for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  Neither the caller nor the library
// allocates: the caller passes inputs and outputs only.
//
// The array `scratch` is a file-scope __device__ variable.  Its name in host code
// is a host-side stand-in, not a device address, so the device address is looked
// up once per device with hipGetSymbolAddress (on the entry point's first call
// on that device, with that device current) and kept per device; every launch
// uses that address.  The device is the stream's (the kernels run there), which
// need not be the caller's current device: the lookup then makes the stream's
// device current for its duration and restores the caller's.  Each GPU the
// library runs on holds its own copy of the array (GDN2_NOALLOC_SCRATCH_BYTES,
// in every process that loads the library, whether or not it calls this entry
// point) until the process ends.  Calls on one GPU share its array: calls that
// overlap on one GPU (different streams, or threads without ordering) race on
// it and must be serialised by the caller.  Nothing in the array needs to start
// at zero -- the forward writes every workspace tile (and clears the segmented
// scan's saturation flag) before reading it -- so the previous call's contents
// are harmless.
#include <hip/hip_runtime.h>

#include <atomic>
#include <stddef.h>

#include "gdn2.h"
#include "gdn2_layout.h"

namespace gdn2 {

int fwd_entry(void* stream, int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
              const void* q, const void* k, const void* v, const void* w, const void* b,
              const void* g, const float* h0, float scale, float* out, float* h_final,
              void* ws, size_t ws_bytes, float* a_dbg, int flags);
size_t fwd_workspace_need(int B, int T, int H, int D, int BT, int in_dtype, int g_dtype,
                          int flags);

namespace {

constexpr size_t kScratchBytes = GDN2_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` per device, resolved on first use.
std::atomic<void*> g_scratch[kMaxDevices];

// The scratch address on the device `stream` belongs to (the current device for
// the null stream), or nullptr if it cannot be resolved.
void* scratch_ptr(hipStream_t stream) {
  int cur = 0, dev = 0;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  dev = cur;
  if (stream && hipStreamGetDevice(stream, &dev) != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    // idempotent: concurrent first calls store the same address
    if (dev != cur && hipSetDevice(dev) != hipSuccess) return nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) return nullptr;
    g_scratch[dev].store(p, std::memory_order_release);
  }
  return p;
}

}  // namespace
}  // namespace gdn2

extern "C" int gdn2_fwd_noalloc(void* stream, int B, int T, int H, int D, int BT,
                                int in_dtype, int g_dtype, const void* q, const void* k,
                                const void* v, const void* w, const void* b, const void* g,
                                const float* h0, float scale, float* out, float* h_final,
                                int flags) {
  using namespace gdn2;
  if (flags & GDN2_FWD_SAVE_A) return GDN2_ERR_FLAGS;   // residuals would not survive
  flags = (flags & ~kFwdNoARegion) | kFwdNoARegion;
  const size_t need = fwd_workspace_need(B, T, H, D, BT, in_dtype, g_dtype, flags);
  if (need > kScratchBytes) return GDN2_ERR_SCRATCH;
  // need == 0: invalid shapes, which fwd_entry reports with their own code, or
  // an empty sequence, which launches no kernel that reads the workspace
  void* ws = need > 0 ? scratch_ptr((hipStream_t)stream) : nullptr;
  if (need > 0 && !ws) return GDN2_ERR_LAUNCH;
  return fwd_entry(stream, B, T, H, D, BT, in_dtype, g_dtype, q, k, v, w, b, g, h0, scale, out,
                   h_final, ws, need > 0 ? kScratchBytes : 0, nullptr, flags);
}
