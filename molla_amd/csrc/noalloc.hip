// noalloc.hip -- mi_matvec_noalloc: mi_matvec without a workspace argument,
// for callers that cannot allocate device memory (code under HIP graph
// capture, serving loops that forbid hipMalloc).  It has no counterpart in
// the reference.
//
// The workspace is `scratch`, a file-scope device array of
// MI_MATVEC_NOALLOC_BYTES.  Each GPU holds its own copy at its own address
// from module load until the process ends.  Host code never passes the
// array's name to a kernel (in host code it is only a stand-in for the
// symbol): the first call on a device, with that device current, resolves
// the device address with hipGetSymbolAddress and keeps it per device.
// Nothing in the matvec workspace has to start at zero (the activation form
// and split-K partial sums are written before they are read), and every call
// on one GPU shares the array, so calls that overlap on one GPU (on
// different streams) race.
#include <mutex>

#include "mi_internal.h"

static __device__ __align__(256) uint8_t scratch[MI_MATVEC_NOALLOC_BYTES];

namespace {

void* g_scratch[mi::kMaxDevices];
std::mutex g_scratch_lock;

// The current device's address of `scratch`, resolved once per device.
int scratch_of_current_device(void** out) {
  int dev = 0;
  int rc = mi::hip_check(hipGetDevice(&dev), "matvec_noalloc: current device");
  if (rc) return rc;
  if (dev < 0 || dev >= mi::kMaxDevices)
    return mi::fail(MI_ERR_DEVICE, "matvec_noalloc: device %d beyond %d", dev, mi::kMaxDevices);
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    rc = mi::hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "matvec_noalloc: scratch address");
    if (rc) return rc;
    if (!p || ((uintptr_t)p & 255)) return mi::fail(MI_ERR_DEVICE, "matvec_noalloc: scratch at %p", p);
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return MI_OK;
}

}  // namespace

extern "C" int mi_matvec_noalloc(mi_stream stream, int kind, const void* w, int64_t row_bytes, int32_t rows,
                                 int32_t cols, const float* x, int32_t tokens, float* y, int32_t epi,
                                 const float* aux) {
  const size_t need = mi_matvec_workspace(cols, tokens);
  if (need == 0) return mi::fail(MI_ERR_SHAPE, "matvec_noalloc: %d columns at %d tokens", cols, tokens);
  if (need > MI_MATVEC_NOALLOC_BYTES)
    return mi::fail(MI_ERR_WORKSPACE, "matvec_noalloc: %d columns at %d tokens need %zu bytes of workspace, above "
                    "the static %u", cols, tokens, need, (unsigned)MI_MATVEC_NOALLOC_BYTES);
  void* work = nullptr;
  int rc = scratch_of_current_device(&work);
  if (rc) return rc;
  return mi_matvec(stream, kind, w, row_bytes, rows, cols, x, tokens, y, epi, aux, work, MI_MATVEC_NOALLOC_BYTES);
}
