// Device scratch for the entry points that allocate nothing.
//
// Some callers cannot call hipMalloc (HIP-graph capture, tight serving loops,
// harnesses that forbid it).  For them the split-K decode partials live in
// one file-scope device array per GPU instead of a caller workspace.  The
// array's host-side name is only a registration handle, not a device address:
// hipGetSymbolAddress, called once per device with that device current (on
// the first no-alloc call on that device), yields each GPU's own copy, and
// every launch uses that pointer.  Every call on one GPU shares its array and
// the array keeps the last call's contents; the decode kernels overwrite
// every partial they read, so nothing needs clearing, but calls that overlap
// on one GPU race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.h"

namespace qxh {

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices];  // per device, resolved once
}  // namespace

hipError_t noalloc_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_scratch[device]) return hipSuccess;
    int current = -1;
    hipError_t e = hipGetDevice(&current);
    if (e != hipSuccess) return e;
    if (current != device) return hipErrorInvalidDevice;  // the caller makes `device` current
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch[device] = p;
    return hipSuccess;
}

void* noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    return g_scratch[device];
}

}  // namespace qxh
