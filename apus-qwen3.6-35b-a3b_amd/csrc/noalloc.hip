// noalloc.hip -- the device memory of the allocation-free entry point
// (apus_hip_gdn_prefill_noalloc): one file-scope array per device, of a
// fixed size, that the entry point carves its intermediates from instead
// of allocating.
//
// In host code the array's name is only a host-side stand-in; the device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device at set-up (ensure_ready, with that device current) and kept here.
// Every call on a GPU shares that GPU's array and leaves its contents
// behind (nothing in it needs to start at zero); calls that overlap on one
// GPU race.
#include <hip/hip_runtime.h>

#include "apus_rt.h"

namespace apus {
namespace noalloc {
__device__ __align__(256) char scratch[kNoAllocScratchBytes];
}  // namespace noalloc

namespace {
constexpr int kMaxDevices = 64;
void *g_noalloc_ptr[kMaxDevices];
}  // namespace

int noalloc_setup(int dev) {
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(kErrUnsupported, "device index %d out of range", dev);
    if (g_noalloc_ptr[dev]) return kOk;
    void *p = nullptr;
    APUS_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc::scratch)));
    if (!p) return set_error(kErrHip, "no device address for the allocation-free scratch");
    g_noalloc_ptr[dev] = p;
    return kOk;
}

void *noalloc_scratch() {
    const int dev = current_device();
    return dev >= 0 && dev < kMaxDevices ? g_noalloc_ptr[dev] : nullptr;
}

}  // namespace apus
