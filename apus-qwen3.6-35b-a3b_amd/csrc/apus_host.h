// apus_host.h -- small host-side helpers for the drop-in (host pointer)
// entry points: stage host arrays into library scratch, copy results back.
#pragma once
#include "apus_rt.h"

namespace apus {

// Copy `bytes` from host into scratch `slot`; returns the device pointer
// or nullptr (error already recorded).
inline void *stage_in(int slot, const void *host, size_t bytes) {
    void *d = scratch(slot, bytes);
    if (!d) return nullptr;
    if (bytes && hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice,
                                stream()) != hipSuccess) {
        set_error(kErrHip, "host->device copy of %zu bytes failed", bytes);
        return nullptr;
    }
    return d;
}

inline int stage_out(void *host, const void *dev, size_t bytes) {
    if (bytes)
        APUS_HIP_TRY(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost,
                                    stream()));
    APUS_HIP_TRY(hipStreamSynchronize(stream()));
    return kOk;
}

inline int launch_check(const char *name) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(kErrHip, "launch of %s failed: %s", name,
                         hipGetErrorString(e));
    return kOk;
}

inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace apus

#define APUS_STAGE(var, type, slot, host, bytes)                             \
    type *var = (type *)::apus::stage_in((slot), (host), (bytes));           \
    if (!var && (bytes)) return ::apus::kErrHip

#define APUS_LAUNCHED(name)                                                  \
    do {                                                                     \
        int r_ = ::apus::launch_check(name);                                 \
        if (r_ != ::apus::kOk) return r_;                                    \
    } while (0)
