// apus_rt.h -- host runtime of libapus_hip: error reporting, the current
// stream, grow-only device scratch, pinned staging and the RoPE table.
//
// Conventions follow the reference's backend hooks (c/backend_metal.h:
// 16-20, 79-88; c/bf16.h:199-205, 250-259): every entry point returns
// int, 0 when it handled the op and nonzero otherwise, with a message
// retrievable through apus_hip_last_error. One compute thread drives the
// library (c/pool.h:7-16 model); it is not safe for concurrent callers.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/apus_hip.h"

namespace apus {

enum Status : int {
    kOk = 0,
    kErrUnsupported = 1,   // shape/config not handled: caller uses its CPU op
    kErrDisabled = 2,      // APUS_HIP_DISABLE set or library not initialised
    kErrArgument = 3,      // invalid argument
    kErrHip = 4,           // HIP runtime error
};

int set_error(int code, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what, const char *file, int line);

// Lazily initialises the device on first use (device 0 unless
// apus_hip_init chose another). Returns kOk or an error code.
int ensure_ready();
hipStream_t stream();
int cu_count();     // compute units of the current device
int current_device();

// bf16-code activation tables (act_tables.hip): for every bf16 code c,
// silu_bf[c] = rnd(x*sigmoid(x)), silu_f[c] = x*sigmoid(x) (fp32) and
// sig_bf[c] = rnd(sigmoid(x)), x = the value of c. Device pointers, filled
// on the library stream at the first call on a device.
struct ActTables {
    const uint16_t *silu_bf = nullptr;
    const float *silu_f = nullptr;
    const uint16_t *sig_bf = nullptr;
};
const ActTables *act_tables();
void set_stream(hipStream_t s);

// Grow-only device scratch, one buffer per slot. Valid until the next
// call with the same slot and a larger size.
enum ScratchSlot { kScratchIn = 0, kScratchIn2, kScratchIn3, kScratchIn4,
                   kScratchIn5, kScratchIn6, kScratchOut, kScratchOut2,
                   kScratchWork, kScratchWork2, kScratchWork3, kScratchMeta,
                   kScratchMeta2, kScratchMeta3,
                   // batched GDN mixer intermediates
                   kScratchGdnQK, kScratchGdnQKR, kScratchGdnV, kScratchGdnGate, kScratchGdnOB,
                   kScratchGdnChunk, kScratchGdnChunk2, kScratchGdnChunk3,
                   kScratchGdnChunk4, kScratchGdnChunk5,
                   kScratchGdnChunk6, kScratchGdnChunk7,
                   // batched attention mixer intermediates
                   kScratchAttnQ, kScratchAttnA, kScratchAttnStat,
                   kScratchAttnPart,
                   // layer entry points: projection outputs, mixer output
                   kScratchLayerA, kScratchLayerB, kScratchLayerC, kScratchLayerD,
                   kScratchLayerY,
                   kScratchSlots };
void *scratch(int slot, size_t bytes);

// Device RoPE table for (rot, theta): [npos][rot] bf16 codes, per
// position cos for pairs 0..rot/2-1 then sin. Computed on the host with
// the platform libm exactly as c/attn.h:251-255 and uploaded; grows to
// cover positions 0..max_pos-1.
const uint16_t *rope_table(size_t rot, double theta, size_t max_pos);

// Stream-ordered upload of a host array through a pinned staging ring: the
// returned device copy is valid for the work the caller enqueues before
// its next upload; the host array may be reused on return; no wait for the
// GPU (the ring recycles a chunk once work enqueued after it completed).
const void *upload_async(const void *host, size_t bytes);
// host -> device copy into caller memory, stream-ordered, without waiting
// (staged through the ring).
int copy_to_device_async(void *dst, const void *host, size_t bytes);

// The allocation-free entry point's per-device scratch (noalloc.hip): its
// size, the set-up taking its device address (once per device, device
// current), and that address for the current device (nullptr before set-up).
constexpr size_t kNoAllocScratchBytes = (size_t)96 << 20;
int noalloc_setup(int dev);
void *noalloc_scratch();

// Device fault word: kernels with bounded waits (k_attn_scores' producer /
// consumer ring) OR a kFault* bit into it when a wait expires, then run on
// to a normal exit; apus_hip_synchronize reads and clears it and reports
// a set bit as an error. spin_limit(): the polls such a wait makes before
// it gives up (apus_hip_set_spin_limit; default kDefaultSpinLimit, about
// a quarter of a second of polling).
constexpr uint32_t kFaultScoresWait = 1u;
constexpr uint32_t kDefaultSpinLimit = 1u << 22;
uint32_t *fault_word();
uint32_t spin_limit();

// The trace sinks set by apus_hip_trace_set (nullptr when tracing is off).
const ApusHipGdnTrace *gdn_trace();
const ApusHipAttnTrace *attn_trace();

// Opt-in per-kernel timing: when enabled (apus_hip_timing_enable), a pair
// of events is recorded on the library stream around each wrapped launch;
// apus_hip_timing_get sums them per kernel name. Disabled: one branch.
int timing_begin(const char *name);
void timing_end(int slot);

}  // namespace apus

#define APUS_TIMED(name, ...)                                                \
    do {                                                                     \
        int ts_ = ::apus::timing_begin(name);                                \
        __VA_ARGS__;                                                         \
        ::apus::timing_end(ts_);                                             \
    } while (0)

#define APUS_HIP_TRY(expr)                                                   \
    do {                                                                     \
        hipError_t e_ = (expr);                                              \
        if (e_ != hipSuccess)                                                \
            return ::apus::hip_fail(e_, #expr, __FILE__, __LINE__);          \
    } while (0)

#define APUS_READY()                                                         \
    do {                                                                     \
        int r_ = ::apus::ensure_ready();                                     \
        if (r_ != ::apus::kOk) return r_;                                    \
    } while (0)
