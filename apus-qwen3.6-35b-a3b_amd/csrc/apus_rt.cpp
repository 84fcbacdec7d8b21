// apus_rt.cpp -- host runtime of libapus_hip (see apus_rt.h).
#include "apus_rt.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <deque>
#include <vector>

#include "../../include/apus_hip.h"

namespace apus {
namespace {

char g_err[512];
int g_ready = 0;
int g_device = 0;
int g_cus = 256;
hipStream_t g_stream = nullptr;
uint32_t *g_fault = nullptr;           // device fault word of the current device
uint32_t g_spin = kDefaultSpinLimit;

struct Buf {
    void *p = nullptr;
    size_t n = 0;
};
Buf g_scratch[kScratchSlots];

struct RopeTab {
    size_t rot = 0;
    double theta = 0.0;
    size_t npos = 0;
    uint16_t *dev = nullptr;
};
RopeTab g_rope;

// RNE narrow on the host, c/bf16.h:268-274 rule.
uint16_t host_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(u >> 16);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

struct TimedKernel {
    const char *name;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
};
bool g_timing = false;
std::vector<TimedKernel> g_timed;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void timing_clear() {
    for (auto &k : g_timed)
        for (auto &p : k.ev) {
            g_event_pool.push_back(p.first);
            g_event_pool.push_back(p.second);
        }
    g_timed.clear();
}

bool disabled_by_env() {
    const char *e = getenv("APUS_HIP_DISABLE");
    return e && *e && strcmp(e, "0") != 0;
}

}  // namespace

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char *what, const char *file, int line) {
    return set_error(kErrHip, "%s failed: %s (%s:%d)", what,
                     hipGetErrorString(e), file, line);
}

int ensure_ready() {
    if (disabled_by_env())
        return set_error(kErrDisabled, "disabled by APUS_HIP_DISABLE");
    if (g_ready) return kOk;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return set_error(kErrDisabled, "no HIP device visible (%s)",
                         hipGetErrorString(e));
    if (g_device >= n)
        return set_error(kErrArgument, "device %d out of range (%d)",
                         g_device, n);
    APUS_HIP_TRY(hipSetDevice(g_device));
    hipDeviceProp_t prop;
    APUS_HIP_TRY(hipGetDeviceProperties(&prop, g_device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return set_error(kErrUnsupported,
                         "device %d is %s; this build targets gfx950",
                         g_device, prop.gcnArchName);
    g_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    g_ready = 1;
    // device set-up the allocation-free entry relies on: its scratch's
    // address and the activation tables (allocated here, never in it)
    if (int r = noalloc_setup(g_device)) {
        g_ready = 0;
        return r;
    }
    if (!act_tables()) {
        g_ready = 0;
        return kErrHip;
    }
    if (!g_fault) {
        if (hipMalloc((void **)&g_fault, 256) != hipSuccess ||
            hipMemset(g_fault, 0, 256) != hipSuccess) {
            g_ready = 0;
            g_fault = nullptr;
            return set_error(kErrHip, "allocation of the device fault word failed");
        }
    }
    return kOk;
}

uint32_t *fault_word() { return g_fault; }
uint32_t spin_limit() { return g_spin; }

int cu_count() { return g_cus; }
int current_device() { return g_device; }

hipStream_t stream() { return g_stream; }
void set_stream(hipStream_t s) { g_stream = s; }

void *scratch(int slot, size_t bytes) {
    Buf &b = g_scratch[slot];
    if (bytes == 0) bytes = 1;
    if (b.n >= bytes) return b.p;
    if (b.p) {
        // pending work may still use the old buffer
        if (hipStreamSynchronize(g_stream) != hipSuccess) return nullptr;
        (void)hipFree(b.p);
        b.p = nullptr;
        b.n = 0;
    }
    size_t want = bytes + bytes / 4;
    if (hipMalloc(&b.p, want) != hipSuccess) {
        b.p = nullptr;
        set_error(kErrHip, "hipMalloc of %zu bytes failed", want);
        return nullptr;
    }
    b.n = want;
    return b.p;
}

// ---- stream-ordered uploads through a pinned ring ------------------------
// Host bytes are copied into a pinned staging ring and sent with an
// asynchronous copy into the matching offset of a device ring, so the
// caller's array is free on return and nothing waits for the GPU. A chunk
// is reused only after an event recorded at a later upload -- i.e. after
// every kernel enqueued before that upload, which includes the chunk's
// consumers -- has completed.
namespace {
struct UploadRing {
    char *host = nullptr, *dev = nullptr;
    size_t cap = 0, head = 0;
    struct Mark {
        size_t begin, end;
        hipEvent_t ev;
    };
    std::deque<Mark> live;
};
UploadRing g_ring;

int ring_reserve(size_t cap) {
    UploadRing &r = g_ring;
    if (r.cap >= cap) return kOk;
    if (r.dev) {
        APUS_HIP_TRY(hipStreamSynchronize(g_stream));
        for (auto &m : r.live)
            if (m.ev) g_event_pool.push_back(m.ev);
        r.live.clear();
        (void)hipFree(r.dev);
        (void)hipHostFree(r.host);
        r.dev = r.host = nullptr;
        r.cap = r.head = 0;
    }
    APUS_HIP_TRY(hipMalloc((void **)&r.dev, cap));
    if (hipHostMalloc((void **)&r.host, cap, hipHostMallocDefault) != hipSuccess) {
        (void)hipFree(r.dev);
        r.dev = nullptr;
        return set_error(kErrHip, "hipHostMalloc of %zu bytes failed", cap);
    }
    r.cap = cap;
    r.head = 0;
    return kOk;
}
}  // namespace

// Stage `bytes` of host data in the ring and copy them to dst (nullptr:
// the ring's own device chunk); returns the device address or nullptr.
static void *ring_put(void *dst, const void *host, size_t bytes) {
    UploadRing &r = g_ring;
    const size_t n = std::max<size_t>((bytes + 255) / 256 * 256, 256);
    if (ring_reserve(std::max<size_t>(n * 4, (size_t)4 << 20)) != kOk) return nullptr;
    // the previous chunk's consumers are all enqueued by now
    if (!r.live.empty() && !r.live.back().ev) {
        hipEvent_t e = take_event();
        if (!e || hipEventRecord(e, g_stream) != hipSuccess) {
            set_error(kErrHip, "event record failed");
            return nullptr;
        }
        r.live.back().ev = e;
    }
    if (r.head + n > r.cap) r.head = 0;
    const size_t b = r.head, en = b + n;
    // wait for (and retire) every live chunk overlapping [b, en)
    for (auto it = r.live.begin(); it != r.live.end();) {
        if (it->begin < en && b < it->end) {
            if (hipEventSynchronize(it->ev) != hipSuccess) {
                set_error(kErrHip, "event wait failed");
                return nullptr;
            }
            g_event_pool.push_back(it->ev);
            it = r.live.erase(it);
        } else {
            ++it;
        }
    }
    if (bytes) memcpy(r.host + b, host, bytes);
    void *to = dst ? dst : r.dev + b;
    if (bytes &&
        hipMemcpyAsync(to, r.host + b, bytes, hipMemcpyHostToDevice, g_stream) != hipSuccess) {
        set_error(kErrHip, "upload of %zu bytes failed", bytes);
        return nullptr;
    }
    r.live.push_back(UploadRing::Mark{b, en, nullptr});
    r.head = en;
    return to;
}

const void *upload_async(const void *host, size_t bytes) {
    return ring_put(nullptr, host, bytes);
}

int copy_to_device_async(void *dst, const void *host, size_t bytes) {
    return ring_put(dst, host, bytes) ? kOk : kErrHip;
}

const uint16_t *rope_table(size_t rot, double theta, size_t max_pos) {
    if (g_rope.dev && g_rope.rot == rot && g_rope.theta == theta &&
        g_rope.npos >= max_pos)
        return g_rope.dev;
    size_t npos = max_pos < 4096 ? 4096 : max_pos;
    if (g_rope.dev && g_rope.rot == rot && g_rope.theta == theta &&
        npos < g_rope.npos * 2)
        npos = g_rope.npos * 2;
    size_t R = rot / 2;
    std::vector<float> invf(R);
    for (size_t i = 0; i < R; i++)
        invf[i] = (float)(1.0 / pow(theta, 2.0 * (double)i / (double)rot));
    std::vector<uint16_t> tab(npos * rot);
    for (size_t p = 0; p < npos; p++) {
        float pos = (float)p;
        uint16_t *row = tab.data() + p * rot;
        for (size_t i = 0; i < R; i++) {
            float ang = pos * invf[i];
            row[i] = host_bf16(cosf(ang));
            row[R + i] = host_bf16(sinf(ang));
        }
    }
    if (g_rope.dev) {
        if (hipStreamSynchronize(g_stream) != hipSuccess) return nullptr;
        (void)hipFree(g_rope.dev);
        g_rope.dev = nullptr;
    }
    if (hipMalloc(&g_rope.dev, tab.size() * 2) != hipSuccess) {
        g_rope.dev = nullptr;
        set_error(kErrHip, "hipMalloc of the rope table failed");
        return nullptr;
    }
    if (hipMemcpy(g_rope.dev, tab.data(), tab.size() * 2,
                  hipMemcpyHostToDevice) != hipSuccess) {
        set_error(kErrHip, "rope table upload failed");
        return nullptr;
    }
    g_rope.rot = rot;
    g_rope.theta = theta;
    g_rope.npos = npos;
    return g_rope.dev;
}

namespace {
ApusHipGdnTrace g_gdn_trace;
ApusHipAttnTrace g_attn_trace;
bool g_gdn_traced = false, g_attn_traced = false;
}  // namespace

const ApusHipGdnTrace *gdn_trace() { return g_gdn_traced ? &g_gdn_trace : nullptr; }
const ApusHipAttnTrace *attn_trace() { return g_attn_traced ? &g_attn_trace : nullptr; }

int timing_begin(const char *name) {
    if (!g_timing) return -1;
    size_t i = 0;
    while (i < g_timed.size() && strcmp(g_timed[i].name, name) != 0) i++;
    if (i == g_timed.size()) g_timed.push_back(TimedKernel{name, {}});
    hipEvent_t a = take_event(), b = take_event();
    if (!a || !b) return -1;
    if (hipEventRecord(a, g_stream) != hipSuccess) return -1;
    g_timed[i].ev.emplace_back(a, b);
    return (int)i;
}

void timing_end(int slot) {
    if (slot < 0 || (size_t)slot >= g_timed.size() || g_timed[slot].ev.empty()) return;
    (void)hipEventRecord(g_timed[slot].ev.back().second, g_stream);
}

}  // namespace apus

using namespace apus;

extern "C" {

int apus_hip_init(int device, char *err, size_t errcap) {
    if (device != g_device) g_fault = nullptr;   // each device gets its own word
    g_device = device;
    g_ready = 0;
    int r = ensure_ready();
    if (r != kOk && err && errcap) snprintf(err, errcap, "%s", g_err);
    return r;
}

int apus_hip_is_enabled(void) { return ensure_ready() == kOk; }

size_t apus_hip_last_error(char *buf, size_t cap) {
    size_t n = strlen(g_err);
    if (buf && cap) snprintf(buf, cap, "%s", g_err);
    return n;
}

int apus_hip_set_stream(void *s) {
    APUS_READY();
    set_stream((hipStream_t)s);
    return kOk;
}

int apus_hip_synchronize(void) {
    APUS_READY();
    APUS_HIP_TRY(hipStreamSynchronize(g_stream));
    uint32_t f = 0;
    APUS_HIP_TRY(hipMemcpy(&f, g_fault, 4, hipMemcpyDeviceToHost));
    if (f) {
        APUS_HIP_TRY(hipMemset(g_fault, 0, 4));
        return set_error(kErrHip, "a kernel's bounded wait expired (fault bits 0x%x: %s); the "
                         "results of the work since the last synchronize are invalid", f,
                         (f & kFaultScoresWait) ? "k_attn_scores score ring" : "unknown");
    }
    return kOk;
}

int apus_hip_set_spin_limit(uint32_t polls) {
    g_spin = polls ? polls : kDefaultSpinLimit;
    return kOk;
}

int apus_hip_malloc(void **dptr, size_t bytes) {
    APUS_READY();
    if (!dptr) return set_error(kErrArgument, "dptr is NULL");
    APUS_HIP_TRY(hipMalloc(dptr, bytes ? bytes : 1));
    return kOk;
}

int apus_hip_free(void *dptr) {
    APUS_READY();
    APUS_HIP_TRY(hipFree(dptr));
    return kOk;
}

int apus_hip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    APUS_READY();
    APUS_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                                g_stream));
    APUS_HIP_TRY(hipStreamSynchronize(g_stream));
    return kOk;
}

int apus_hip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    APUS_READY();
    APUS_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                                g_stream));
    APUS_HIP_TRY(hipStreamSynchronize(g_stream));
    return kOk;
}

int apus_hip_timing_enable(int on) {
    APUS_READY();
    APUS_HIP_TRY(hipStreamSynchronize(g_stream));
    timing_clear();
    g_timing = on != 0;
    return kOk;
}

int apus_hip_timing_get(const char *name, double *total_ms, size_t *count) {
    APUS_READY();
    if (!name || !total_ms || !count) return set_error(kErrArgument, "NULL argument");
    APUS_HIP_TRY(hipStreamSynchronize(g_stream));
    *total_ms = 0.0;
    *count = 0;
    for (auto &k : g_timed) {
        if (strcmp(k.name, name) != 0) continue;
        for (auto &p : k.ev) {
            float ms = 0.0f;
            APUS_HIP_TRY(hipEventElapsedTime(&ms, p.first, p.second));
            *total_ms += ms;
        }
        *count = k.ev.size();
    }
    return kOk;
}

int apus_hip_trace_set(const ApusHipGdnTrace *gdn, const ApusHipAttnTrace *attn) {
    g_gdn_traced = gdn != nullptr;
    g_attn_traced = attn != nullptr;
    if (gdn) g_gdn_trace = *gdn;
    if (attn) g_attn_trace = *attn;
    return kOk;
}

int apus_hip_memset(void *dst, int value, size_t bytes) {
    APUS_READY();
    APUS_HIP_TRY(hipMemsetAsync(dst, value, bytes, g_stream));
    return kOk;
}

}  // extern "C"
