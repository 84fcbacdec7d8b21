// gdn_mixer.h -- pieces of the batched GDN mixer shared by the decode
// (gdn_mixer.hip) and chunked prefill (gdn_prefill.hip) entry points.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/apus_hip.h"
#include "apus_rt.h"

namespace apus {

// Per-call device intermediates (library scratch).
struct GdnScratch {
    uint16_t *qk = nullptr;       // [Ttot][2][hk*128]: conv+SiLU codes of q, k
    float *qkr = nullptr;         // [Ttot][2][hk]: their l2norm factors (q, then k)
    uint16_t *vconv = nullptr;    // [Ttot][hv*128]: conv+SiLU of the v channels
    float2 *gate = nullptr;       // [Ttot][hv]: (exp(g), beta)
    uint16_t *ob = nullptr;       // [Ttot][hv*128]: rnd(recurrence output)
    float *graw = nullptr;        // [Ttot][hv]: g itself (log decay), when requested
};

// Token offsets of up to kGdnCuInline sequences by value (kernel
// arguments), so a small prefill needs no device copy of its metadata.
constexpr int kGdnCuInline = 256;
struct GdnCu {
    int32_t cu[kGdnCuInline + 1];
};

int gdn_check_layer(const ApusHipGdnLayer *L);
int gdn_check_offsets(size_t B, const int32_t *cu);
// conv + l2norm + gates for every token (reads the old conv state). The
// intermediates go to w's buffers when w->qk is set (a caller workspace),
// else to library scratch.
// Token offsets: dcu (device) when non-null, else from the host array cu
// by value (B <= kGdnCuInline). slots (device, nullable): the conv-state
// slot of each sequence (identity when null).
int gdn_prep(const ApusHipGdnLayer *L, size_t B, const int32_t *cu, const int32_t *dcu,
             size_t Ttot, const uint16_t *qkv, const uint16_t *a,
             const uint16_t *b, const uint16_t *conv_state, GdnScratch *w,
             bool want_graw, const int32_t *slots, const ApusHipGdnTrace *tr = nullptr);
// gated RMSNorm of w->ob into y, then the new conv state
int gdn_post(const ApusHipGdnLayer *L, size_t B, const int32_t *cu, const int32_t *dcu,
             size_t Ttot, const GdnScratch *w, const uint16_t *z,
             const uint16_t *qkv, uint16_t *conv_state, uint16_t *y, const int32_t *slots);

}  // namespace apus
