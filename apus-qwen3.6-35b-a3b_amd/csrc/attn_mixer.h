// attn_mixer.h -- shared pieces of the batched gated-GQA mixer.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/apus_hip.h"
#include "apus_rt.h"

namespace apus {

// Per-call sequence metadata, passed by value as a kernel argument for up
// to kAttnInlineSeqs sequences (no host->device copy on the decode path).
constexpr int kAttnInlineSeqs = 224;
struct AttnSeqs {
    int32_t n;                          // sequences
    int32_t ks1, ks2;                   // keys per score split / per P.V split
    int32_t cu[kAttnInlineSeqs + 1];    // token offsets
    int32_t pos0[kAttnInlineSeqs];      // tokens already cached
    int32_t soff[kAttnInlineSeqs + 1];  // score-split offsets
    int32_t soff2[kAttnInlineSeqs + 1]; // P.V-split offsets
};

int attn_check_layer(const ApusHipAttnLayer *L);

// q/k (1+w) RMSNorm, RoPE at each token's position, append k and v to the
// device caches; writes the roped q into qn [Ttot, nh, d].
// dmeta: device copy of the metadata when it does not fit by value (else
// NULL); max_pos: one past the largest position written (RoPE table size);
// maxnb: attn_max_vblocks of the call.
int attn_prep(const ApusHipAttnLayer *L, const AttnSeqs &sq, const int32_t *dmeta,
              size_t Ttot, size_t max_pos, int maxnb, const uint16_t *qg, const uint16_t *k,
              const uint16_t *v, uint16_t *kcache, uint16_t *vcache, size_t max_seq,
              uint16_t *qn);

// the most 32-position V-cache blocks one sequence's new tokens touch
int attn_max_vblocks(size_t B, const int32_t *cu, const int32_t *pos0);

}  // namespace apus
