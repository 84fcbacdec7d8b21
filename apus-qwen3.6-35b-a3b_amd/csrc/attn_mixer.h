// attn_mixer.h -- shared pieces of the batched gated-GQA mixer: the KV
// cache's block addressing and the per-call sequence metadata.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/apus_hip.h"
#include "apus_rt.h"
#include "apus_dev.h"

namespace apus {

// ---- KV cache blocks ------------------------------------------------------
// The cache is a set of blocks of KVB = 32 positions. Block b (positions
// 32b .. 32b+31) of the sequence whose block-table row is h has the id
//     id = btab ? btab[h * bstride + b] : h * bstride + b
// and lives at
//     K: k + id * nkv*32*D, laid out [nkv][32][D]   (rows: d contiguous)
//     V: v + id * nkv*D*32, laid out [nkv][D][32]   (transposed)
// The flat layout of apus_hip_attn_decode / _prefill is the identity table
// (row h = the sequence's batch index, bstride = max_seq / 32): each
// sequence's blocks are consecutive. A paged cache (apus_hip_kv_pool_*)
// passes its block table. K rows keep d contiguous for the QK^T MFMA
// operand; V is transposed so the P.V operand is 8 consecutive keys of one
// d in one 16-byte load, and a kv head's 32 keys x 256 d are one
// contiguous 16 KiB piece.
constexpr int KVB = 32;
struct KvRef {
    uint16_t *k, *v;
    const int32_t *btab;        // nullptr: identity (flat) table
    int32_t bstride;            // blocks per table row
};
__device__ __forceinline__ size_t kv_block_id(const KvRef &r, int h, int b) {
    return r.btab ? (size_t)r.btab[(size_t)h * r.bstride + b] : (size_t)h * r.bstride + b;
}
// the same for a wave-uniform (h, b): a scalar load into a scalar register,
// so addresses built on it stay scalar bases and the lookup never waits on
// (or makes the compiler drain) the vector-memory counter
__device__ __forceinline__ size_t kv_block_id_u(const KvRef &r, int h, int b) {
    if (!r.btab) return (size_t)h * r.bstride + b;
    const int hu = __builtin_amdgcn_readfirstlane(h), bu = __builtin_amdgcn_readfirstlane(b);
    return (size_t)(uint32_t)sload_i32(r.btab + (size_t)hu * r.bstride, (uint32_t)r.bstride * 4, bu);
}

// ---- per-call sequence metadata ------------------------------------------
// Passed by value as a kernel argument for up to kAttnInlineSeqs sequences
// (no host->device copy on the decode path), else as a device array
// cu[B+1] | pos0[B] | ccap[B+1] | hd[B].
constexpr int kAttnInlineSeqs = 224;
struct AttnSeqs {
    int32_t n;                          // sequences
    int32_t T1, T2;                     // keys per score / P.V wavefront (multiples of 64)
    int32_t cu[kAttnInlineSeqs + 1];    // token offsets
    int32_t pos0[kAttnInlineSeqs];      // tokens already cached
    int32_t ccap[kAttnInlineSeqs + 1];  // prefix sums of cap = ceil64(pos0 + tokens)
    int32_t hd[kAttnInlineSeqs];        // block-table row of each sequence
};

int attn_check_layer(const ApusHipAttnLayer *L);

// Metadata of one call: checks the offsets and positions against the cache
// capacity (bstride blocks per sequence), fills sq (by value) or uploads
// the device copy (*dmeta), and for decode picks the per-wavefront key
// counts T1 / T2 of the balanced splits (max_tok: most tokens of one
// sequence). rows: block-table row per sequence (NULL: the batch index).
int attn_meta(size_t B, const int32_t *cu, const int32_t *pos0, const int32_t *rows,
              size_t bstride, size_t nkv, int max_new, AttnSeqs *sq, const int32_t **dmeta,
              size_t *max_tok);

// q/k (1+w) RMSNorm, RoPE at each token's position, append k and v to the
// cache; writes the roped q into qn [Ttot, nh, d] (with qrows false, only
// the k rows and the appends: the caller forms q itself). max_pos: one past
// the largest position written (RoPE table size); maxnb: attn_max_vblocks.
int attn_prep(const ApusHipAttnLayer *L, const AttnSeqs &sq, const int32_t *dmeta,
              size_t Ttot, size_t max_pos, int maxnb, const uint16_t *qg, const uint16_t *k,
              const uint16_t *v, const KvRef &kv, uint16_t *qn, bool qrows = true);

// the most 32-position cache blocks one sequence's new tokens touch
int attn_max_vblocks(size_t B, const int32_t *cu, const int32_t *pos0);

// Flat-layout KvRef of B sequences of max_seq positions each.
KvRef kv_flat(uint16_t *kcache, uint16_t *vcache, size_t max_seq);

// The KvRef of a paged cache for a call of B sequences at table rows
// rows[s] writing positions up to pos0[s] + (cu[s+1] - cu[s]): refuses a
// row outside the table and, when the descriptor carries the rows'
// reserved block counts, a closed row or one that has not reserved the
// blocks the call writes.
int kv_paged_ref(const ApusHipKvCache *c, size_t B, const int32_t *rows, const int32_t *cu,
                 const int32_t *pos0, KvRef *r);

// Prefill on a cache given as a KvRef (flat or paged).
int attn_prefill_kv(const ApusHipAttnLayer *L, size_t B, const int32_t *cu, const int32_t *pos0,
                    const int32_t *rows, const uint16_t *qg, const uint16_t *k,
                    const uint16_t *v, const KvRef &kv, uint16_t *y);
// Decode on a cache given as a KvRef (flat or paged).
int attn_decode_kv(const ApusHipAttnLayer *L, size_t B, const int32_t *cu, const int32_t *pos0,
                   const int32_t *rows, const uint16_t *qg, const uint16_t *k,
                   const uint16_t *v, const KvRef &kv, uint16_t *y);

}  // namespace apus
