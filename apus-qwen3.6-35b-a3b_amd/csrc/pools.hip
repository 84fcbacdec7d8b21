// pools.hip -- device state managers for serving: a paged KV cache (blocks
// of 32 positions, a block table per sequence row) for the full-attention
// layers, and a pool of per-sequence GDN states (conv state + recurrent
// state) indexed by slot, for the linear-attention layers.
//
// The reference engine is single-sequence: each full-attention layer owns
// one flat [max_seq][nkv][d] cache and each GDN layer one state
// (c/layer.h:159-167, allocated per model at c/model.h:615-616), and its
// MTP path snapshots the GDN state and rewinds the cache position
// (c/mtp.h:70-75). Here many sequences share fixed device pools: a
// sequence takes KV blocks as it grows (no max_seq reservation) and a GDN
// slot for its lifetime; a rollback is a position rewind for the KV cache
// and an out-of-place decode for the GDN state
// (apus_hip_gdn_decode_slots with separate input and output slots).
//
// All bookkeeping is on the host; the device sees the block arrays, the
// block table and the state arrays. Table updates and slot zeroing are
// stream-ordered on the library stream (no host wait).
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "../../include/apus_hip.h"
#include "apus_host.h"
#include "apus_rt.h"

using namespace apus;

namespace {

constexpr int KVB = 32;

// zero n 16-byte units at p (a fill kernel: stream-ordered like the
// mixers, and never a memset node in a captured graph)
__global__ void k_zero16(uint4 *__restrict__ p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0, 0, 0, 0);
}

int zero_async(void *p, size_t bytes) {
    if (bytes % 16 || (uintptr_t)p % 16) return set_error(kErrArgument, "unaligned zero fill");
    const size_t n = bytes / 16;
    if (!n) return kOk;
    k_zero16<<<(unsigned)std::min<size_t>((n + 255) / 256, 1024), 256, 0, stream()>>>((uint4 *)p, n);
    return launch_check("k_zero16");
}

}  // namespace

struct ApusHipKvPool {
    size_t nlayers, nkv, d, nblocks, max_rows, max_blocks;
    std::vector<uint16_t *> k, v;          // per layer: nblocks blocks of nkv*32*d
    int32_t *dtab = nullptr;               // device [max_rows][max_blocks]
    std::vector<int32_t> htab;             // host copy of the table
    std::vector<int32_t> nused;            // blocks held per row; -1: row free
    std::vector<int32_t> free_blocks, free_rows;
};

struct ApusHipGdnPool {
    size_t nlayers, cd, hv, dk, dv, nslots;
    std::vector<uint16_t *> conv;          // per layer [nslots][cd*3] bf16
    std::vector<float *> S;                // per layer [nslots][hv][dk*dv] f32 (device layout)
    std::vector<char> used;
    std::vector<int32_t> free_slots;
};

extern "C" {

// ---- paged KV cache ---------------------------------------------------------

int apus_hip_kv_pool_create(size_t nlayers, size_t nkv, size_t d, size_t nblocks,
                            size_t max_rows, size_t max_blocks, ApusHipKvPool **out) {
    APUS_READY();
    if (!out) return set_error(kErrArgument, "NULL output");
    *out = nullptr;
    if (!nlayers || !nkv || d != 256 || !nblocks || !max_rows || !max_blocks ||
        nblocks > 0x7fffffff || max_blocks > 0x7fffffff || max_rows > 0x7fffffff)
        return set_error(kErrArgument, "bad KV pool dimensions (d must be 256)");
    auto *p = new ApusHipKvPool{nlayers, nkv, d, nblocks, max_rows, max_blocks, {}, {}, nullptr,
                                {}, {}, {}, {}};
    const size_t bytes = nblocks * nkv * KVB * d * 2;
    auto fail = [&](int r) {
        for (auto x : p->k) (void)hipFree(x);
        for (auto x : p->v) (void)hipFree(x);
        if (p->dtab) (void)hipFree(p->dtab);
        delete p;
        return r;
    };
    for (size_t l = 0; l < nlayers; l++) {
        void *a = nullptr, *b = nullptr;
        if (hipMalloc(&a, bytes) != hipSuccess)
            return fail(set_error(kErrHip, "hipMalloc of %zu bytes of KV blocks failed", bytes));
        p->k.push_back((uint16_t *)a);
        if (hipMalloc(&b, bytes) != hipSuccess)
            return fail(set_error(kErrHip, "hipMalloc of %zu bytes of KV blocks failed", bytes));
        p->v.push_back((uint16_t *)b);
    }
    const size_t tbytes = (max_rows * max_blocks * 4 + 15) / 16 * 16;
    if (hipMalloc((void **)&p->dtab, tbytes) != hipSuccess)
        return fail(set_error(kErrHip, "hipMalloc of the block table failed"));
    p->htab.assign(max_rows * max_blocks, 0);
    p->nused.assign(max_rows, -1);
    for (size_t i = nblocks; i-- > 0;) p->free_blocks.push_back((int32_t)i);
    for (size_t i = max_rows; i-- > 0;) p->free_rows.push_back((int32_t)i);
    // entries past a row's blocks hold block 0: a valid address, never read
    if (int r = zero_async(p->dtab, tbytes)) return fail(r);
    *out = p;
    return kOk;
}

int apus_hip_kv_pool_destroy(ApusHipKvPool *p) {
    APUS_READY();
    if (!p) return kOk;
    APUS_HIP_TRY(hipStreamSynchronize(stream()));
    for (auto x : p->k) (void)hipFree(x);
    for (auto x : p->v) (void)hipFree(x);
    (void)hipFree(p->dtab);
    delete p;
    return kOk;
}

int apus_hip_kv_pool_cache(const ApusHipKvPool *p, size_t layer, ApusHipKvCache *out) {
    if (!p || !out || layer >= p->nlayers) return set_error(kErrArgument, "bad pool or layer");
    out->k = p->k[layer];
    out->v = p->v[layer];
    out->block_table = p->dtab;
    out->max_blocks = p->max_blocks;
    out->max_rows = p->max_rows;
    out->row_blocks = p->nused.data();
    return kOk;
}

int apus_hip_kv_seq_open(ApusHipKvPool *p, int32_t *row) {
    if (!p || !row) return set_error(kErrArgument, "NULL argument");
    if (p->free_rows.empty()) return set_error(kErrUnsupported, "no free block-table row");
    *row = p->free_rows.back();
    p->free_rows.pop_back();
    p->nused[*row] = 0;
    return kOk;
}

int apus_hip_kv_seq_reserve(ApusHipKvPool *p, int32_t row, size_t ntok) {
    APUS_READY();
    if (!p || row < 0 || (size_t)row >= p->max_rows || p->nused[row] < 0)
        return set_error(kErrArgument, "row %d is not open", row);
    const size_t need = (ntok + KVB - 1) / KVB, have = (size_t)p->nused[row];
    if (need > p->max_blocks)
        return set_error(kErrArgument, "%zu positions exceed the %zu blocks of a row", ntok,
                         p->max_blocks);
    if (need <= have) return kOk;
    if (need - have > p->free_blocks.size())
        return set_error(kErrUnsupported, "KV pool exhausted (%zu blocks free, %zu needed)",
                         p->free_blocks.size(), need - have);
    int32_t *ent = p->htab.data() + (size_t)row * p->max_blocks;
    const size_t nfree = p->free_blocks.size();
    for (size_t b = have; b < need; b++) ent[b] = p->free_blocks[nfree - 1 - (b - have)];
    // the device table first: if its update cannot be enqueued, the host
    // bookkeeping stays as it was (the blocks remain free, the row its size)
    if (int r = copy_to_device_async(p->dtab + (size_t)row * p->max_blocks + have, ent + have,
                                     (need - have) * 4))
        return r;
    p->free_blocks.resize(nfree - (need - have));
    p->nused[row] = (int32_t)need;
    return kOk;
}

int apus_hip_kv_seq_close(ApusHipKvPool *p, int32_t row) {
    if (!p || row < 0 || (size_t)row >= p->max_rows || p->nused[row] < 0)
        return set_error(kErrArgument, "row %d is not open", row);
    const int32_t *ent = p->htab.data() + (size_t)row * p->max_blocks;
    for (int32_t b = p->nused[row]; b-- > 0;) p->free_blocks.push_back(ent[b]);
    p->nused[row] = -1;
    p->free_rows.push_back(row);
    return kOk;
}

size_t apus_hip_kv_pool_free_blocks(const ApusHipKvPool *p) {
    return p ? p->free_blocks.size() : 0;
}

// ---- GDN state pool -----------------------------------------------------------

int apus_hip_gdn_pool_create(size_t nlayers, size_t hk, size_t hv, size_t dk, size_t dv,
                             size_t nslots, ApusHipGdnPool **out) {
    APUS_READY();
    if (!out) return set_error(kErrArgument, "NULL output");
    *out = nullptr;
    if (!nlayers || !nslots || nslots > 0x7fffffff || dk != 128 || dv != 128 || hv != 2 * hk ||
        !hk)
        return set_error(kErrArgument, "bad GDN pool dimensions (dk = dv = 128, hv = 2 hk)");
    const size_t cd = 2 * hk * dk + hv * dv;
    auto *p = new ApusHipGdnPool{nlayers, cd, hv, dk, dv, nslots, {}, {}, {}, {}};
    auto fail = [&](int r) {
        for (auto x : p->conv) (void)hipFree(x);
        for (auto x : p->S) (void)hipFree(x);
        delete p;
        return r;
    };
    for (size_t l = 0; l < nlayers; l++) {
        void *a = nullptr, *b = nullptr;
        if (hipMalloc(&a, nslots * cd * 3 * 2) != hipSuccess)
            return fail(set_error(kErrHip, "hipMalloc of the conv-state pool failed"));
        p->conv.push_back((uint16_t *)a);
        if (hipMalloc(&b, nslots * hv * dk * dv * 4) != hipSuccess)
            return fail(set_error(kErrHip, "hipMalloc of the recurrent-state pool failed"));
        p->S.push_back((float *)b);
    }
    p->used.assign(nslots, 0);
    for (size_t i = nslots; i-- > 0;) p->free_slots.push_back((int32_t)i);
    *out = p;
    return kOk;
}

int apus_hip_gdn_pool_destroy(ApusHipGdnPool *p) {
    APUS_READY();
    if (!p) return kOk;
    APUS_HIP_TRY(hipStreamSynchronize(stream()));
    for (auto x : p->conv) (void)hipFree(x);
    for (auto x : p->S) (void)hipFree(x);
    delete p;
    return kOk;
}

int apus_hip_gdn_pool_state(const ApusHipGdnPool *p, size_t layer, uint16_t **conv, float **S) {
    if (!p || layer >= p->nlayers || !conv || !S) return set_error(kErrArgument, "bad pool or layer");
    *conv = p->conv[layer];
    *S = p->S[layer];
    return kOk;
}

int apus_hip_gdn_slot_open(ApusHipGdnPool *p, int32_t *slot) {
    APUS_READY();
    if (!p || !slot) return set_error(kErrArgument, "NULL argument");
    if (p->free_slots.empty()) return set_error(kErrUnsupported, "no free GDN state slot");
    const int32_t s = p->free_slots.back();
    // a new sequence starts from zero state (c/layer.h:219-227)
    for (size_t l = 0; l < p->nlayers; l++) {
        if (int r = zero_async(p->conv[l] + (size_t)s * p->cd * 3, p->cd * 3 * 2)) return r;
        if (int r = zero_async(p->S[l] + (size_t)s * p->hv * p->dk * p->dv, p->hv * p->dk * p->dv * 4))
            return r;
    }
    p->free_slots.pop_back();
    p->used[s] = 1;
    *slot = s;
    return kOk;
}

// Copy one sequence's state between a slot of one layer and caller arrays
// in the reference layout (conv [conv_dim*3] bf16, S [hv][dk][dv] f32;
// device pointers), stream-ordered.
static int slot_xfer(ApusHipGdnPool *p, size_t layer, int32_t slot, bool load, uint16_t *conv,
                     float *S) {
    if (!p || layer >= p->nlayers || slot < 0 || (size_t)slot >= p->nslots || !p->used[slot])
        return set_error(kErrArgument, "bad layer or slot %d is not open", slot);
    if (!conv || !S) return set_error(kErrArgument, "NULL state array");
    uint16_t *pc = p->conv[layer] + (size_t)slot * p->cd * 3;
    float *pS = p->S[layer] + (size_t)slot * p->hv * p->dk * p->dv;
    const size_t cb = p->cd * 3 * 2;
    if (load) {
        APUS_HIP_TRY(hipMemcpyAsync(pc, conv, cb, hipMemcpyDeviceToDevice, stream()));
        return apus_hip_gdn_state_pack(S, pS, p->hv);
    }
    APUS_HIP_TRY(hipMemcpyAsync(conv, pc, cb, hipMemcpyDeviceToDevice, stream()));
    return apus_hip_gdn_state_unpack(pS, S, p->hv);
}

int apus_hip_gdn_slot_load(ApusHipGdnPool *p, size_t layer, int32_t slot,
                           const uint16_t *conv, const float *S) {
    APUS_READY();
    return slot_xfer(p, layer, slot, true, const_cast<uint16_t *>(conv), const_cast<float *>(S));
}

int apus_hip_gdn_slot_store(ApusHipGdnPool *p, size_t layer, int32_t slot, uint16_t *conv,
                            float *S) {
    APUS_READY();
    return slot_xfer(p, layer, slot, false, conv, S);
}

int apus_hip_gdn_slot_close(ApusHipGdnPool *p, int32_t slot) {
    if (!p || slot < 0 || (size_t)slot >= p->nslots || !p->used[slot])
        return set_error(kErrArgument, "slot %d is not open", slot);
    p->used[slot] = 0;
    p->free_slots.push_back(slot);
    return kOk;
}

}  // extern "C"
