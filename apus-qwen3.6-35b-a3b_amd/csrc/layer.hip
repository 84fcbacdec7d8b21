// layer.hip -- one hybrid-model layer's token mixer with the projections on
// either side of it (c/layer.h:236-286 for a GDN layer, :288-331 for a
// full-attention layer): ln1 (the layer's normed input, [Ttot][H]) in,
// ao (the mixer's output projection, [Ttot][H]) out, for B sequences of
// 1..k new tokens (decode / MTP verify).
//
// The input projections the reference runs as separate gemvs over the
// same ln1 -- in_proj_qkv, _z, _b, _a (c/layer.h:250-253), or wq, wk, wv
// (c/layer.h:300-302) -- are ONE MFMA GEMM launch here: its output rows
// come from the weight matrices in turn and its epilogue stores each
// segment's columns straight into the layout the mixer reads (qkv, z, b, a
// or qg, k, v), so ln1 is read once and no split or copy follows. Then the
// fused decode mixer (gdn_mixer.hip / attn_mixer.hip), then w_out / wo on
// the mixer's output (c/layer.h:274, :322).
//
// Fusing the projections into the mixer kernels themselves does not pay
// at decode batch sizes: a mixer workgroup owns one (sequence, head), so
// each would re-read its head's weight slice (the GDN in_proj slice of a K
// head is 3.2 MB, w_out's 1 MB) once per sequence -- B times the weight
// bytes, against the 2-6 MB of activations per step the separate GEMMs
// move through HBM.
#include <stdint.h>

#include "../../include/apus_hip.h"
#include "apus_host.h"
#include "attn_mixer.h"
#include "gdn_mixer.h"
#include "proj.h"

using namespace apus;

namespace {

int check_w(const uint16_t *p, const char *what) {
    if (!p) return set_error(kErrArgument, "NULL %s", what);
    if ((uintptr_t)p % 16) return set_error(kErrUnsupported, "%s must be 16-byte aligned", what);
    return kOk;
}

// The GDN layer: in_proj (qkv | z | b | a) -> mixer -> w_out. slot_in /
// slot_out: the state pool's slot maps (HOST), or null for the flat state
// arrays.
int gdn_layer_run(const ApusHipGdnLayer *L, const ApusHipGdnProj *P, size_t B,
                  const int32_t *slot_in, const int32_t *slot_out, const int32_t *cu,
                  const uint16_t *ln1, uint16_t *conv, float *S, uint16_t *ao) {
    if (int r = gdn_check_layer(L)) return r;
    if (!P) return set_error(kErrArgument, "NULL projections");
    if (B == 0) return kOk;
    if (int r = gdn_check_offsets(B, cu)) return r;
    const size_t H = P->hidden, T = (size_t)cu[B];
    const size_t cd = 2 * L->hk * L->dk + L->hv * L->dv, vd = L->hv * L->dv, hv = L->hv;
    if (H == 0 || H % 32 || vd % 32 || hv % 32)
        return set_error(kErrUnsupported, "GDN layer projections need hidden, value_dim and hv "
                         "multiples of 32 (hidden=%zu hv=%zu)", H, hv);
    for (auto [p, n] : {std::pair{P->w_qkv, "w_qkv"}, {P->w_z, "w_z"}, {P->w_b, "w_b"},
                        {P->w_a, "w_a"}, {P->w_out, "w_out"}})
        if (int r = check_w(p, n)) return r;
    if (int r = check_w(ln1, "ln1")) return r;
    if (!ao) return set_error(kErrArgument, "NULL output");
    if (T == 0) return kOk;
    if (int r = gemm_tile_check(ln1, T, cd + vd + 2 * hv, H)) return r;
    if (int r = gemm_tile_check(ln1, T, H, vd)) return r;
    uint16_t *qkv = (uint16_t *)scratch(kScratchLayerA, T * cd * 2);
    uint16_t *z = (uint16_t *)scratch(kScratchLayerB, T * vd * 2);
    uint16_t *ab = (uint16_t *)scratch(kScratchLayerC, T * 2 * hv * 2);
    uint16_t *y = (uint16_t *)scratch(kScratchLayerY, T * vd * 2);
    if (!qkv || !z || !ab || !y) return kErrHip;
    uint16_t *a = ab, *b = ab + T * hv;
    GemmSegs in{};
    in.n = 4;
    in.row0[0] = 0;
    in.row0[1] = (int)cd;
    in.row0[2] = (int)(cd + vd);
    in.row0[3] = (int)(cd + vd + hv);
    in.row0[4] = (int)(cd + vd + 2 * hv);
    in.w[0] = P->w_qkv; in.y[0] = qkv; in.ldy[0] = (int)cd;
    in.w[1] = P->w_z;   in.y[1] = z;   in.ldy[1] = (int)vd;
    in.w[2] = P->w_b;   in.y[2] = b;   in.ldy[2] = (int)hv;
    in.w[3] = P->w_a;   in.y[3] = a;   in.ldy[3] = (int)hv;
    if (int r = gemm_tile(in, ln1, T, H, "k_gemm_tile_in")) return r;
    const int rc = slot_in ? apus_hip_gdn_decode_slots(L, B, slot_in, slot_out, cu, qkv, z, a, b,
                                                       conv, S, y)
                           : apus_hip_gdn_decode(L, B, cu, qkv, z, a, b, conv, S, y);
    if (rc) return rc;
    GemmSegs out{};
    out.n = 1;
    out.row0[1] = (int)H;
    out.w[0] = P->w_out; out.y[0] = ao; out.ldy[0] = (int)H;
    return gemm_tile(out, y, T, vd, "k_gemm_tile_out");
}

// The full-attention layer: wq | wk | wv -> mixer -> wo. rows: the paged
// cache's block-table rows (HOST), or null for the flat cache (kv built by
// the caller).
int attn_layer_run(const ApusHipAttnLayer *L, const ApusHipAttnProj *P, size_t B,
                   const int32_t *rows, const int32_t *cu, const int32_t *pos0,
                   const uint16_t *ln1, const KvRef &kv, uint16_t *ao) {
    if (int r = attn_check_layer(L)) return r;
    if (!P) return set_error(kErrArgument, "NULL projections");
    if (B == 0) return kOk;
    if (int r = gdn_check_offsets(B, cu)) return r;
    const size_t H = P->hidden, T = (size_t)cu[B];
    const size_t nq = L->nh * 2 * L->d, nk = L->nkv * L->d, no = L->nh * L->d;
    if (H == 0 || H % 32)
        return set_error(kErrUnsupported, "attention layer projections need hidden a multiple "
                         "of 32 (hidden=%zu)", H);
    for (auto [p, n] : {std::pair{P->wq, "wq"}, {P->wk, "wk"}, {P->wv, "wv"}, {P->wo, "wo"}})
        if (int r = check_w(p, n)) return r;
    if (int r = check_w(ln1, "ln1")) return r;
    if (!ao) return set_error(kErrArgument, "NULL output");
    if (T == 0) return kOk;
    if (int r = gemm_tile_check(ln1, T, nq + 2 * nk, H)) return r;
    if (int r = gemm_tile_check(ln1, T, H, no)) return r;
    uint16_t *qg = (uint16_t *)scratch(kScratchLayerA, T * nq * 2);
    uint16_t *k = (uint16_t *)scratch(kScratchLayerB, T * nk * 2);
    uint16_t *v = (uint16_t *)scratch(kScratchLayerC, T * nk * 2);
    uint16_t *y = (uint16_t *)scratch(kScratchLayerY, T * no * 2);
    if (!qg || !k || !v || !y) return kErrHip;
    GemmSegs in{};
    in.n = 3;
    in.row0[1] = (int)nq;
    in.row0[2] = (int)(nq + nk);
    in.row0[3] = (int)(nq + 2 * nk);
    in.w[0] = P->wq; in.y[0] = qg; in.ldy[0] = (int)nq;
    in.w[1] = P->wk; in.y[1] = k;  in.ldy[1] = (int)nk;
    in.w[2] = P->wv; in.y[2] = v;  in.ldy[2] = (int)nk;
    if (int r = gemm_tile(in, ln1, T, H, "k_gemm_tile_in")) return r;
    if (int r = attn_decode_kv(L, B, cu, pos0, rows, qg, k, v, kv, y)) return r;
    GemmSegs out{};
    out.n = 1;
    out.row0[1] = (int)H;
    out.w[0] = P->wo; out.y[0] = ao; out.ldy[0] = (int)H;
    return gemm_tile(out, y, T, no, "k_gemm_tile_out");
}

}  // namespace

extern "C" {

int apus_hip_gdn_layer_decode(const ApusHipGdnLayer *L, const ApusHipGdnProj *P, size_t B,
                              const int32_t *cu, const uint16_t *ln1, uint16_t *conv_state,
                              float *S, uint16_t *ao) {
    APUS_READY();
    return gdn_layer_run(L, P, B, nullptr, nullptr, cu, ln1, conv_state, S, ao);
}

int apus_hip_gdn_layer_decode_slots(const ApusHipGdnLayer *L, const ApusHipGdnProj *P, size_t B,
                                    const int32_t *slot_in, const int32_t *slot_out,
                                    const int32_t *cu, const uint16_t *ln1, uint16_t *conv,
                                    float *S, uint16_t *ao) {
    APUS_READY();
    if (B && (!slot_in || !slot_out)) return set_error(kErrArgument, "NULL slot map");
    return gdn_layer_run(L, P, B, slot_in, slot_out, cu, ln1, conv, S, ao);
}

int apus_hip_attn_layer_decode(const ApusHipAttnLayer *L, const ApusHipAttnProj *P, size_t B,
                               const int32_t *cu, const int32_t *pos0, const uint16_t *ln1,
                               uint16_t *kcache, uint16_t *vcache, size_t max_seq,
                               uint16_t *ao) {
    APUS_READY();
    if (max_seq % KVB != 0) return set_error(kErrArgument, "max_seq must be a multiple of %d", KVB);
    return attn_layer_run(L, P, B, nullptr, cu, pos0, ln1, kv_flat(kcache, vcache, max_seq), ao);
}

int apus_hip_attn_layer_decode_paged(const ApusHipAttnLayer *L, const ApusHipAttnProj *P,
                                     size_t B, const int32_t *rows, const int32_t *cu,
                                     const int32_t *pos0, const uint16_t *ln1,
                                     const ApusHipKvCache *kv, uint16_t *ao) {
    APUS_READY();
    KvRef r;
    if (int e = kv_paged_ref(kv, B, rows, cu, pos0, &r)) return e;
    return attn_layer_run(L, P, B, rows, cu, pos0, ln1, r, ao);
}

}  // extern "C"
