/*
 * tests/c_host/host_layer.c -- a C11 host on include/apus_hip.h.
 *
 * The reference engine is C11 and calls its attention ops directly from
 * its layer code (c/layer.h:236-331 decode, 427-564 prefill). This program
 * stands in for that engine: it drives one Gated DeltaNet layer and one
 * gated-GQA layer through the tier-2 entry points with the reference's
 * fail-soft hook pattern (c/bf16.h:199-205: a nonzero return means "run
 * the CPU kernel"), and the weak stubs a CPU-only build links
 * (c/bf16.h:250-259), here as weak references to the shared library.
 * Built twice: linked against libapus_hip.so, and without it (every entry
 * point then resolves to NULL and each call site takes the CPU path).
 *
 * Usage: host_layer OUTDIR. Prints "hip" when every call ran on the GPU,
 * "fallback <reason>" when the engine would have stayed on its CPU path.
 * With "hip" it writes the inputs and results as raw little-endian arrays
 * OUTDIR/<name>.bin for the test to check against the oracle:
 *   GDN: 3 sequences prefilled from zero state (70, 5, 33 tokens), then one
 *        decode token each; conv state and S (reference layout) after.
 *   GQA: 2 sequences prefilled from position 0 (40, 7 tokens) into a flat
 *        cache, then a verify step of 2 and 1 tokens.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "apus_hip.h"

/* ---- weak references: a binary built without libapus_hip links
 * unchanged, every entry point then resolves to NULL, and each call site
 * falls through to the CPU kernel (the role of the reference's weak
 * Metal stubs, c/bf16.h:250-259, for a shared library: a weak DEFINITION
 * in the executable would shadow the library's at run time) ---------- */
#pragma weak apus_hip_init
#pragma weak apus_hip_last_error
#pragma weak apus_hip_malloc
#pragma weak apus_hip_free
#pragma weak apus_hip_memcpy_h2d
#pragma weak apus_hip_memcpy_d2h
#pragma weak apus_hip_synchronize
#pragma weak apus_hip_gdn_state_unpack
#pragma weak apus_hip_gdn_prefill
#pragma weak apus_hip_gdn_decode
#pragma weak apus_hip_attn_prefill
#pragma weak apus_hip_attn_decode
#pragma weak apus_hip_attn_cache_unpack
#define HIP_LINKED(fn) ((fn) != NULL)

/* ---- deterministic inputs ------------------------------------------------ */
static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64(void) {                     /* splitmix64 */
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double uniform01(void) { return (double)(next_u64() >> 11) * 0x1.0p-53; }
static float normal(void) {                          /* Box-Muller */
    double u = uniform01(), v = uniform01();
    if (u < 1e-300) u = 1e-300;
    return (float)(sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v));
}
static uint16_t bf16_of(float x) {                   /* RNE, c/bf16.h:268-274 rule */
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(u >> 16);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
static uint16_t *bf16_normal(size_t n, float std, float mean) {
    uint16_t *p = malloc(n * 2);
    for (size_t i = 0; i < n; i++) p[i] = bf16_of(normal() * std + mean);
    return p;
}

/* ---- device helpers with the fail-soft convention ------------------------ */
static const char *g_outdir;
static char g_reason[512];

static int fail(const char *what) {
    char msg[400] = "";
    if (HIP_LINKED(apus_hip_last_error)) apus_hip_last_error(msg, sizeof msg);
    snprintf(g_reason, sizeof g_reason, "%s: %s", what, msg);
    return 1;
}
static void *dev_copy(const void *h, size_t n) {
    void *d = NULL;
    if (apus_hip_malloc(&d, n) != 0) return NULL;
    if (h && apus_hip_memcpy_h2d(d, h, n) != 0) return NULL;
    return d;
}
static void dump(const char *name, const void *h, size_t n) {
    char path[1024];
    snprintf(path, sizeof path, "%s/%s.bin", g_outdir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(h, 1, n, f) != n) {
        fprintf(stderr, "cannot write %s\n", path);
        exit(3);
    }
    fclose(f);
}
static int dump_dev(const char *name, const void *d, size_t n) {
    void *h = malloc(n);
    if (apus_hip_memcpy_d2h(h, d, n) != 0) return fail(name);
    dump(name, h, n);
    free(h);
    return 0;
}

/* ---- the GDN layer: prefill then decode (c/layer.h:427-492, 236-286) ---- */
static int gdn_layer(void) {
    enum { HK = 16, HV = 32, DK = 128, DV = 128, CD = 2 * HK * DK + HV * DV, VD = HV * DV };
    const size_t B = 3;
    const int32_t cu_p[4] = {0, 70, 75, 108}, cu_d[4] = {0, 1, 2, 3};
    const size_t Tp = 108, Td = 3;
    uint16_t *conv_w = bf16_normal((size_t)CD * 4, 0.1f, 0.0f);
    float A_log[HV], dt_bias[HV];
    for (int h = 0; h < HV; h++) {
        A_log[h] = (float)(uniform01() * 2.7);
        dt_bias[h] = 1.0f;
    }
    uint16_t *onorm_w = bf16_normal(DV, 0.1f, 1.0f);
    uint16_t *qkv_p = bf16_normal(Tp * CD, 1, 0), *z_p = bf16_normal(Tp * VD, 1, 0);
    uint16_t *a_p = bf16_normal(Tp * HV, 1, 0), *b_p = bf16_normal(Tp * HV, 1, 0);
    uint16_t *qkv_d = bf16_normal(Td * CD, 1, 0), *z_d = bf16_normal(Td * VD, 1, 0);
    uint16_t *a_d = bf16_normal(Td * HV, 1, 0), *b_d = bf16_normal(Td * HV, 1, 0);
    dump("gdn_conv_w", conv_w, (size_t)CD * 4 * 2);
    dump("gdn_A_log", A_log, sizeof A_log);
    dump("gdn_dt_bias", dt_bias, sizeof dt_bias);
    dump("gdn_onorm_w", onorm_w, DV * 2);
    dump("gdn_qkv_p", qkv_p, Tp * CD * 2);
    dump("gdn_z_p", z_p, Tp * VD * 2);
    dump("gdn_a_p", a_p, Tp * HV * 2);
    dump("gdn_b_p", b_p, Tp * HV * 2);
    dump("gdn_qkv_d", qkv_d, Td * CD * 2);
    dump("gdn_z_d", z_d, Td * VD * 2);
    dump("gdn_a_d", a_d, Td * HV * 2);
    dump("gdn_b_d", b_d, Td * HV * 2);

    if (!HIP_LINKED(apus_hip_malloc)) return fail("apus_hip_malloc");
    ApusHipGdnLayer L = {HK, HV, DK, DV, dev_copy(conv_w, (size_t)CD * 4 * 2),
                         dev_copy(A_log, sizeof A_log), dev_copy(dt_bias, sizeof dt_bias),
                         dev_copy(onorm_w, DV * 2)};
    /* zero state (apus_layer_state_zero, c/layer.h:219-227) */
    uint16_t *conv0 = calloc(B * CD * 3, 2);
    float *S0 = calloc(B * HV * DK * DV, 4);
    uint16_t *d_conv = dev_copy(conv0, B * CD * 3 * 2);
    float *d_S = dev_copy(S0, B * HV * DK * DV * 4);   /* zeros: same in both layouts */
    uint16_t *d_qkv_p = dev_copy(qkv_p, Tp * CD * 2), *d_z_p = dev_copy(z_p, Tp * VD * 2);
    uint16_t *d_a_p = dev_copy(a_p, Tp * HV * 2), *d_b_p = dev_copy(b_p, Tp * HV * 2);
    uint16_t *d_qkv_d = dev_copy(qkv_d, Td * CD * 2), *d_z_d = dev_copy(z_d, Td * VD * 2);
    uint16_t *d_a_d = dev_copy(a_d, Td * HV * 2), *d_b_d = dev_copy(b_d, Td * HV * 2);
    uint16_t *d_y_p = dev_copy(NULL, Tp * VD * 2), *d_y_d = dev_copy(NULL, Td * VD * 2);
    float *d_Sref = dev_copy(NULL, B * HV * DK * DV * 4);
    if (!L.conv_w || !L.A_log || !L.dt_bias || !L.onorm_w || !d_conv || !d_S || !d_y_p ||
        !d_y_d || !d_Sref || !d_qkv_p || !d_qkv_d)
        return fail("gdn buffers");

    /* the hook pattern of the layer call sites: not linked or nonzero ->
     * the engine runs its CPU kernel (here: report and stop) */
    if (!HIP_LINKED(apus_hip_gdn_prefill) ||
        apus_hip_gdn_prefill(&L, B, cu_p, d_qkv_p, d_z_p, d_a_p, d_b_p, d_conv, d_S, d_y_p) != 0)
        return fail("apus_hip_gdn_prefill");
    if (!HIP_LINKED(apus_hip_gdn_decode) ||
        apus_hip_gdn_decode(&L, B, cu_d, d_qkv_d, d_z_d, d_a_d, d_b_d, d_conv, d_S, d_y_d) != 0)
        return fail("apus_hip_gdn_decode");
    if (apus_hip_gdn_state_unpack(d_S, d_Sref, B * HV) != 0) return fail("state unpack");
    if (apus_hip_synchronize() != 0) return fail("synchronize");
    if (dump_dev("gdn_y_p", d_y_p, Tp * VD * 2) || dump_dev("gdn_y_d", d_y_d, Td * VD * 2) ||
        dump_dev("gdn_conv", d_conv, B * CD * 3 * 2) ||
        dump_dev("gdn_S", d_Sref, B * HV * DK * DV * 4))
        return 1;
    void *bufs[] = {(void *)L.conv_w, (void *)L.A_log, (void *)L.dt_bias, (void *)L.onorm_w,
                    d_conv, d_S, d_qkv_p, d_z_p, d_a_p, d_b_p, d_qkv_d, d_z_d, d_a_d, d_b_d,
                    d_y_p, d_y_d, d_Sref};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) apus_hip_free(bufs[i]);
    free(conv_w); free(onorm_w); free(qkv_p); free(z_p); free(a_p); free(b_p);
    free(qkv_d); free(z_d); free(a_d); free(b_d); free(conv0); free(S0);
    return 0;
}

/* ---- the GQA layer: prefill then verify (c/layer.h:498-564, 288-331) ---- */
static int attn_layer(void) {
    enum { NH = 16, NKV = 2, D = 256, MAXSEQ = 64 };
    const size_t B = 2;
    const int32_t cu_p[3] = {0, 40, 47}, pos_p[2] = {0, 0};
    const int32_t cu_d[3] = {0, 2, 3}, pos_d[2] = {40, 7};
    const size_t Tp = 47, Td = 3;
    uint16_t *qn_w = bf16_normal(D, 0.1f, 0), *kn_w = bf16_normal(D, 0.1f, 0);
    uint16_t *qg_p = bf16_normal(Tp * NH * 2 * D, 1, 0), *k_p = bf16_normal(Tp * NKV * D, 1, 0);
    uint16_t *v_p = bf16_normal(Tp * NKV * D, 1, 0);
    uint16_t *qg_d = bf16_normal(Td * NH * 2 * D, 1, 0), *k_d = bf16_normal(Td * NKV * D, 1, 0);
    uint16_t *v_d = bf16_normal(Td * NKV * D, 1, 0);
    dump("attn_qn_w", qn_w, D * 2);
    dump("attn_kn_w", kn_w, D * 2);
    dump("attn_qg_p", qg_p, Tp * NH * 2 * D * 2);
    dump("attn_k_p", k_p, Tp * NKV * D * 2);
    dump("attn_v_p", v_p, Tp * NKV * D * 2);
    dump("attn_qg_d", qg_d, Td * NH * 2 * D * 2);
    dump("attn_k_d", k_d, Td * NKV * D * 2);
    dump("attn_v_d", v_d, Td * NKV * D * 2);
    ApusHipAttnLayer L = {NH, NKV, D, 64, 1e7, dev_copy(qn_w, D * 2), dev_copy(kn_w, D * 2)};
    const size_t cache = B * MAXSEQ * NKV * D * 2;
    uint16_t *d_k = dev_copy(NULL, cache), *d_v = dev_copy(NULL, cache);
    uint16_t *d_qg_p = dev_copy(qg_p, Tp * NH * 2 * D * 2), *d_k_p = dev_copy(k_p, Tp * NKV * D * 2);
    uint16_t *d_v_p = dev_copy(v_p, Tp * NKV * D * 2);
    uint16_t *d_qg_d = dev_copy(qg_d, Td * NH * 2 * D * 2), *d_k_d = dev_copy(k_d, Td * NKV * D * 2);
    uint16_t *d_v_d = dev_copy(v_d, Td * NKV * D * 2);
    uint16_t *d_y_p = dev_copy(NULL, Tp * NH * D * 2), *d_y_d = dev_copy(NULL, Td * NH * D * 2);
    uint16_t *d_kr = dev_copy(NULL, MAXSEQ * NKV * D * 2), *d_vr = dev_copy(NULL, MAXSEQ * NKV * D * 2);
    if (!L.qn_w || !L.kn_w || !d_k || !d_v || !d_y_p || !d_y_d || !d_kr || !d_vr)
        return fail("attention buffers");
    if (!HIP_LINKED(apus_hip_attn_prefill) ||
        apus_hip_attn_prefill(&L, B, cu_p, pos_p, d_qg_p, d_k_p, d_v_p, d_k, d_v, MAXSEQ, d_y_p))
        return fail("apus_hip_attn_prefill");
    if (!HIP_LINKED(apus_hip_attn_decode) ||
        apus_hip_attn_decode(&L, B, cu_d, pos_d, d_qg_d, d_k_d, d_v_d, d_k, d_v, MAXSEQ, d_y_d))
        return fail("apus_hip_attn_decode");
    if (apus_hip_synchronize() != 0) return fail("synchronize");
    if (dump_dev("attn_y_p", d_y_p, Tp * NH * D * 2) || dump_dev("attn_y_d", d_y_d, Td * NH * D * 2))
        return 1;
    for (size_t s = 0; s < B; s++) {            /* caches in the reference layout */
        const size_t n = (size_t)pos_d[s] + (size_t)(cu_d[s + 1] - cu_d[s]);
        const size_t per = (size_t)MAXSEQ * NKV * D;
        char nk[32], nv[32];
        if (apus_hip_attn_cache_unpack(d_k + s * per, d_v + s * per, n, NKV, D, MAXSEQ, d_kr, d_vr))
            return fail("cache unpack");
        snprintf(nk, sizeof nk, "attn_kc%zu", s);
        snprintf(nv, sizeof nv, "attn_vc%zu", s);
        if (dump_dev(nk, d_kr, n * NKV * D * 2) || dump_dev(nv, d_vr, n * NKV * D * 2)) return 1;
    }
    void *bufs[] = {(void *)L.qn_w, (void *)L.kn_w, d_k, d_v, d_qg_p, d_k_p, d_v_p, d_qg_d,
                    d_k_d, d_v_d, d_y_p, d_y_d, d_kr, d_vr};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) apus_hip_free(bufs[i]);
    free(qn_w); free(kn_w); free(qg_p); free(k_p); free(v_p); free(qg_d); free(k_d); free(v_d);
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s OUTDIR\n", argv[0]);
        return 2;
    }
    g_outdir = argv[1];
    char err[256];
    /* enable once at start-up, next to apus_metal_enable (c/bf16.h:250) */
    if (!HIP_LINKED(apus_hip_init)) {
        printf("fallback init: hip backend not linked\n");
        return 0;
    }
    if (apus_hip_init(0, err, sizeof err) != 0) {
        printf("fallback init: %s\n", err);
        return 0;
    }
    if (gdn_layer() != 0 || attn_layer() != 0) {
        printf("fallback %s\n", g_reason);
        return 0;
    }
    printf("hip\n");
    return 0;
}
