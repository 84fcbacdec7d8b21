/*
 * oracle/ref_shim.c -- builds the REFERENCE's own scalar anchors
 * (c/gdn.h, c/attn.h, c/bf16.h, c/pool.h, compiled from their sources
 * under /root/reference/c, never copied) into oracle/_ref/libapus_ref.so.
 * TEST INFRASTRUCTURE: used only to pin the oracle restatement bitwise
 * and, optionally, as bench.py's "reference" CPU baseline.
 *
 * Besides the reference's exported op symbols (apus_gdn_*, apus_attn_*,
 * apus_bf16_gemv_scalar / _gemm_scalar), the projection hot paths
 * (ref_bf16_gemv_hot / _gemm_hot) and two drivers that sequence those ops exactly as the
 * reference's layer does between its projections, for B sequences run
 * one after another (the reference engine is single-sequence):
 *   ref_gdn_mixer  -- c/layer.h:445-489 (conv over the span, then per
 *                     token beta, decay, l2norm, repeat, step_mt, rnd,
 *                     onorm);
 *   ref_attn_mixer -- c/layer.h:520-561 (per token norms, rope, append;
 *                     one gqa_mt over the span; per token outgate).
 * Signatures match orc_gdn_mixer / orc_attn_mixer (oracle/apus_oracle.h)
 * minus the thread argument (the reference pool reads APUS_THREADS).
 */
#define APUS_BF16_IMPLEMENTATION
#define APUS_GDN_IMPLEMENTATION
#define APUS_ATTN_IMPLEMENTATION
#include "bf16.h"
#include "gdn.h"
#include "attn.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int ref_pool_threads(void) { return apus_pool_threads(); }

/* The projection hot paths without a backend hook installed: the x86
 * threaded gemv / gemm of the reference's CPU build (c/bf16.h:178-222). */
void ref_bf16_gemv_hot(const uint16_t *w, const uint16_t *x, uint16_t *y,
                       size_t O, size_t K) {
    apus_bf16_gemv_hot_cpu(w, x, y, O, K);
}
void ref_bf16_gemm_hot(const uint16_t *w, const uint16_t *x, uint16_t *y,
                       size_t M, size_t O, size_t K) {
    apus_bf16_gemm_hot_cpu(w, x, y, M, O, K);
}

void ref_gdn_mixer(size_t hk, size_t hv, size_t dk, size_t dv,
                   const uint16_t *conv_w, const float *A_log,
                   const float *dt_bias, const uint16_t *onorm_w, size_t B,
                   const int32_t *cu, const uint16_t *qkv, const uint16_t *z,
                   const uint16_t *a, const uint16_t *b,
                   uint16_t *conv_state, float *S, uint16_t *y) {
    size_t kd = hk * dk, vd = hv * dv, cd = 2 * kd + vd, rep = hv / hk;
    float qscale = (float)pow((double)dk, -0.5);
    uint16_t *qc = malloc((size_t)cu[B] * cd * 2);
    uint16_t *beta = malloc(hv * 2), *ob = malloc(vd * 2);
    float *g = malloc(hv * 4), *o = malloc(vd * 4);
    float *qn = malloc(kd * 4), *kn = malloc(kd * 4);
    float *qr = malloc(hv * dk * 4), *kr = malloc(hv * dk * 4);
    for (size_t s = 0; s < B; s++) {
        size_t t0 = (size_t)cu[s], t1 = (size_t)cu[s + 1];
        uint16_t *cst = conv_state + s * cd * 3;
        float *Ss = S + s * hv * dk * dv;
        apus_gdn_conv1d(qkv + t0 * cd, conv_w, qc + t0 * cd, cd, t1 - t0,
                        cst);
        for (size_t t = t0; t < t1; t++) {
            apus_gdn_beta(b + t * hv, beta, hv);
            apus_gdn_decay(a + t * hv, A_log, dt_bias, g, hv);
            apus_gdn_l2norm(qc + t * cd, qn, hk, dk, qscale);
            apus_gdn_l2norm(qc + t * cd + kd, kn, hk, dk, 1.0f);
            for (size_t h = 0; h < hk; h++)
                for (size_t r = 0; r < rep; r++) {
                    memcpy(qr + (h * rep + r) * dk, qn + h * dk, dk * 4);
                    memcpy(kr + (h * rep + r) * dk, kn + h * dk, dk * 4);
                }
            apus_gdn_step_mt(Ss, qr, kr, qc + t * cd + 2 * kd, g, beta, o,
                             hv, dk, dv);
            for (size_t i = 0; i < vd; i++) ob[i] = apus_bf16_bits(o[i]);
            apus_gdn_onorm(ob, z + t * vd, onorm_w, y + t * vd, hv, dv);
        }
    }
    free(qc); free(beta); free(ob); free(g); free(o);
    free(qn); free(kn); free(qr); free(kr);
}

void ref_attn_mixer(size_t nh, size_t nkv, size_t d, size_t rot,
                    double theta, const uint16_t *qn_w, const uint16_t *kn_w,
                    size_t B, const int32_t *cu, const int32_t *pos0,
                    const uint16_t *qg, const uint16_t *k, const uint16_t *v,
                    uint16_t *kcache, uint16_t *vcache, size_t cache_stride,
                    uint16_t *y) {
    float scale = (float)(1.0 / sqrt((double)d));
    size_t Tmax = 0;
    for (size_t s = 0; s < B; s++)
        if ((size_t)(cu[s + 1] - cu[s]) > Tmax)
            Tmax = (size_t)(cu[s + 1] - cu[s]);
    uint16_t *qn = malloc(Tmax * nh * d * 2), *ao = malloc(Tmax * nh * d * 2);
    uint16_t *gate = malloc(nh * d * 2), *kn = malloc(nkv * d * 2);
    for (size_t s = 0; s < B; s++) {
        size_t t0 = (size_t)cu[s], tc = (size_t)cu[s + 1] - t0;
        uint16_t *kc = kcache + s * cache_stride;
        uint16_t *vc = vcache + s * cache_stride;
        for (size_t t = 0; t < tc; t++) {
            size_t pos = (size_t)pos0[s] + t, tt = t0 + t;
            for (size_t h = 0; h < nh; h++)
                apus_attn_rmsnorm(qg + (tt * nh + h) * 2 * d, qn_w,
                                  qn + (t * nh + h) * d, d);
            for (size_t h = 0; h < nkv; h++)
                apus_attn_rmsnorm(k + (tt * nkv + h) * d, kn_w, kn + h * d,
                                  d);
            for (size_t h = 0; h < nh; h++)
                apus_attn_rope(qn + (t * nh + h) * d, qn + (t * nh + h) * d,
                               d, rot, (float)pos, theta);
            for (size_t h = 0; h < nkv; h++)
                apus_attn_rope(kn + h * d, kn + h * d, d, rot, (float)pos,
                               theta);
            memcpy(kc + pos * nkv * d, kn, nkv * d * 2);
            memcpy(vc + pos * nkv * d, v + tt * nkv * d, nkv * d * 2);
        }
        apus_attn_gqa_mt(qn, kc, vc, ao, tc, (size_t)pos0[s] + tc, nh, nkv,
                         d, scale);
        for (size_t t = 0; t < tc; t++) {
            size_t tt = t0 + t;
            for (size_t h = 0; h < nh; h++)
                memcpy(gate + h * d, qg + (tt * nh + h) * 2 * d + d, d * 2);
            apus_attn_outgate(ao + t * nh * d, gate, y + tt * nh * d,
                              nh * d);
        }
    }
    free(qn); free(ao); free(gate); free(kn);
}
