/*
 * oracle/apus_oracle.c -- CPU restatement of the apus-qwen attention hot
 * path. TEST INFRASTRUCTURE ONLY (see apus_oracle.h): the parity checker
 * and the timed CPU baseline; the product library never links it.
 *
 * Each function cites the reference lines whose arithmetic it restates.
 * Build: -std=c11 -O2 -ffp-contract=off -fno-tree-vectorize -fopenmp
 * (oracle/Makefile), matching the reference's pinned FP flags.
 */
#include "apus_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define ORC_CONV_K 4u
#define ORC_EPS 1e-6f

/* ---- bf16 (c/bf16.h:261-278: exact widen; RNE narrow, NaN kept) ------- */
float orc_bf16_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

uint16_t orc_bf16_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u)        /* NaN: keep sign+payload */
        return (uint16_t)(u >> 16);
    uint32_t lsb = (u >> 16) & 1u;              /* ties to even */
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

float orc_bf16_round(float x) { return orc_bf16_f32(orc_bf16_bits(x)); }

void orc_bf16_narrow(const float *x, uint16_t *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = orc_bf16_bits(x[i]);
}

static inline float f32(uint16_t b) { return orc_bf16_f32(b); }
static inline uint16_t rnd(float x) { return orc_bf16_bits(x); }

static inline float sigm(float z) { return 1.0f / (1.0f + expf(-z)); }

int orc_max_threads(void) { return omp_get_max_threads(); }

static int nthr(int n) { return n > 0 ? n : omp_get_max_threads(); }

/* ---- (a) conv1d k=4 + SiLU (c/gdn.h:19-33 contract, 220-245) --------- */
static inline uint16_t conv_channel(const uint16_t *wc, uint16_t s0,
                                    uint16_t s1, uint16_t s2, uint16_t x) {
    /* taps in ascending window order: oldest state first, input last */
    float acc = 0.0f;
    acc += f32(wc[0]) * f32(s0);
    acc += f32(wc[1]) * f32(s1);
    acc += f32(wc[2]) * f32(s2);
    acc += f32(wc[3]) * f32(x);
    float co = f32(rnd(acc));                      /* rounding point 1 */
    return rnd(co * sigm(co));                     /* rounding point 2 */
}

void orc_gdn_conv1d_step(const uint16_t *x, const uint16_t *w,
                         uint16_t *out, size_t C, uint16_t *state) {
    for (size_t c = 0; c < C; c++) {
        uint16_t *st = state + c * (ORC_CONV_K - 1);
        out[c] = conv_channel(w + c * ORC_CONV_K, st[0], st[1], st[2], x[c]);
        st[0] = st[1];
        st[1] = st[2];
        st[2] = x[c];
    }
}

void orc_gdn_conv1d(const uint16_t *x, const uint16_t *w, uint16_t *out,
                    size_t C, size_t T, uint16_t *state) {
    for (size_t t = 0; t < T; t++)
        orc_gdn_conv1d_step(x + t * C, w, out + t * C, C, state);
}

/* ---- (b) decay (c/gdn.h:34-40, 212-214, 322-328) --------------------- */
static inline float softplus(float x) {
    return x > 20.0f ? x : log1pf(expf(x));
}

void orc_gdn_decay(const uint16_t *a, const float *A_log,
                   const float *dt_bias, float *g, size_t H) {
    for (size_t h = 0; h < H; h++) {
        float t = f32(a[h]) + dt_bias[h];
        g[h] = -expf(A_log[h]) * softplus(t);
    }
}

/* ---- (b2) beta (c/gdn.h:41-42, 366-370) ------------------------------- */
void orc_gdn_beta(const uint16_t *b, uint16_t *beta, size_t H) {
    for (size_t h = 0; h < H; h++)
        beta[h] = rnd(sigm(f32(b[h])));
}

/* ---- (c) l2norm (c/gdn.h:43-49, 402-416) ------------------------------ */
void orc_gdn_l2norm(const uint16_t *x, float *y, size_t H, size_t D,
                    float scale) {
    for (size_t h = 0; h < H; h++) {
        const uint16_t *xh = x + h * D;
        float *yh = y + h * D;
        float ss = 0.0f;
        for (size_t i = 0; i < D; i++) {
            float v = f32(xh[i]);
            ss += v * v;
        }
        float rs = 1.0f / sqrtf(ss + ORC_EPS);
        for (size_t i = 0; i < D; i++) {
            float t = f32(xh[i]) * rs;             /* (x*rs) then *scale */
            yh[i] = t * scale;
        }
    }
}

/* ---- (d) delta-rule step (c/gdn.h:50-67, 471-504) ---------------------
 * Column-separable restatement: column j of S needs only k, q, beta, dec,
 * v[j] and S[:,j]. Each pass keeps the reference's ascending-i order per
 * column and its one-rounding-per-op flow, so the values are identical to
 * running the four full passes of the anchor. */
void orc_gdn_step_head(float *Sh, const float *qh, const float *kh,
                       const uint16_t *vh, float g, float beta, float *oh,
                       size_t Dk, size_t Dv) {
    float dec = expf(g);
    for (size_t i = 0; i < Dk * Dv; i++)
        Sh[i] = Sh[i] * dec;
    for (size_t j = 0; j < Dv; j++) {
        float kv = 0.0f;
        for (size_t i = 0; i < Dk; i++)
            kv += kh[i] * Sh[i * Dv + j];
        float delta = (f32(vh[j]) - kv) * beta;
        float acc = 0.0f;
        for (size_t i = 0; i < Dk; i++) {
            float s = Sh[i * Dv + j] + kh[i] * delta;
            Sh[i * Dv + j] = s;
            acc += qh[i] * s;
        }
        oh[j] = acc;
    }
}

void orc_gdn_step(float *S, const float *q, const float *k,
                  const uint16_t *v, const float *g, const uint16_t *beta,
                  float *o, size_t H, size_t Dk, size_t Dv) {
    for (size_t h = 0; h < H; h++)
        orc_gdn_step_head(S + h * Dk * Dv, q + h * Dk, k + h * Dk,
                          v + h * Dv, g[h], f32(beta[h]), o + h * Dv, Dk,
                          Dv);
}

void orc_gdn_step_mt(float *S, const float *q, const float *k,
                     const uint16_t *v, const float *g,
                     const uint16_t *beta, float *o, size_t H, size_t Dk,
                     size_t Dv, int nthreads) {
    long HH = (long)H;
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
    for (long h = 0; h < HH; h++)
        orc_gdn_step_head(S + (size_t)h * Dk * Dv, q + (size_t)h * Dk,
                          k + (size_t)h * Dk, v + (size_t)h * Dv, g[h],
                          f32(beta[h]), o + (size_t)h * Dv, Dk, Dv);
}

void orc_gdn_recurrent(float *S, const float *q, const float *k,
                       const uint16_t *v, const float *g,
                       const uint16_t *beta, float *o, size_t T, size_t H,
                       size_t Dk, size_t Dv) {
    for (size_t t = 0; t < T; t++)
        orc_gdn_step(S, q + t * H * Dk, k + t * H * Dk, v + t * H * Dv,
                     g + t * H, beta + t * H, o + t * H * Dv, H, Dk, Dv);
}

/* ---- (e) RMSNormGated (c/gdn.h:68-75, 639-661) ------------------------ */
void orc_gdn_onorm(const uint16_t *o, const uint16_t *z, const uint16_t *w,
                   uint16_t *y, size_t H, size_t D) {
    for (size_t h = 0; h < H; h++) {
        const uint16_t *oh = o + h * D, *zh = z + h * D;
        uint16_t *yh = y + h * D;
        float ss = 0.0f;
        for (size_t d = 0; d < D; d++) {
            float v = f32(oh[d]);
            ss += v * v;
        }
        float rs = 1.0f / sqrtf(ss / (float)D + ORC_EPS);
        for (size_t d = 0; d < D; d++) {
            float x1 = f32(rnd(f32(oh[d]) * rs));
            float x2 = f32(rnd(x1 * f32(w[d])));
            float zf = f32(zh[d]);
            float gate = zf * sigm(zf);
            yh[d] = rnd(x2 * gate);
        }
    }
}

/* ---- attn (a) (1+w) RMSNorm (c/attn.h:18-26, 175-186) ----------------- */
void orc_attn_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *y,
                      size_t N) {
    float ss = 0.0f;
    for (size_t i = 0; i < N; i++) {
        float v = f32(x[i]);
        ss += v * v;
    }
    float rs = 1.0f / sqrtf(ss / (float)N + ORC_EPS);
    for (size_t i = 0; i < N; i++) {
        float n = f32(x[i]) * rs;
        y[i] = rnd(n * (1.0f + f32(w[i])));
    }
}

/* ---- attn (b) partial NeoX RoPE (c/attn.h:27-38, 244-266) ------------- */
void orc_attn_rope_table(float pos, size_t rot, double theta, uint16_t *cs) {
    size_t R = rot / 2;
    for (size_t i = 0; i < R; i++) {
        double e = 2.0 * (double)i / (double)rot;
        float invf = (float)(1.0 / pow(theta, e));
        float ang = pos * invf;
        cs[i] = rnd(cosf(ang));
        cs[R + i] = rnd(sinf(ang));
    }
}

void orc_attn_rope(const uint16_t *x, uint16_t *y, size_t D, size_t rot,
                   float pos, double theta) {
    size_t R = rot / 2;
    for (size_t i = 0; i < R; i++) {
        double e = 2.0 * (double)i / (double)rot;
        float invf = (float)(1.0 / pow(theta, e));
        float ang = pos * invf;
        float c = f32(rnd(cosf(ang))), s = f32(rnd(sinf(ang)));
        float lo = f32(x[i]), hi = f32(x[i + R]);
        float a0 = orc_bf16_round(lo * c), a1 = orc_bf16_round(-hi * s);
        float b0 = orc_bf16_round(hi * c), b1 = orc_bf16_round(lo * s);
        y[i] = rnd(a0 + a1);
        y[i + R] = rnd(b0 + b1);
    }
    if (x != y)
        for (size_t i = rot; i < D; i++) y[i] = x[i];
}

/* ---- attn (c) eager GQA (c/attn.h:39-52, 337-368, 450-471) ------------ */
void orc_attn_gqa_row(const uint16_t *qh, const uint16_t *kc,
                      const uint16_t *vc, uint16_t *oh, size_t Hkv,
                      size_t D, float scale, uint16_t *abuf, float *ebuf,
                      size_t p) {
    size_t rs = Hkv * D;                           /* cache row stride */
    for (size_t j = 0; j <= p; j++) {
        const uint16_t *kr = kc + j * rs;
        float dot = 0.0f;
        for (size_t d = 0; d < D; d++) dot += f32(qh[d]) * f32(kr[d]);
        abuf[j] = rnd(f32(rnd(dot)) * scale);
    }
    float m = f32(abuf[0]);
    for (size_t j = 1; j <= p; j++)
        if (f32(abuf[j]) > m) m = f32(abuf[j]);
    float s = 0.0f;
    for (size_t j = 0; j <= p; j++) {
        ebuf[j] = expf(f32(abuf[j]) - m);
        s += ebuf[j];
    }
    for (size_t j = 0; j <= p; j++) abuf[j] = rnd(ebuf[j] / s);
    for (size_t d = 0; d < D; d++) {
        float acc = 0.0f;
        for (size_t j = 0; j <= p; j++)
            acc += f32(abuf[j]) * f32(vc[j * rs + d]);
        oh[d] = rnd(acc);
    }
}

void orc_attn_gqa(const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                  uint16_t *o, size_t Tq, size_t Tk, size_t H, size_t Hkv,
                  size_t D, float scale, uint16_t *abuf, float *ebuf) {
    size_t grp = H / Hkv;
    for (size_t t = 0; t < Tq; t++)
        for (size_t h = 0; h < H; h++) {
            size_t hk = h / grp;
            orc_attn_gqa_row(q + (t * H + h) * D, kc + hk * D, vc + hk * D,
                             o + (t * H + h) * D, Hkv, D, scale, abuf, ebuf,
                             Tk - Tq + t);
        }
}

void orc_attn_gqa_decode(const uint16_t *q, const uint16_t *kc,
                         const uint16_t *vc, uint16_t *o, size_t Tk,
                         size_t H, size_t Hkv, size_t D, float scale,
                         uint16_t *abuf, float *ebuf) {
    orc_attn_gqa(q, kc, vc, o, 1, Tk, H, Hkv, D, scale, abuf, ebuf);
}

void orc_attn_gqa_mt(const uint16_t *q, const uint16_t *kc,
                     const uint16_t *vc, uint16_t *o, size_t Tq, size_t Tk,
                     size_t H, size_t Hkv, size_t D, float scale,
                     int nthreads) {
    size_t grp = H / Hkv;
    long units = (long)(Tq * H);
#pragma omp parallel num_threads(nthr(nthreads))
    {
        uint16_t *ab = malloc(Tk * sizeof *ab);
        float *eb = malloc(Tk * sizeof *eb);
#pragma omp for schedule(static)
        for (long u = 0; u < units; u++) {
            size_t t = (size_t)u / H, h = (size_t)u % H, hk = h / grp;
            orc_attn_gqa_row(q + (t * H + h) * D, kc + hk * D, vc + hk * D,
                             o + (t * H + h) * D, Hkv, D, scale, ab, eb,
                             Tk - Tq + t);
        }
        free(ab);
        free(eb);
    }
}

/* ---- attn (d) output gate (c/attn.h:53-58, 524-531) ------------------- */
void orc_attn_outgate(const uint16_t *o, const uint16_t *gate, uint16_t *y,
                      size_t N) {
    for (size_t i = 0; i < N; i++) {
        float g = f32(rnd(sigm(f32(gate[i]))));
        y[i] = rnd(f32(o[i]) * g);
    }
}

/* ---- projections (c/bf16.h:285-300: per output an ascending fp32 sum of
 * widened products, one rounding per multiply and per add, then RNE; the
 * gemm is the gemv per row). Outputs are independent, so the OpenMP split
 * over (m, o) leaves every sum's order unchanged. */
void orc_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                   size_t M, size_t O, size_t K) {
#pragma omp parallel for schedule(static)
    for (long u = 0; u < (long)(M * O); u++) {
        const size_t m = (size_t)u / O, o = (size_t)u % O;
        const uint16_t *wr = w + o * K, *xr = x + m * K;
        float acc = 0.0f;
        for (size_t k = 0; k < K; k++) acc += f32(wr[k]) * f32(xr[k]);
        y[m * O + o] = rnd(acc);
    }
}

/* ---- GDN mixer (c/layer.h:236-286 decode, 427-492 prefill) ------------
 * Phase 1 (per sequence): conv over the sequence's tokens, then per token
 * beta, decay, l2norm of the K heads. Phase 2 (per (sequence, v-head)):
 * the recurrence over the sequence's tokens in ascending order, reading
 * the K-head norms through the repeat-interleave map hv -> hv/(hv/hk),
 * which is the values of the reference's memcpy expansion
 * (c/layer.h:261-268). Phase 3 (per token): rnd then onorm. */
void orc_gdn_mixer(const OrcGdnDims *dm, const uint16_t *conv_w,
                   const float *A_log, const float *dt_bias,
                   const uint16_t *onorm_w, size_t B, const int32_t *cu,
                   const uint16_t *qkv, const uint16_t *z,
                   const uint16_t *a, const uint16_t *b,
                   uint16_t *conv_state, float *S, uint16_t *y,
                   OrcGdnTrace *tr, int nthreads) {
    size_t hk = dm->hk, hv = dm->hv, dk = dm->dk, dv = dm->dv;
    size_t kd = hk * dk, vd = hv * dv, cd = 2 * kd + vd;
    size_t rep = hv / hk;
    size_t Ttot = (size_t)cu[B];
    float qscale = (float)pow((double)dk, -0.5);
    int nt = nthr(nthreads);
    uint16_t *qc = malloc(Ttot * cd * sizeof *qc);
    float *qn = malloc(Ttot * kd * sizeof *qn);
    float *kn = malloc(Ttot * kd * sizeof *kn);
    float *g = malloc(Ttot * hv * sizeof *g);
    uint16_t *bt = malloc(Ttot * hv * sizeof *bt);
    float *o = malloc(Ttot * vd * sizeof *o);
    long BB = (long)B;

#pragma omp parallel for schedule(static) num_threads(nt)
    for (long s = 0; s < BB; s++) {
        size_t t0 = (size_t)cu[s], t1 = (size_t)cu[s + 1];
        orc_gdn_conv1d(qkv + t0 * cd, conv_w, qc + t0 * cd, cd, t1 - t0,
                       conv_state + (size_t)s * cd * 3);
        for (size_t t = t0; t < t1; t++) {
            orc_gdn_beta(b + t * hv, bt + t * hv, hv);
            orc_gdn_decay(a + t * hv, A_log, dt_bias, g + t * hv, hv);
            orc_gdn_l2norm(qc + t * cd, qn + t * kd, hk, dk, qscale);
            orc_gdn_l2norm(qc + t * cd + kd, kn + t * kd, hk, dk, 1.0f);
        }
    }

    long units = (long)(B * hv);
#pragma omp parallel for schedule(static) num_threads(nt)
    for (long u = 0; u < units; u++) {
        size_t s = (size_t)u / hv, h = (size_t)u % hv, kh = h / rep;
        float *Sh = S + (s * hv + h) * dk * dv;
        for (size_t t = (size_t)cu[s]; t < (size_t)cu[s + 1]; t++)
            orc_gdn_step_head(Sh, qn + t * kd + kh * dk,
                              kn + t * kd + kh * dk,
                              qc + t * cd + 2 * kd + h * dv, g[t * hv + h],
                              f32(bt[t * hv + h]), o + t * vd + h * dv, dk,
                              dv);
    }

    long TT = (long)Ttot;
#pragma omp parallel for schedule(static) num_threads(nt)
    for (long t = 0; t < TT; t++) {
        uint16_t *ob = malloc(vd * sizeof *ob);
        for (size_t i = 0; i < vd; i++) ob[i] = rnd(o[(size_t)t * vd + i]);
        orc_gdn_onorm(ob, z + (size_t)t * vd, onorm_w, y + (size_t)t * vd,
                      hv, dv);
        if (tr && tr->rec_o)
            memcpy(tr->rec_o + (size_t)t * vd, ob, vd * sizeof *ob);
        free(ob);
    }
    if (tr) {
        if (tr->qkv_conv) memcpy(tr->qkv_conv, qc, Ttot * cd * sizeof *qc);
        if (tr->beta) memcpy(tr->beta, bt, Ttot * hv * sizeof *bt);
        if (tr->gdecay) memcpy(tr->gdecay, g, Ttot * hv * sizeof *g);
    }
    free(qc); free(qn); free(kn); free(g); free(bt); free(o);
}

/* ---- attention mixer (c/layer.h:288-331 decode, 498-564 prefill) ------ */
/* per token: q/k (1+w) norm, rope at its own position, cache append
 * (c/layer.h:300-316) */
void orc_attn_prep_off(const OrcAttnDims *dm, const uint16_t *qn_w,
                       const uint16_t *kn_w, size_t B, const int32_t *cu,
                       const int32_t *pos0, const uint16_t *qg,
                       const uint16_t *k, const uint16_t *v,
                       uint16_t *kcache, uint16_t *vcache,
                       const size_t *cache_off, uint16_t *qn, uint16_t *kf,
                       int nthreads) {
    size_t nh = dm->nh, nkv = dm->nkv, d = dm->d, rot = dm->rot;
    int nt = nthr(nthreads);
    long BB = (long)B;
#pragma omp parallel for schedule(static) num_threads(nt)
    for (long s = 0; s < BB; s++) {
        uint16_t *kc = kcache + cache_off[s];
        uint16_t *vc = vcache + cache_off[s];
        for (size_t t = (size_t)cu[s]; t < (size_t)cu[s + 1]; t++) {
            size_t pos = (size_t)pos0[s] + (t - (size_t)cu[s]);
            for (size_t h = 0; h < nh; h++) {
                uint16_t *qh = qn + (t * nh + h) * d;
                orc_attn_rmsnorm(qg + (t * nh + h) * 2 * d, qn_w, qh, d);
                orc_attn_rope(qh, qh, d, rot, (float)pos, dm->theta);
            }
            uint16_t *krow = kc + pos * nkv * d;
            for (size_t h = 0; h < nkv; h++) {
                orc_attn_rmsnorm(k + (t * nkv + h) * d, kn_w, krow + h * d,
                                 d);
                orc_attn_rope(krow + h * d, krow + h * d, d, rot, (float)pos,
                              dm->theta);
            }
            memcpy(vc + pos * nkv * d, v + t * nkv * d,
                   nkv * d * sizeof *v);
            if (kf) memcpy(kf + t * nkv * d, krow, nkv * d * sizeof *krow);
        }
    }
}

void orc_attn_mixer_off(const OrcAttnDims *dm, const uint16_t *qn_w,
                        const uint16_t *kn_w, size_t B, const int32_t *cu,
                        const int32_t *pos0, const uint16_t *qg,
                        const uint16_t *k, const uint16_t *v,
                        uint16_t *kcache, uint16_t *vcache,
                        const size_t *cache_off, uint16_t *y, uint16_t *qf,
                        uint16_t *kf, uint16_t *attno, int nthreads) {
    size_t nh = dm->nh, nkv = dm->nkv, d = dm->d;
    size_t Ttot = (size_t)cu[B];
    float scale = (float)(1.0 / sqrt((double)d));
    int nt = nthr(nthreads);
    uint16_t *qn = malloc(Ttot * nh * d * sizeof *qn);
    uint16_t *ao = malloc(Ttot * nh * d * sizeof *ao);

    orc_attn_prep_off(dm, qn_w, kn_w, B, cu, pos0, qg, k, v, kcache, vcache,
                      cache_off, qn, kf, nthreads);

    /* (sequence, token, head) rows, each over its causal key range */
    size_t grp = nh / nkv;
    size_t maxk = 0;
    for (size_t s = 0; s < B; s++) {
        size_t tk = (size_t)pos0[s] + (size_t)(cu[s + 1] - cu[s]);
        if (tk > maxk) maxk = tk;
    }
    long units = (long)(Ttot * nh);
#pragma omp parallel num_threads(nt)
    {
        uint16_t *ab = malloc((maxk + 1) * sizeof *ab);
        float *eb = malloc((maxk + 1) * sizeof *eb);
#pragma omp for schedule(dynamic, 4)
        for (long u = 0; u < units; u++) {
            size_t t = (size_t)u / nh, h = (size_t)u % nh, hk = h / grp;
            size_t s = 0;
            while ((size_t)cu[s + 1] <= t) s++;
            size_t p = (size_t)pos0[s] + (t - (size_t)cu[s]);
            orc_attn_gqa_row(qn + (t * nh + h) * d,
                             kcache + cache_off[s] + hk * d,
                             vcache + cache_off[s] + hk * d,
                             ao + (t * nh + h) * d, nkv, d, scale, ab, eb, p);
        }
        free(ab);
        free(eb);
    }

#pragma omp parallel for schedule(static) num_threads(nt)
    for (long tt = 0; tt < (long)Ttot; tt++) {
        size_t t = (size_t)tt;
        uint16_t *gate = malloc(nh * d * sizeof *gate);
        for (size_t h = 0; h < nh; h++)
            memcpy(gate + h * d, qg + (t * nh + h) * 2 * d + d,
                   d * sizeof *gate);
        orc_attn_outgate(ao + t * nh * d, gate, y + t * nh * d, nh * d);
        free(gate);
    }
    if (qf) memcpy(qf, qn, Ttot * nh * d * sizeof *qn);
    if (attno) memcpy(attno, ao, Ttot * nh * d * sizeof *ao);
    free(qn);
    free(ao);
}

void orc_attn_mixer(const OrcAttnDims *dm, const uint16_t *qn_w,
                    const uint16_t *kn_w, size_t B, const int32_t *cu,
                    const int32_t *pos0, const uint16_t *qg,
                    const uint16_t *k, const uint16_t *v, uint16_t *kcache,
                    uint16_t *vcache, size_t cache_stride, uint16_t *y,
                    uint16_t *qf, uint16_t *kf, int nthreads) {
    size_t *off = malloc((B + 1) * sizeof *off);
    for (size_t s = 0; s < B; s++) off[s] = s * cache_stride;
    orc_attn_mixer_off(dm, qn_w, kn_w, B, cu, pos0, qg, k, v, kcache, vcache,
                       off, y, qf, kf, NULL, nthreads);
    free(off);
}
