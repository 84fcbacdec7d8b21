/*
 * oracle/apus_oracle.h -- CPU restatement of the apus-qwen attention hot
 * path (Gated DeltaNet ops of c/gdn.h, gated-GQA ops of c/attn.h, the RNE
 * narrow of c/bf16.h, and the mixer wiring of c/layer.h), in plain C11.
 *
 * THIS IS TEST INFRASTRUCTURE. It is the parity checker for the HIP
 * library and the timed CPU baseline of bench.py. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (libapus_hip.so) never links or calls it.
 *
 * Numerics: built with -O2 -ffp-contract=off, so every fp32 mul and add is
 * one IEEE rounding in the written order, exactly as the reference anchors
 * (reference Makefile:24-26). libm (expf, log1pf, sqrtf, cosf, sinf, pow)
 * is the platform glibc, like the reference on Linux.
 *
 * Pinning (how each function is checked; the tests under tests/ do it):
 *   - bitwise against the reference's own scalar anchors compiled from
 *     /root/reference/c into oracle/_ref (every op below, every mixer);
 *   - against float64 truths written in the tests, with the reference's
 *     esc-normalised tolerance (tests/m4a/test_gdn.c:84-95 design);
 *   - against exact corners (beta(0)=0x3F00, decay a+dt=0 -> -e^A ln2,
 *     rope pos 0 == identity, g=0/beta=0 leaves S unchanged, ...).
 *
 * Layouts follow the reference exactly: bf16 travels as uint16_t codes,
 * fp32 as float, dims as size_t, row-major everywhere.
 */
#ifndef APUS_ORACLE_H
#define APUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 storage helpers (c/bf16.h:261-278) -------------------------- */
float    orc_bf16_f32(uint16_t b);
uint16_t orc_bf16_bits(float x);
float    orc_bf16_round(float x);
/* array form of orc_bf16_bits (for exhaustive tests of the rule) */
void     orc_bf16_narrow(const float *x, uint16_t *y, size_t n);

/* ---- Gated DeltaNet ops (c/gdn.h contract (a)-(e), lines 17-75) ------- */
/* (a) causal depthwise conv1d k=4 + SiLU, two rounding points
 *     (c/gdn.h:220-245 step, 314-318 prefill). state [C*3], j=0 oldest. */
void orc_gdn_conv1d_step(const uint16_t *x, const uint16_t *w,
                         uint16_t *out, size_t C, uint16_t *state);
void orc_gdn_conv1d(const uint16_t *x, const uint16_t *w, uint16_t *out,
                    size_t C, size_t T, uint16_t *state);
/* (b) decay g = -expf(A_log)*softplus(a+dt_bias)   (c/gdn.h:322-328) */
void orc_gdn_decay(const uint16_t *a, const float *A_log,
                   const float *dt_bias, float *g, size_t H);
/* (b2) beta = rnd(sigmoid(b))                       (c/gdn.h:366-370) */
void orc_gdn_beta(const uint16_t *b, uint16_t *beta, size_t H);
/* (c) per-head L2 norm, fp32 out, (x*rs)*scale      (c/gdn.h:402-416) */
void orc_gdn_l2norm(const uint16_t *x, float *y, size_t H, size_t D,
                    float scale);
/* (d) delta-rule step for one head                  (c/gdn.h:471-504) */
void orc_gdn_step_head(float *Sh, const float *qh, const float *kh,
                       const uint16_t *vh, float g, float beta, float *oh,
                       size_t Dk, size_t Dv);
/* (d) all heads, one token                           (c/gdn.h:587-595) */
void orc_gdn_step(float *S, const float *q, const float *k,
                  const uint16_t *v, const float *g, const uint16_t *beta,
                  float *o, size_t H, size_t Dk, size_t Dv);
/* (d) threaded over heads (c/gdn.h:619-625); nthreads <= 0 means all. */
void orc_gdn_step_mt(float *S, const float *q, const float *k,
                     const uint16_t *v, const float *g,
                     const uint16_t *beta, float *o, size_t H, size_t Dk,
                     size_t Dv, int nthreads);
/* (d) strict loop of step over T tokens              (c/gdn.h:627-635) */
void orc_gdn_recurrent(float *S, const float *q, const float *k,
                       const uint16_t *v, const float *g,
                       const uint16_t *beta, float *o, size_t T, size_t H,
                       size_t Dk, size_t Dv);
/* (e) RMSNormGated, direct weight, three roundings   (c/gdn.h:639-661) */
void orc_gdn_onorm(const uint16_t *o, const uint16_t *z, const uint16_t *w,
                   uint16_t *y, size_t H, size_t D);

/* ---- gated-GQA ops (c/attn.h contract (a)-(d), lines 16-58) ----------- */
/* (a) (1+w) RMSNorm, single rounding                  (c/attn.h:175-186) */
void orc_attn_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *y,
                      size_t N);
/* (b) partial NeoX RoPE                               (c/attn.h:244-266) */
void orc_attn_rope(const uint16_t *x, uint16_t *y, size_t D, size_t rot,
                   float pos, double theta);
/* (c) one attention row, keys 0..p of one kv head     (c/attn.h:337-368) */
void orc_attn_gqa_row(const uint16_t *qh, const uint16_t *kc,
                      const uint16_t *vc, uint16_t *oh, size_t Hkv,
                      size_t D, float scale, uint16_t *abuf, float *ebuf,
                      size_t p);
/* (c) causal eager GQA                                (c/attn.h:450-471) */
void orc_attn_gqa(const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                  uint16_t *o, size_t Tq, size_t Tk, size_t H, size_t Hkv,
                  size_t D, float scale, uint16_t *abuf, float *ebuf);
void orc_attn_gqa_decode(const uint16_t *q, const uint16_t *kc,
                         const uint16_t *vc, uint16_t *o, size_t Tk,
                         size_t H, size_t Hkv, size_t D, float scale,
                         uint16_t *abuf, float *ebuf);
/* (c) threaded over (row, head) units                 (c/attn.h:507-520) */
void orc_attn_gqa_mt(const uint16_t *q, const uint16_t *kc,
                     const uint16_t *vc, uint16_t *o, size_t Tq, size_t Tk,
                     size_t H, size_t Hkv, size_t D, float scale,
                     int nthreads);
/* (d) sigmoid output gate                             (c/attn.h:524-531) */
/* y [M][O] = rnd(w [O][K] . x [M][K]) in the reference's order
 * (c/bf16.h:285-300) */
void orc_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                   size_t M, size_t O, size_t K);
void orc_attn_outgate(const uint16_t *o, const uint16_t *gate, uint16_t *y,
                      size_t N);

/* ---- mixer wiring (c/layer.h:236-331 decode, 427-564 prefill) --------
 * The hot path between the input projections and the output projection:
 * GDN takes the in_proj_{qkv,z,a,b} outputs and produces the onorm output
 * that feeds w_out; full attention takes the q_proj ([q|gate] per head),
 * k_proj, v_proj outputs and produces the gated output that feeds wo.
 * Batched over B independent sequences: sequence s owns tokens
 * cu[s] .. cu[s+1]-1 of the packed token arrays and its own state. */
typedef struct {
    size_t hk, hv, dk, dv;          /* 16, 32, 128, 128 */
} OrcGdnDims;

typedef struct {
    size_t nh, nkv, d, rot;         /* 16, 2, 256, 64 */
    double theta;                   /* 1e7 */
} OrcAttnDims;

/* Optional named-intermediate capture (c/layer.h:172-189 names); any
 * member may be NULL. Rows are packed tokens. */
typedef struct {
    uint16_t *qkv_conv;             /* [Ttot, conv_dim] */
    uint16_t *beta;                 /* [Ttot, hv] */
    float    *gdecay;               /* [Ttot, hv] */
    uint16_t *rec_o;                /* [Ttot, hv*dv] (post-rnd) */
} OrcGdnTrace;

/* GDN mixer for B sequences. qkv [Ttot, conv_dim], z [Ttot, hv*dv],
 * a,b [Ttot, hv]; conv_state [B, conv_dim*3]; S [B, hv*dk*dv];
 * y [Ttot, hv*dv]. Per sequence the tokens run in ascending order exactly
 * as c/layer.h:452-489 (conv over the span, then per token beta, decay,
 * l2norm q/k, repeat-interleave, step, rnd, onorm). Threads split the
 * (sequence, v-head) step units; results are thread-count independent. */
void orc_gdn_mixer(const OrcGdnDims *dm, const uint16_t *conv_w,
                   const float *A_log, const float *dt_bias,
                   const uint16_t *onorm_w, size_t B, const int32_t *cu,
                   const uint16_t *qkv, const uint16_t *z,
                   const uint16_t *a, const uint16_t *b,
                   uint16_t *conv_state, float *S, uint16_t *y,
                   OrcGdnTrace *tr, int nthreads);

/* Full-attention mixer for B sequences. qg [Ttot, nh, 2d] ([q|gate] per
 * head), k,v [Ttot, nkv, d]; kcache/vcache: sequence s at
 * kcache + s*cache_stride with layout [max_seq, nkv, d]; pos0[s] = tokens
 * already in sequence s's cache. The new tokens are normed, roped at
 * pos0+t, appended, then attended causally (c/layer.h:520-561).
 * y [Ttot, nh*d] = outgate(attention, gate). qf/kf (optional, NULL ok)
 * capture the post-norm post-rope q [Ttot,nh*d] and k [Ttot,nkv*d]. */
void orc_attn_mixer(const OrcAttnDims *dm, const uint16_t *qn_w,
                    const uint16_t *kn_w, size_t B, const int32_t *cu,
                    const int32_t *pos0, const uint16_t *qg,
                    const uint16_t *k, const uint16_t *v, uint16_t *kcache,
                    uint16_t *vcache, size_t cache_stride, uint16_t *y,
                    uint16_t *qf, uint16_t *kf, int nthreads);

/* As orc_attn_mixer with sequence s's caches at kcache/vcache +
 * cache_off[s] (element offsets; each [>= pos0+new, nkv, d]); attno
 * (optional) captures the attention output before the gate [Ttot,nh*d]. */
void orc_attn_mixer_off(const OrcAttnDims *dm, const uint16_t *qn_w,
                        const uint16_t *kn_w, size_t B, const int32_t *cu,
                        const int32_t *pos0, const uint16_t *qg,
                        const uint16_t *k, const uint16_t *v,
                        uint16_t *kcache, uint16_t *vcache,
                        const size_t *cache_off, uint16_t *y, uint16_t *qf,
                        uint16_t *kf, uint16_t *attno, int nthreads);

/* The mixer's first phase only (c/layer.h:300-316): per token q/k norm,
 * rope and the cache append; qn [Ttot, nh*d] receives the roped q. */
void orc_attn_prep_off(const OrcAttnDims *dm, const uint16_t *qn_w,
                       const uint16_t *kn_w, size_t B, const int32_t *cu,
                       const int32_t *pos0, const uint16_t *qg,
                       const uint16_t *k, const uint16_t *v,
                       uint16_t *kcache, uint16_t *vcache,
                       const size_t *cache_off, uint16_t *qn, uint16_t *kf,
                       int nthreads);

/* Host-side RoPE table (c/attn.h:251-255 per pair): cs[2*R] bf16 codes,
 * cos then sin, for one position. */
void orc_attn_rope_table(float pos, size_t rot, double theta, uint16_t *cs);

/* Number of threads OpenMP would use for nthreads <= 0. */
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif /* APUS_ORACLE_H */
