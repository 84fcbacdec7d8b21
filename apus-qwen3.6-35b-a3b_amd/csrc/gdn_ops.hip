// gdn_ops.hip -- Gated DeltaNet ops for gfx950.
//
// Two tiers:
//  * drop-in ops (apus_hip_gdn_*): the argument lists of c/gdn.h:107-192,
//    host pointers, every sum in the reference's ascending order with one
//    IEEE rounding per mul/add (this file is compiled with FP contraction
//    off), so results equal the scalar anchors up to libm ulps;
//  * the fused batched decode (apus_hip_gdn_decode): conv1d+SiLU, beta,
//    decay, l2norm, the delta-rule step, rnd and the gated RMSNorm in one
//    kernel per (sequence, K head), state streamed once from HBM.
#include <stdint.h>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"

using namespace apus;

namespace {

constexpr float kEps = 1e-6f;

// ---- (a) conv1d k=4 + SiLU, one thread per channel -------------------
// c/gdn.h:19-33, 220-245: acc over the 4 taps oldest first, rnd, SiLU, rnd.
__device__ __forceinline__ uint16_t conv_tap4(const float w[4], float s0,
                                              float s1, float s2, float x) {
    float acc = 0.0f;
    acc = acc + w[0] * s0;
    acc = acc + w[1] * s1;
    acc = acc + w[2] * s2;
    acc = acc + w[3] * x;
    float co = rndf(acc);
    return f2bf(co * sigmoid_cr(co));
}

__global__ void k_conv1d(const uint16_t *__restrict__ x,
                         const uint16_t *__restrict__ w,
                         uint16_t *__restrict__ out, size_t C, size_t T,
                         uint16_t *__restrict__ state) {
    size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    float wf[4];
    for (int i = 0; i < 4; i++) wf[i] = bf2f(w[c * 4 + i]);
    uint16_t s0 = state[c * 3 + 0], s1 = state[c * 3 + 1],
             s2 = state[c * 3 + 2];
    for (size_t t = 0; t < T; t++) {
        uint16_t xv = x[t * C + c];
        out[t * C + c] = conv_tap4(wf, bf2f(s0), bf2f(s1), bf2f(s2), bf2f(xv));
        s0 = s1;
        s1 = s2;
        s2 = xv;
    }
    state[c * 3 + 0] = s0;
    state[c * 3 + 1] = s1;
    state[c * 3 + 2] = s2;
}

// ---- (b) decay, (b2) beta --------------------------------------------
__device__ __forceinline__ float decay_of(uint16_t a, float A_log,
                                         float dt_bias) {
    float t = bf2f(a) + dt_bias;
    return -exp_cr(A_log) * softplus_cr(t);
}

__global__ void k_decay(const uint16_t *a, const float *A_log,
                        const float *dt_bias, float *g, size_t H) {
    size_t h = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (h < H) g[h] = decay_of(a[h], A_log[h], dt_bias[h]);
}

__global__ void k_beta(const uint16_t *b, uint16_t *beta, size_t H) {
    size_t h = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (h < H) beta[h] = f2bf(sigmoid_cr(bf2f(b[h])));
}

// ---- (c) l2norm: one thread per head, ascending sum ------------------
__global__ void k_l2norm(const uint16_t *x, float *y, size_t H, size_t D,
                         float scale) {
    size_t h = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= H) return;
    const uint16_t *xh = x + h * D;
    float ss = 0.0f;
    for (size_t i = 0; i < D; i++) {
        float v = bf2f(xh[i]);
        ss = ss + v * v;
    }
    float rs = 1.0f / sqrtf(ss + kEps);
    for (size_t i = 0; i < D; i++) y[h * D + i] = (bf2f(xh[i]) * rs) * scale;
}

// ---- (d) delta-rule recurrence, generic dims --------------------------
// One block per head, one thread per value column j (strided when Dv >
// blockDim). Column j of S needs only k, q, beta, exp(g), v[j] and S[:,j]
// (c/gdn.h:482-503), and each column keeps the ascending-i sums.
__global__ void k_recurrent(float *__restrict__ S, const float *q,
                            const float *k, const uint16_t *v,
                            const float *g, const uint16_t *beta, float *o,
                            size_t T, size_t H, size_t Dk, size_t Dv) {
    size_t h = blockIdx.x;
    float *Sh = S + h * Dk * Dv;
    for (size_t t = 0; t < T; t++) {
        const float *qh = q + (t * H + h) * Dk;
        const float *kh = k + (t * H + h) * Dk;
        float dec = exp_cr(g[t * H + h]);
        float bt = bf2f(beta[t * H + h]);
        for (size_t j = threadIdx.x; j < Dv; j += blockDim.x) {
            float kv = 0.0f;
            for (size_t i = 0; i < Dk; i++) {
                float s = Sh[i * Dv + j] * dec;
                Sh[i * Dv + j] = s;
                kv = kv + kh[i] * s;
            }
            float delta = (bf2f(v[(t * H + h) * Dv + j]) - kv) * bt;
            float acc = 0.0f;
            for (size_t i = 0; i < Dk; i++) {
                float s = Sh[i * Dv + j] + kh[i] * delta;
                Sh[i * Dv + j] = s;
                acc = acc + qh[i] * s;
            }
            o[(t * H + h) * Dv + j] = acc;
        }
    }
}

// ---- (e) onorm: one block per head -----------------------------------
__global__ void k_onorm(const uint16_t *o, const uint16_t *z,
                        const uint16_t *w, uint16_t *y, size_t D) {
    size_t h = blockIdx.x;
    const uint16_t *oh = o + h * D, *zh = z + h * D;
    __shared__ float rs_s;
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (size_t d = 0; d < D; d++) {
            float v = bf2f(oh[d]);
            ss = ss + v * v;
        }
        rs_s = 1.0f / sqrtf(ss / (float)D + kEps);
    }
    __syncthreads();
    float rs = rs_s;
    for (size_t d = threadIdx.x; d < D; d += blockDim.x) {
        float x1 = rndf(bf2f(oh[d]) * rs);
        float x2 = rndf(x1 * bf2f(w[d]));
        float zf = bf2f(zh[d]);
        y[h * D + d] = f2bf(x2 * (zf * sigmoid_cr(zf)));
    }
}

// ---- fused batched decode ---------------------------------------------
// One workgroup per (sequence, K head), 2*128 threads. Thread t < 128
// owns q channel t of the K head, t >= 128 its k channel t-128 (conv +
// l2norm); thread t also owns value column j = t % 128 of v-head
// 2*kh + t/128 (conv of that v channel, the delta step on that S column,
// the gated norm of that output). The S column lives in 128 VGPRs across
// all of the sequence's tokens: one read and one write of the state.
constexpr int DK = 128, DV = 128, REP = 2, NT = REP * DV;

__global__ __launch_bounds__(NT) void k_gdn_decode(
    const int32_t *__restrict__ cu, const uint16_t *__restrict__ qkv,
    const uint16_t *__restrict__ z, const uint16_t *__restrict__ a,
    const uint16_t *__restrict__ b, const uint16_t *__restrict__ conv_w,
    const float *__restrict__ A_log, const float *__restrict__ dt_bias,
    const uint16_t *__restrict__ onorm_w, uint16_t *__restrict__ conv_state,
    float *__restrict__ S, uint16_t *__restrict__ y, int hk, float qscale) {
    const int s = blockIdx.x / hk, kh = blockIdx.x % hk;
    const int tid = threadIdx.x, r = tid / DV, j = tid % DV;
    const int hv = hk * REP, h = kh * REP + r;
    const size_t kd = (size_t)hk * DK, vd = (size_t)hv * DV;
    const size_t cd = 2 * kd + vd;

    __shared__ float raw[NT];          // conv outputs of q (0..127), k
    __shared__ float qn[DK], kn[DK];   // normalised q (scaled), k
    __shared__ float ob[REP][DV];      // rnd(o) per v-head
    __shared__ float rsq[2], rso[REP], gd[REP], bt[REP];

    // channel ownership
    const size_t cqk = tid < DK ? (size_t)kh * DK + tid
                                : kd + (size_t)kh * DK + (tid - DK);
    const size_t cv = 2 * kd + (size_t)h * DV + j;
    float wq[4], wv[4];
    for (int i = 0; i < 4; i++) {
        wq[i] = bf2f(conv_w[cqk * 4 + i]);
        wv[i] = bf2f(conv_w[cv * 4 + i]);
    }
    uint16_t *stq = conv_state + (size_t)s * cd * 3 + cqk * 3;
    uint16_t *stv = conv_state + (size_t)s * cd * 3 + cv * 3;
    uint16_t q0 = stq[0], q1 = stq[1], q2 = stq[2];
    uint16_t v0 = stv[0], v1 = stv[1], v2 = stv[2];

    float *Sc = S + ((size_t)s * hv + h) * DK * DV + j;
    float sr[DK];
#pragma unroll
    for (int i = 0; i < DK; i++) sr[i] = Sc[(size_t)i * DV];

    const float wo = bf2f(onorm_w[j]);
    const int t0 = cu[s], t1 = cu[s + 1];
    for (int t = t0; t < t1; t++) {
        const uint16_t *xt = qkv + (size_t)t * cd;
        uint16_t xq = xt[cqk], xv = xt[cv];
        uint16_t cqv = conv_tap4(wq, bf2f(q0), bf2f(q1), bf2f(q2), bf2f(xq));
        uint16_t cvv = conv_tap4(wv, bf2f(v0), bf2f(v1), bf2f(v2), bf2f(xv));
        q0 = q1; q1 = q2; q2 = xq;
        v0 = v1; v1 = v2; v2 = xv;
        raw[tid] = bf2f(cqv);
        __syncthreads();
        if (tid == 0 || tid == DK) {           // q sum by wave 0, k by wave 2
            const float *xr = raw + tid;
            float ss = 0.0f;
            for (int i = 0; i < DK; i++) ss = ss + xr[i] * xr[i];
            rsq[tid / DK] = 1.0f / sqrtf(ss + kEps);
        } else if (tid == 64 || tid == 64 + DV) {   // waves 1 and 3
            int hh = kh * REP + tid / DV;
            gd[tid / DV] = exp_cr(decay_of(a[(size_t)t * hv + hh], A_log[hh],
                                           dt_bias[hh]));
            bt[tid / DV] = rndf(sigmoid_cr(bf2f(b[(size_t)t * hv + hh])));
        }
        __syncthreads();
        if (tid < DK)
            qn[tid] = (raw[tid] * rsq[0]) * qscale;
        else
            kn[tid - DK] = raw[tid] * rsq[1];
        __syncthreads();

        const float dec = gd[r], beta = bt[r];
        float kv = 0.0f;
#pragma unroll
        for (int i = 0; i < DK; i++) {
            sr[i] = sr[i] * dec;
            kv = kv + kn[i] * sr[i];
        }
        const float delta = (bf2f(cvv) - kv) * beta;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < DK; i++) {
            sr[i] = sr[i] + kn[i] * delta;
            acc = acc + qn[i] * sr[i];
        }
        const float o = rndf(acc);
        ob[r][j] = o;
        __syncthreads();
        if (j == 0) {
            float ss = 0.0f;
            for (int d = 0; d < DV; d++) ss = ss + ob[r][d] * ob[r][d];
            rso[r] = 1.0f / sqrtf(ss / (float)DV + kEps);
        }
        __syncthreads();
        const float x1 = rndf(o * rso[r]);
        const float x2 = rndf(x1 * wo);
        const float zf = bf2f(z[(size_t)t * vd + (size_t)h * DV + j]);
        y[(size_t)t * vd + (size_t)h * DV + j] = f2bf(x2 * (zf * sigmoid_cr(zf)));
    }
    stq[0] = q0; stq[1] = q1; stq[2] = q2;
    stv[0] = v0; stv[1] = v1; stv[2] = v2;
#pragma unroll
    for (int i = 0; i < DK; i++) Sc[(size_t)i * DV] = sr[i];
}

}  // namespace

// ======================================================================
// C ABI
// ======================================================================
extern "C" {

int apus_hip_gdn_conv1d(const uint16_t *x, const uint16_t *w, uint16_t *out,
                        size_t C, size_t T, uint16_t *state) {
    APUS_READY();
    APUS_STAGE(dx, uint16_t, kScratchIn, x, T * C * 2);
    APUS_STAGE(dw, uint16_t, kScratchIn2, w, C * 4 * 2);
    APUS_STAGE(ds, uint16_t, kScratchIn3, state, C * 3 * 2);
    uint16_t *dout = (uint16_t *)scratch(kScratchOut, T * C * 2);
    if (!dout) return kErrHip;
    if (C) {
        k_conv1d<<<cdiv(C, 256), 256, 0, stream()>>>(dx, dw, dout, C, T, ds);
        APUS_LAUNCHED("k_conv1d");
    }
    if (int r = stage_out(out, dout, T * C * 2)) return r;
    return stage_out(state, ds, C * 3 * 2);
}

int apus_hip_gdn_conv1d_step(const uint16_t *x, const uint16_t *w,
                             uint16_t *out, size_t C, uint16_t *state) {
    return apus_hip_gdn_conv1d(x, w, out, C, 1, state);
}

int apus_hip_gdn_decay(const uint16_t *a, const float *A_log,
                       const float *dt_bias, float *g, size_t H) {
    APUS_READY();
    APUS_STAGE(da, uint16_t, kScratchIn, a, H * 2);
    APUS_STAGE(dA, float, kScratchIn2, A_log, H * 4);
    APUS_STAGE(dd, float, kScratchIn3, dt_bias, H * 4);
    float *dg = (float *)scratch(kScratchOut, H * 4);
    if (!dg) return kErrHip;
    if (H) {
        k_decay<<<cdiv(H, 256), 256, 0, stream()>>>(da, dA, dd, dg, H);
        APUS_LAUNCHED("k_decay");
    }
    return stage_out(g, dg, H * 4);
}

int apus_hip_gdn_beta(const uint16_t *b, uint16_t *beta, size_t H) {
    APUS_READY();
    APUS_STAGE(db, uint16_t, kScratchIn, b, H * 2);
    uint16_t *dbeta = (uint16_t *)scratch(kScratchOut, H * 2);
    if (!dbeta) return kErrHip;
    if (H) {
        k_beta<<<cdiv(H, 256), 256, 0, stream()>>>(db, dbeta, H);
        APUS_LAUNCHED("k_beta");
    }
    return stage_out(beta, dbeta, H * 2);
}

int apus_hip_gdn_l2norm(const uint16_t *x, float *y, size_t H, size_t D,
                        float scale) {
    APUS_READY();
    APUS_STAGE(dx, uint16_t, kScratchIn, x, H * D * 2);
    float *dy = (float *)scratch(kScratchOut, H * D * 4);
    if (!dy) return kErrHip;
    if (H) {
        k_l2norm<<<cdiv(H, 64), 64, 0, stream()>>>(dx, dy, H, D, scale);
        APUS_LAUNCHED("k_l2norm");
    }
    return stage_out(y, dy, H * D * 4);
}

int apus_hip_gdn_recurrent(float *S, const float *q, const float *k,
                           const uint16_t *v, const float *g,
                           const uint16_t *beta, float *o, size_t T,
                           size_t H, size_t Dk, size_t Dv) {
    APUS_READY();
    APUS_STAGE(dS, float, kScratchIn, S, H * Dk * Dv * 4);
    APUS_STAGE(dq, float, kScratchIn2, q, T * H * Dk * 4);
    APUS_STAGE(dk, float, kScratchIn3, k, T * H * Dk * 4);
    APUS_STAGE(dv, uint16_t, kScratchIn4, v, T * H * Dv * 2);
    APUS_STAGE(dg, float, kScratchIn5, g, T * H * 4);
    APUS_STAGE(db, uint16_t, kScratchIn6, beta, T * H * 2);
    float *dout = (float *)scratch(kScratchOut, T * H * Dv * 4);
    if (!dout) return kErrHip;
    if (H && Dv) {
        unsigned nt = Dv < 256 ? (unsigned)((Dv + 63) / 64 * 64) : 256u;
        k_recurrent<<<(unsigned)H, nt, 0, stream()>>>(dS, dq, dk, dv, dg, db,
                                                      dout, T, H, Dk, Dv);
        APUS_LAUNCHED("k_recurrent");
    }
    if (int r = stage_out(o, dout, T * H * Dv * 4)) return r;
    return stage_out(S, dS, H * Dk * Dv * 4);
}

int apus_hip_gdn_step(float *S, const float *q, const float *k,
                      const uint16_t *v, const float *g, const uint16_t *beta,
                      float *o, size_t H, size_t Dk, size_t Dv) {
    return apus_hip_gdn_recurrent(S, q, k, v, g, beta, o, 1, H, Dk, Dv);
}

int apus_hip_gdn_step_mt(float *S, const float *q, const float *k,
                         const uint16_t *v, const float *g,
                         const uint16_t *beta, float *o, size_t H, size_t Dk,
                         size_t Dv) {
    return apus_hip_gdn_recurrent(S, q, k, v, g, beta, o, 1, H, Dk, Dv);
}

int apus_hip_gdn_onorm(const uint16_t *o, const uint16_t *z,
                       const uint16_t *w, uint16_t *y, size_t H, size_t D) {
    APUS_READY();
    APUS_STAGE(dov, uint16_t, kScratchIn, o, H * D * 2);
    APUS_STAGE(dz, uint16_t, kScratchIn2, z, H * D * 2);
    APUS_STAGE(dw, uint16_t, kScratchIn3, w, D * 2);
    uint16_t *dy = (uint16_t *)scratch(kScratchOut, H * D * 2);
    if (!dy) return kErrHip;
    if (H && D) {
        k_onorm<<<(unsigned)H, 128, 0, stream()>>>(dov, dz, dw, dy, D);
        APUS_LAUNCHED("k_onorm");
    }
    return stage_out(y, dy, H * D * 2);
}

int apus_hip_gdn_decode(const ApusHipGdnLayer *L, size_t B,
                        const int32_t *cu, const uint16_t *qkv,
                        const uint16_t *z, const uint16_t *a,
                        const uint16_t *b, uint16_t *conv_state, float *S,
                        uint16_t *y) {
    APUS_READY();
    if (!L || !cu) return set_error(kErrArgument, "NULL layer or offsets");
    if (L->dk != DK || L->dv != DV || L->hv != REP * L->hk || L->hk == 0)
        return set_error(kErrUnsupported,
                         "gdn_decode supports dk=dv=128, hv=2*hk (got hk=%zu "
                         "hv=%zu dk=%zu dv=%zu)",
                         L->hk, L->hv, L->dk, L->dv);
    if (B == 0) return kOk;
    for (size_t s = 0; s < B; s++)
        if (cu[s + 1] < cu[s] || cu[0] != 0)
            return set_error(kErrArgument, "token offsets must ascend from 0");
    const int32_t *dcu =
        (const int32_t *)upload_small(kScratchMeta, cu, (B + 1) * 4);
    if (!dcu) return kErrHip;
    float qscale = (float)pow((double)L->dk, -0.5);
    k_gdn_decode<<<(unsigned)(B * L->hk), NT, 0, stream()>>>(
        dcu, qkv, z, a, b, L->conv_w, L->A_log, L->dt_bias, L->onorm_w,
        conv_state, S, y, (int)L->hk, qscale);
    APUS_LAUNCHED("k_gdn_decode");
    return kOk;
}

}  // extern "C"
