// gdn_ops.hip -- Gated DeltaNet ops for gfx950.
//
// Drop-in ops (apus_hip_gdn_*): the argument lists of c/gdn.h:107-192,
// host pointers, every sum in the reference's ascending order with one
// IEEE rounding per mul/add (FP contraction is off), so results equal the
// scalar anchors up to libm ulps. The batched device-resident mixer lives
// in gdn_mixer.hip.
#include <stdint.h>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"
#include "gdn_dev.h"

using namespace apus;

namespace {

constexpr float kEps = 1e-6f;

// ---- (a) conv1d k=4 + SiLU, one thread per channel -------------------
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

}  // extern "C"
