// attn_ops.hip -- gated-GQA drop-in ops for gfx950 (c/attn.h:87-158).
//
// Host-pointer entry points with the reference's argument lists. Every
// reduction keeps the reference's ascending order and one IEEE rounding
// per op (FP contraction is off for this file), so outputs equal the
// scalar anchors up to libm ulps (expf in the softmax and the gate).
// RoPE reads cos/sin codes computed on the host with the platform libm
// exactly as c/attn.h:251-255, so RoPE itself is bit-exact.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"

using namespace apus;

namespace {

constexpr float kEps = 1e-6f;

// (a) (1+w) RMSNorm over `rows` rows of N; one block per row.
__global__ void k_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *y,
                          size_t N) {
    const uint16_t *xr = x + (size_t)blockIdx.x * N;
    uint16_t *yr = y + (size_t)blockIdx.x * N;
    __shared__ float rs_s;
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (size_t i = 0; i < N; i++) {
            float v = bf2f(xr[i]);
            ss = ss + v * v;
        }
        rs_s = 1.0f / sqrtf(ss / (float)N + kEps);
    }
    __syncthreads();
    float rs = rs_s;
    for (size_t i = threadIdx.x; i < N; i += blockDim.x)
        yr[i] = f2bf((bf2f(xr[i]) * rs) * (1.0f + bf2f(w[i])));
}

// (b) partial NeoX RoPE of one vector with a host-made cos/sin row.
__global__ void k_rope(const uint16_t *x, uint16_t *y, size_t D, size_t rot,
                       const uint16_t *cs) {
    size_t R = rot / 2;
    for (size_t i = threadIdx.x; i < D; i += blockDim.x) {
        if (i < R) {
            float c = bf2f(cs[i]), s = bf2f(cs[R + i]);
            float lo = bf2f(x[i]), hi = bf2f(x[i + R]);
            y[i] = f2bf(rndf(lo * c) + rndf(-hi * s));
            y[i + R] = f2bf(rndf(hi * c) + rndf(lo * s));
        } else if (i >= rot) {
            y[i] = x[i];
        }
    }
}

// (c) eager GQA rows, one block per (row, head) unit in [u0, u0+nu).
// Scores, max, ascending exp-sum, bf16 P and the ascending P.V follow
// c/attn.h:337-368 step for step. abuf/ebuf: [nu][Tk] scratch.
__global__ __launch_bounds__(256) void k_gqa_rows(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ vc, uint16_t *__restrict__ o, size_t Tq,
    size_t Tk, size_t H, size_t Hkv, size_t D, float scale, size_t u0,
    uint16_t *__restrict__ abuf, float *__restrict__ ebuf) {
    const size_t u = u0 + blockIdx.x;
    const size_t t = u / H, h = u % H, hk = h / (H / Hkv);
    const size_t p = Tk - Tq + t;
    const size_t rs = Hkv * D;
    const uint16_t *qh = q + (t * H + h) * D;
    const uint16_t *kb = kc + hk * D, *vb = vc + hk * D;
    uint16_t *ab = abuf + (size_t)blockIdx.x * Tk;
    float *eb = ebuf + (size_t)blockIdx.x * Tk;
    __shared__ float red[256];
    __shared__ float m_s, s_s;

    float mloc = -INFINITY;
    for (size_t j = threadIdx.x; j <= p; j += blockDim.x) {
        const uint16_t *kr = kb + j * rs;
        float dot = 0.0f;
        for (size_t d = 0; d < D; d++) dot = dot + bf2f(qh[d]) * bf2f(kr[d]);
        uint16_t A = f2bf(rndf(dot) * scale);
        ab[j] = A;
        mloc = fmaxf(mloc, bf2f(A));
    }
    red[threadIdx.x] = mloc;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off)
            red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + off]);
        __syncthreads();
    }
    if (threadIdx.x == 0) m_s = red[0];
    __syncthreads();
    const float m = m_s;
    for (size_t j = threadIdx.x; j <= p; j += blockDim.x)
        eb[j] = exp_cr(bf2f(ab[j]) - m);
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (size_t j = 0; j <= p; j++) s = s + eb[j];
        s_s = s;
    }
    __syncthreads();
    const float s = s_s;
    for (size_t j = threadIdx.x; j <= p; j += blockDim.x)
        ab[j] = f2bf(eb[j] / s);
    __syncthreads();
    for (size_t d = threadIdx.x; d < D; d += blockDim.x) {
        float acc = 0.0f;
        for (size_t j = 0; j <= p; j++)
            acc = acc + bf2f(ab[j]) * bf2f(vb[j * rs + d]);
        o[(t * H + h) * D + d] = f2bf(acc);
    }
}

// (d) sigmoid output gate.
__global__ void k_outgate(const uint16_t *o, const uint16_t *gate,
                          uint16_t *y, size_t N) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < N) {
        float g = rndf(sigmoid_cr(bf2f(gate[i])));
        y[i] = f2bf(bf2f(o[i]) * g);
    }
}

uint16_t host_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(u >> 16);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

}  // namespace

extern "C" {

int apus_hip_attn_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *y,
                          size_t N) {
    APUS_READY();
    APUS_STAGE(dx, uint16_t, kScratchIn, x, N * 2);
    APUS_STAGE(dw, uint16_t, kScratchIn2, w, N * 2);
    uint16_t *dy = (uint16_t *)scratch(kScratchOut, N * 2);
    if (!dy) return kErrHip;
    if (N) {
        k_rmsnorm<<<1, 256, 0, stream()>>>(dx, dw, dy, N);
        APUS_LAUNCHED("k_rmsnorm");
    }
    return stage_out(y, dy, N * 2);
}

int apus_hip_attn_rope(const uint16_t *x, uint16_t *y, size_t D, size_t rot,
                       float pos, double theta) {
    APUS_READY();
    if (rot > D || (rot & 1))
        return set_error(kErrArgument, "rope: rot=%zu must be even and <= D=%zu",
                         rot, D);
    size_t R = rot / 2;
    std::vector<uint16_t> cs(rot ? rot : 1);
    for (size_t i = 0; i < R; i++) {
        float invf = (float)(1.0 / pow(theta, 2.0 * (double)i / (double)rot));
        float ang = pos * invf;
        cs[i] = host_bf16(cosf(ang));
        cs[R + i] = host_bf16(sinf(ang));
    }
    APUS_STAGE(dx, uint16_t, kScratchIn, x, D * 2);
    APUS_STAGE(dcs, uint16_t, kScratchIn2, cs.data(), cs.size() * 2);
    uint16_t *dy = (uint16_t *)scratch(kScratchOut, D * 2);
    if (!dy) return kErrHip;
    if (D) {
        k_rope<<<1, 256, 0, stream()>>>(dx, dy, D, rot, dcs);
        APUS_LAUNCHED("k_rope");
    }
    return stage_out(y, dy, D * 2);
}

int apus_hip_attn_gqa(const uint16_t *q, const uint16_t *kc,
                      const uint16_t *vc, uint16_t *o, size_t Tq, size_t Tk,
                      size_t H, size_t Hkv, size_t D, float scale,
                      uint16_t *abuf, float *ebuf) {
    (void)abuf;
    (void)ebuf;   // device scratch replaces the caller's CPU scratch
    APUS_READY();
    if (Tq > Tk || Hkv == 0 || H % Hkv)
        return set_error(kErrArgument, "gqa: need Tq<=Tk and Hkv | H");
    APUS_STAGE(dq, uint16_t, kScratchIn, q, Tq * H * D * 2);
    APUS_STAGE(dk, uint16_t, kScratchIn2, kc, Tk * Hkv * D * 2);
    APUS_STAGE(dv, uint16_t, kScratchIn3, vc, Tk * Hkv * D * 2);
    uint16_t *dout = (uint16_t *)scratch(kScratchOut, Tq * H * D * 2);
    if (!dout) return kErrHip;
    size_t units = Tq * H;
    size_t per = Tk ? ((size_t)256 << 20) / (Tk * 6) : units;
    if (per < 1) per = 1;
    if (per > 65535) per = 65535;
    size_t nb = units < per ? units : per;
    uint16_t *da = (uint16_t *)scratch(kScratchWork, nb * Tk * 2);
    float *de = (float *)scratch(kScratchWork2, nb * Tk * 4);
    if (!da || !de) return kErrHip;
    for (size_t u0 = 0; u0 < units; u0 += per) {
        size_t n = units - u0 < per ? units - u0 : per;
        k_gqa_rows<<<(unsigned)n, 256, 0, stream()>>>(
            dq, dk, dv, dout, Tq, Tk, H, Hkv, D, scale, u0, da, de);
        APUS_LAUNCHED("k_gqa_rows");
    }
    return stage_out(o, dout, Tq * H * D * 2);
}

int apus_hip_attn_gqa_decode(const uint16_t *q, const uint16_t *kc,
                             const uint16_t *vc, uint16_t *o, size_t Tk,
                             size_t H, size_t Hkv, size_t D, float scale,
                             uint16_t *abuf, float *ebuf) {
    return apus_hip_attn_gqa(q, kc, vc, o, 1, Tk, H, Hkv, D, scale, abuf,
                             ebuf);
}

int apus_hip_attn_gqa_mt(const uint16_t *q, const uint16_t *kc,
                         const uint16_t *vc, uint16_t *o, size_t Tq,
                         size_t Tk, size_t H, size_t Hkv, size_t D,
                         float scale) {
    return apus_hip_attn_gqa(q, kc, vc, o, Tq, Tk, H, Hkv, D, scale, nullptr,
                             nullptr);
}

int apus_hip_attn_gqa_decode_mt(const uint16_t *q, const uint16_t *kc,
                                const uint16_t *vc, uint16_t *o, size_t Tk,
                                size_t H, size_t Hkv, size_t D, float scale) {
    return apus_hip_attn_gqa(q, kc, vc, o, 1, Tk, H, Hkv, D, scale, nullptr,
                             nullptr);
}

int apus_hip_attn_outgate(const uint16_t *o, const uint16_t *gate,
                          uint16_t *y, size_t N) {
    APUS_READY();
    APUS_STAGE(dov, uint16_t, kScratchIn, o, N * 2);
    APUS_STAGE(dg, uint16_t, kScratchIn2, gate, N * 2);
    uint16_t *dy = (uint16_t *)scratch(kScratchOut, N * 2);
    if (!dy) return kErrHip;
    if (N) {
        k_outgate<<<cdiv(N, 256), 256, 0, stream()>>>(dov, dg, dy, N);
        APUS_LAUNCHED("k_outgate");
    }
    return stage_out(y, dy, N * 2);
}

}  // extern "C"
