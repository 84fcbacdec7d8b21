// gdn_dev.h -- Gated DeltaNet device helpers shared by the drop-in ops and
// the batched mixer kernels.
#pragma once
#include "apus_dev.h"

namespace apus {

// rnd(co * sigmoid(co)) for a bf16 value co, with the sigmoid as the
// reference forms it (exp correctly rounded, fp32 add and divide, fp32
// product; c/gdn.h:19-33). An fp32 evaluation through the hardware exp2 and
// reciprocal lands within ~11 ulp of that product for |co| <= 16 (x log2(e)
// rounding ~5.5 ulp through exp2, exp2 and rcp 1 ulp each, the remaining
// roundings), so its bf16 rounding is the reference's unless the product
// lies within 16 ulp of a rounding midpoint (every finite code is checked
// against the reference formula by the conv1d op's test). ok = false for
// those, for |co| outside [2^-60, 16] and for non-finite co: the caller
// then takes the reference formula (or the bf16-code table).
__device__ __forceinline__ uint16_t silu_fast(float co, bool &ok) {
    const float ax = fabsf(co);
    const float e = __builtin_amdgcn_exp2f(co * -1.44269504088896341f);
    const float p = co * __builtin_amdgcn_rcpf(1.0f + e);
    const uint32_t b = __float_as_uint(p), lo = b & 0xffffu;
    ok = ax <= 16.0f && ax >= 0x1p-60f && (lo > 0x8000u + 16u || lo + 16u < 0x8000u);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ uint16_t silu_bf16(float co) {
    bool ok;
    const uint16_t r = silu_fast(co, ok);
    return ok ? r : f2bf(co * sigmoid_cr(co));
}

// Causal conv1d k=4 + SiLU for one channel (c/gdn.h:19-33, 220-228): the
// four taps accumulate oldest first with one rounding per mul and add,
// then rnd (point 1), SiLU in fp32, rnd (point 2).
__device__ __forceinline__ uint16_t conv_tap4(const float w[4], float s0,
                                              float s1, float s2, float x) {
    float acc = 0.0f;
    acc = acc + w[0] * s0;
    acc = acc + w[1] * s1;
    acc = acc + w[2] * s2;
    acc = acc + w[3] * x;
    return silu_bf16(rndf(acc));
}

// The 4-tap conv sum in tap order, as a bf16 code (the SiLU table's index).
__device__ __forceinline__ uint16_t conv_sum4_code(const float w[4], float s0, float s1, float s2,
                                                   float x) {
    float acc = 0.0f;
    acc = acc + w[0] * s0;
    acc = acc + w[1] * s1;
    acc = acc + w[2] * s2;
    acc = acc + w[3] * x;
    return f2bf(acc);
}

// The same with the SiLU taken from the bf16-code table (act_tables.hip):
// rnd(co * sigmoid(co)) is a function of co's code, so the result is
// identical.
__device__ __forceinline__ uint16_t conv_tap4_tab(const float w[4], float s0, float s1,
                                                  float s2, float x,
                                                  const uint16_t *__restrict__ silu_bf) {
    return silu_bf[conv_sum4_code(w, s0, s1, s2, x)];
}

// Decay gate g = -exp(A_log) * softplus(a + dt_bias) (c/gdn.h:34-40).
__device__ __forceinline__ float decay_of(uint16_t a, float A_log,
                                          float dt_bias) {
    float t = bf2f(a) + dt_bias;
    return -exp_cr(A_log) * softplus_cr(t);
}

// Ascending sum of squares of a row of 128 bf16 codes (16-byte aligned),
// one rounding per mul and add (the l2norm's ordered sum, c/gdn.h:402-416).
// The squares of bf16 values are exact in fp32 (8-bit significands) when
// in the normal range, so one fused multiply-add rounds where the
// reference's multiply-then-add does (only a square below 2^-126 could
// differ, and only while the running sum is that small too).
__device__ __forceinline__ float row_sumsq(const uint16_t *row) {
    typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));
    const u16x8_t *x8 = reinterpret_cast<const u16x8_t *>(row);
    float ss = 0.0f;
#pragma unroll 4
    for (int j = 0; j < 128 / 8; j++) {
        const u16x8_t v = x8[j];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float x = bf2f(v[i]);
            ss = fmaf(x, x, ss);
        }
    }
    return ss;
}

// eps of the q/k l2norm, 1/sqrt(sum x^2 + eps) (c/gdn.h:402-416)
constexpr float kL2Eps = 1e-6f;

}  // namespace apus
