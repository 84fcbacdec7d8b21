// gdn_dev.h -- Gated DeltaNet device helpers shared by the drop-in ops and
// the batched mixer kernels.
#pragma once
#include "apus_dev.h"

namespace apus {

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
    float co = rndf(acc);
    return f2bf(co * sigmoid_cr(co));
}

// The same with the SiLU taken from the bf16-code table (act_tables.hip):
// rnd(co * sigmoid(co)) is a function of co's code, so the result is
// identical.
__device__ __forceinline__ uint16_t conv_tap4_tab(const float w[4], float s0, float s1,
                                                  float s2, float x,
                                                  const uint16_t *__restrict__ silu_bf) {
    float acc = 0.0f;
    acc = acc + w[0] * s0;
    acc = acc + w[1] * s1;
    acc = acc + w[2] * s2;
    acc = acc + w[3] * x;
    return silu_bf[f2bf(acc)];
}

// Decay gate g = -exp(A_log) * softplus(a + dt_bias) (c/gdn.h:34-40).
__device__ __forceinline__ float decay_of(uint16_t a, float A_log,
                                          float dt_bias) {
    float t = bf2f(a) + dt_bias;
    return -exp_cr(A_log) * softplus_cr(t);
}

}  // namespace apus
