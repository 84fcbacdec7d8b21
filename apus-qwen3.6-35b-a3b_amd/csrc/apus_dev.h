// apus_dev.h -- device helpers shared by the gfx950 kernels.
//
// bf16 storage travels as uint16_t codes. Widening is exact (code << 16);
// narrowing is round-to-nearest-even with NaN passed through, the same
// rule as the reference's apus_bf16_bits (c/bf16.h:268-274).
//
// Transcendentals that feed a bf16 rounding point (sigmoid, softplus,
// decay) are evaluated in float64 and rounded once to float32, i.e. the
// correctly rounded fp32 value in all but astronomically rare cases.
// glibc's expf/log1pf are within an ulp of that, so results match the
// reference's anchors except at isolated rounding ties; the reference
// itself treats libm as a tolerance class (c/gdn.h:77-82).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace apus {

__device__ __forceinline__ float bf2f(uint16_t b) {
    return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ uint16_t f2bf(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(u >> 16);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float rndf(float x) { return bf2f(f2bf(x)); }

__device__ __forceinline__ float exp_cr(float x) {
    return (float)exp((double)x);
}

__device__ __forceinline__ float sigmoid_cr(float z) {
    return 1.0f / (1.0f + exp_cr(-z));
}

__device__ __forceinline__ float softplus_cr(float x) {
    return x > 20.0f ? x : (float)log1p((double)exp_cr(x));
}

// Exact IEEE single ops that the compiler may not fuse or reorder. The
// kernels that promise reference-order results are compiled with FP
// contraction off as well; these make the intent explicit at call sites.
__device__ __forceinline__ float fmul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fadd(float a, float b) { return __fadd_rn(a, b); }

}  // namespace apus
