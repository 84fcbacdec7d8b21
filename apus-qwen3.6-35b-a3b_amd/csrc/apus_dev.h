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

// exp(x) for x <= 0 in fp32 via the hardware exp2 with the rounding error
// of x*log2(e) folded back in (a few ulp). For the tolerance-class paths
// (attention scores, chunked GDN decay factors), not for rounding points
// that must match the reference.
__device__ __forceinline__ float exp_fast(float x) {
    if (x == -INFINITY) return 0.0f;
    const float L2E = 1.44269504088896341f;
    const float t = x * L2E;
    const float r = fmaf(x, L2E, -t) + x * 1.925963001e-8f;
    const float e = __builtin_amdgcn_exp2f(t);
    return fmaf(e, r * 0.693147180559945f, e);
}

// Value of `v` in lane `src` of the wavefront (src must be uniform).
__device__ __forceinline__ float lane_bcast(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// Raw buffer access: one buffer resource (base + size in SGPRs) per tile,
// a per-lane VGPR byte offset and a uniform (SGPR/immediate) byte offset.
// A 128-row column walk then costs one address VGPR instead of a 64-bit
// pointer per row, which is what keeps a 128-float column in registers
// at 3 waves per SIMD. Out-of-range offsets read 0 and drop writes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base,
                                                           uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                             (int)bytes, 0x00020000);
}
__device__ __forceinline__ float buf_ld(__amdgpu_buffer_rsrc_t r, int voff,
                                        int soff) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void buf_st(__amdgpu_buffer_rsrc_t r, int voff,
                                       int soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r,
                                          voff, soff, 0);
}

// 16-byte raw buffer access, bound to the LLVM intrinsics by name. The
// __builtin_amdgcn_raw_buffer_{load,store}_b128 builtins of this toolchain
// (ROCm 7.2 clang) lower to single-dword instructions, leaving three of the
// four lanes undefined; the float-vector intrinsic keeps all four.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ f32x4_t llvm_raw_ptr_buffer_load_v4f32(__amdgpu_buffer_rsrc_t r, int voff,
                                                  int soff, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v4f32");
__device__ void llvm_raw_ptr_buffer_store_v4f32(f32x4_t v, __amdgpu_buffer_rsrc_t r,
                                                int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.store.v4f32");

// Streaming (non-temporal, cache policy bit 1) variants: a tile that is
// read once and written once per call should not displace reusable lines
// from L2/MALL; on the GDN state stream this is worth ~15% of bandwidth.
constexpr int kCpolNT = 2;
__device__ __forceinline__ f32x4_t buf_ld4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return llvm_raw_ptr_buffer_load_v4f32(r, voff, soff, kCpolNT);
}
__device__ __forceinline__ void buf_st4(__amdgpu_buffer_rsrc_t r, int voff, int soff,
                                        f32x4_t v) {
    llvm_raw_ptr_buffer_store_v4f32(v, r, voff, soff, kCpolNT);
}

// ---- global -> LDS DMA ----------------------------------------------------
// buffer_load ... lds: each lane's 16 bytes land at the LDS byte address in
// M0 + 16 * lane, without passing through VGPRs. Issued from inline asm, so
// the compiler does not count these loads: the caller waits for them with
// an explicit s_waitcnt vmcnt before reading the LDS they fill, and waits
// for its own reads of that LDS (lgkmcnt) before refilling it.
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// Buffer resource (SGPRs) over `bytes` bytes at base; offsets past the
// end read as zero.
__device__ __forceinline__ i32x4 dma_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                 __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff),
                 __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// A wave-uniform 4-byte read through the scalar cache (s_buffer_load):
// the value lands in an SGPR and is counted by lgkmcnt, never by the
// vector-memory counter, so reading it cannot make a wave wait for its
// streaming loads (a vector load inside a branch also makes the compiler
// drain that counter at the join). bytes bounds the resource; reads past
// it return 0.
__device__ int llvm_s_buffer_load_i32(i32x4 rsrc, int off, int aux)
    __asm("llvm.amdgcn.s.buffer.load.i32");
__device__ __forceinline__ int sload_i32(const int32_t *base, uint32_t bytes, int index) {
    return llvm_s_buffer_load_i32(dma_rsrc(base, bytes), index * 4, 0);
}

// one 16-byte copy per lane from byte offset voff (per lane) + soff
// (uniform) to LDS byte address lds (uniform) + 16 * lane
__device__ __forceinline__ void dma16(i32x4 r, int voff, int soff, uint32_t lds) {
    soff = __builtin_amdgcn_readfirstlane(soff);
    lds = __builtin_amdgcn_readfirstlane(lds);
    // (M0 is bound as an operand, so the compiler sets it and knows it changed)
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
                 :: "v"(voff), "s"(r), "s"(soff), "{m0}"(lds) : "memory");
}

// Exact IEEE single ops that the compiler may not fuse or reorder. The
// kernels that promise reference-order results are compiled with FP
// contraction off as well; these make the intent explicit at call sites.
__device__ __forceinline__ float fmul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fadd(float a, float b) { return __fadd_rn(a, b); }

}  // namespace apus
