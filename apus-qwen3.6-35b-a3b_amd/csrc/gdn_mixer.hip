// gdn_mixer.hip -- batched, device-resident Gated DeltaNet mixer for gfx950:
// the op sequence of c/layer.h:250-273 for B sequences.
//
// Device state layout (tier 2). The recurrent state of one (sequence,
// v-head) is a 128x128 fp32 matrix S[i][j] (i = key dim, j = value dim,
// reference layout c/gdn.h:149-156). In HBM the library keeps it "column
// packed": for column half c = j/64, row quad q = i/4, lane l = j%64 and
// r = i%4, element S[i][j] sits at
//     ((c*32 + q)*64 + l)*4 + r        (floats, within the 64 KiB matrix)
// so the wavefront that owns columns c*64..c*64+63 reads four consecutive
// rows of its column with one 16-byte load per lane and 1 KiB per
// instruction: 32 loads per lane cover the column, well inside the 63
// outstanding memory instructions a wave can track. apus_hip_gdn_state_
// pack/unpack convert from/to the reference layout.
//
// Kernels:
//   k_gdn_decode  fused decode/verify, one workgroup per (sequence, K head)
//   k_gdn_prep    conv + l2norm + gates for every token (prefill)
//   k_gdn_post    gated RMSNorm + new conv state (prefill)
//   k_gdn_pack / k_gdn_unpack  state layout conversion
//
// Every sum keeps the reference's ascending order with one IEEE rounding
// per op (FP contraction is off), so y and S equal the scalar anchors up
// to libm ulps in the gates.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"
#include "gdn_dev.h"
#include "gdn_mixer.h"

using namespace apus;

namespace {

constexpr int DK = 128, DV = 128, REP = 2;
constexpr float kEps = 1e-6f;

__device__ __forceinline__ int seq_of(const int32_t *cu, int B, int t) {
    int lo = 0, hi = B - 1;          // largest s with cu[s] <= t
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// ---- state layout conversion -------------------------------------------
__device__ __forceinline__ size_t packed_index(int i, int j) {
    return ((size_t)((j >> 6) * 32 + (i >> 2)) * 64 + (j & 63)) * 4 + (i & 3);
}

__global__ void k_gdn_pack(const float *__restrict__ src, float *__restrict__ dst,
                           size_t nmat) {
    size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nmat * DK * DV) return;
    size_t m = e / (DK * DV), w = e % (DK * DV);
    int i = (int)(w / DV), j = (int)(w % DV);
    dst[m * DK * DV + packed_index(i, j)] = src[e];
}

__global__ void k_gdn_unpack(const float *__restrict__ src, float *__restrict__ dst,
                             size_t nmat) {
    size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nmat * DK * DV) return;
    size_t m = e / (DK * DV), w = e % (DK * DV);
    int i = (int)(w / DV), j = (int)(w % DV);
    dst[e] = src[m * DK * DV + packed_index(i, j)];
}

// ---- fused decode -------------------------------------------------------
// One workgroup per item (sequence, K head), 4 wavefronts, two workgroups
// per CU (the state tile lives in registers: 128 per lane). Item (s, kh)
// serves v-heads 2kh and 2kh+1; wave w serves v-head r = w >> 1, value
// columns (w & 1)*64 + lane of it; thread t also owns q channel t
// (t < 128) or k channel t-128 of the K head, and the t-th of the item's
// 256 v channels.
//
// The reference evaluates c/layer.h:250-273 + c/gdn.h:471-504 token by
// token; every op and operand order of that is kept, but scheduled so that
// no serial single-lane chain runs once per token. Per chunk of up to KT
// tokens:
//   A  conv of q, k, v and silu(z) for all the chunk's tokens (thread-
//      parallel); then the 2n l2-norm sums and the 2n gate pairs, one lane
//      each, in parallel (waves 0 and 1); normalised q, k to LDS.
//   B  the recurrence, each wave on its own columns with no barrier.
//   C  the 2n output-norm sums in parallel lanes, then y.
// With one token the state tile is loaded before phase A (the gate math
// runs under the loads); with several, after it (the tile's 128 registers
// are then not live through phase A). The other workgroup on the CU runs
// while this one waits for memory or sits in a serial phase.
//
// MODE 0: one token per sequence; 1: up to KT; 2: any number, in chunks of
// KT (the host picks the mode from the largest token count).
// Token offsets arrive by value for up to kInlineSeqs sequences, and with
// them the state slot maps when all 3B+1 words fit (B <= 320): then a
// slotted step uploads nothing. cu[0..B] are the offsets, cu[B+1..2B] the
// input slots and cu[2B+1..3B] the output slots.
constexpr int kInlineSeqs = 480;
constexpr int kInlineWords = 2 * kInlineSeqs + 1;
template <int NW> struct CuArgsN {
    int32_t cu[NW];
};
using CuArgs = CuArgsN<kInlineWords>;
// A call of a few sequences passes a short argument block instead: the
// launch copies the whole by-value block, and 3.8 KiB of it cost ~0.3 us of
// a one-sequence step.
constexpr int kSmallWords = 16;

constexpr int KT = 4;                          // tokens per chunk

// Ascending sum of squares of 128 LDS floats, each a bf16 value (one
// rounding per mul and add; fused as in apus::row_sumsq, exact for the
// same reason). Unrolled by four 16-byte reads: enough reads in flight to
// cover most of their latency, few enough registers to run beside a live
// state tile.
__device__ __forceinline__ float sumsq128(const float *x) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    float ss = 0.0f;
#pragma unroll 4
    for (int i = 0; i < 32; i++) {
        const float4 v = x4[i];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    return ss;
}

// ---- phase B: the recurrence of one chunk on one wave's columns ---------
// c/gdn.h:482-503 on column j for the chunk's n tokens: per token a decay +
// k.S pass and an update + q.S pass. k and q reach every lane as LDS
// broadcast reads, four values per 16-byte read, so the VALU only does the
// seven operations per state element that the reference's rounding order
// needs. Reads run two groups of four rows ahead; a memory clobber and a
// scheduling barrier per group keep the compiler from hoisting them all
// (the state slice holds 128 registers). o_k = rnd(q_k . S_k) goes to
// ob[k] and, when tracing, to tr[k * tr_stride].
__device__ __forceinline__ void recur_chunk(float (&sr)[DK], const float (*raw)[2 * DK],
                                            const float2 (*gt)[REP], const float (*cvs)[256],
                                            float (*ob)[REP][DV], int n, int r, int j, int tid,
                                            uint16_t *tr, size_t tr_stride) {
#pragma unroll 1
    for (int k = 0; k < n; k++) {
        const float4 *K4 = reinterpret_cast<const float4 *>(&raw[k][DK]);
        const float4 *Q4 = reinterpret_cast<const float4 *>(&raw[k][0]);
        float kv = 0.0f;
        {   // decay and k.S
            const float g = gt[k][r].x;
            float4 kn0 = K4[0], kn1 = K4[1];
#pragma unroll
            for (int i4 = 0; i4 < DK / 4; i4++) {
                const float4 kk = kn0;
                kn0 = kn1;
                if (i4 + 2 < DK / 4) kn1 = K4[i4 + 2];
                const float ke[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int i = 4 * i4 + e;
                    sr[i] = sr[i] * g;
                    kv = kv + ke[e] * sr[i];
                }
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        {   // update and q.S
            const float delta = (cvs[k][tid] - kv) * gt[k][r].y;
            float acc = 0.0f;
            float4 kn0 = K4[0], kn1 = K4[1];
            float4 qn0 = Q4[0], qn1 = Q4[1];
#pragma unroll
            for (int i4 = 0; i4 < DK / 4; i4++) {
                const float4 kk = kn0, qq = qn0;
                kn0 = kn1;
                qn0 = qn1;
                if (i4 + 2 < DK / 4) {
                    kn1 = K4[i4 + 2];
                    qn1 = Q4[i4 + 2];
                }
                const float ke[4] = {kk.x, kk.y, kk.z, kk.w};
                const float qe[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int i = 4 * i4 + e;
                    sr[i] = sr[i] + ke[e] * delta;
                    acc = acc + qe[e] * sr[i];
                }
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            }
            const float o = rndf(acc);
            ob[k][r][j] = o;
            if (tr) tr[(size_t)k * tr_stride] = f2bf(o);      // (trace) rec_o
        }
    }
}

template <int MODE, int NW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_gdn_decode(
    CuArgsN<NW> ca, const int32_t *__restrict__ dcu, int nseq, const uint16_t *qkv,
    const uint16_t *z, const uint16_t *a, const uint16_t *b, const uint16_t *conv_w,
    const float *A_log, const float *dt_bias, const uint16_t *onorm_w,
    const uint16_t *conv_state, const float *S, uint16_t *conv_out, float *S_out,
    uint16_t *y, int hk, float qscale, const int32_t *__restrict__ slot_in,
    const int32_t *__restrict__ slot_out, int slots_inline, uint16_t *tr_ob) {
    constexpr int KTT = MODE == 0 ? 1 : KT;
    __shared__ __attribute__((aligned(16))) float raw[KTT][2 * DK];  // conv q, k; then normed
    __shared__ __attribute__((aligned(16))) float ob[KTT][REP][DV];  // rnd(o)
    __shared__ float cvs[KTT][256], zgs[KTT][256];   // thread t's conv(v), silu(z)
    __shared__ float rsq[KTT][2], rso[KTT][REP];
    __shared__ float2 gt[KTT][REP];                                   // exp(g), beta

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv_ = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = wv_ >> 1, half = wv_ & 1, j = half * 64 + lane;
    const int hv = hk * REP;
    const int kd = hk * DK, vd = hv * DV, cd = 2 * kd + vd;
    const int s = blockIdx.x / hk, kh = blockIdx.x % hk;
    const bool inl = dcu == nullptr;
    const int a0 = inl ? ca.cu[s] : 0, a1 = inl ? ca.cu[s + 1] : 0;
    int d0 = 0, d1 = 0;
    if (!inl) {
        d0 = dcu[s];
        d1 = dcu[s + 1];
    }
    const int t0 = __builtin_amdgcn_readfirstlane(inl ? a0 : d0);
    const int t1 = __builtin_amdgcn_readfirstlane(inl ? a1 : d1);
    if (t0 == t1) return;
    const int nt = t1 - t0;
    // the state slots this sequence reads and writes (identity without a
    // slot map)
    const int ia = slots_inline ? ca.cu[nseq + 1 + s] : 0;
    const int oa = slots_inline ? ca.cu[2 * nseq + 1 + s] : 0;
    int id = s, od = s;
    if (!slots_inline && slot_in) id = slot_in[s];
    if (!slots_inline && slot_out) od = slot_out[s];
    const int si = __builtin_amdgcn_readfirstlane(slots_inline ? ia : id);
    const int so = __builtin_amdgcn_readfirstlane(slots_inline ? oa : od);
    const int h = kh * REP + r;
    const int cqk = tid < DK ? kh * DK + tid : kd + kh * DK + (tid - DK);
    const int cvg = 2 * kd + kh * REP * DV + tid;   // this thread's v channel
    // gate lanes: wave 1, lane 2k + rr serves token k, v-head 2kh + rr
    const int gk = lane >> 1, grr = lane & 1, gh = kh * REP + grr;

    // Small operands (raw bits).
    const uint2 cwq = *reinterpret_cast<const uint2 *>(conv_w + (size_t)cqk * 4);
    const uint2 cwv = *reinterpret_cast<const uint2 *>(conv_w + (size_t)cvg * 4);
    const uint16_t *stq = conv_state + (size_t)si * cd * 3 + (size_t)cqk * 3;
    const uint16_t *stv = conv_state + (size_t)si * cd * 3 + (size_t)cvg * 3;
    uint32_t w0 = stq[0], w1 = stq[1], w2 = stq[2];
    uint32_t u0 = stv[0], u1 = stv[1], u2 = stv[2];
    uint32_t wo_b = onorm_w[j];
    uint32_t alog_b = __float_as_uint(A_log[gh]), dtb_b = __float_as_uint(dt_bias[gh]);
    uint32_t xq[KTT], xv[KTT], zc[KTT], ag = 0, bg = 0;
    const int n0 = MODE == 0 ? 1 : min(nt, KTT);
#pragma unroll
    for (int k = 0; k < KTT; k++) {
        if (k < n0) {
            const size_t t = (size_t)(t0 + k);
            xq[k] = qkv[t * cd + cqk];
            xv[k] = qkv[t * cd + cvg];
            zc[k] = z[t * vd + kh * REP * DV + tid];
        }
    }
    if (gk < n0) {
        ag = a[(size_t)(t0 + gk) * hv + gh];
        bg = b[(size_t)(t0 + gk) * hv + gh];
    }
    uint32_t c0x = cwq.x, c0y = cwq.y, c1x = cwv.x, c1y = cwv.y;
    const int voff = (half * 32 * 64 + lane) * 16;
    float sr[DK];
    // This wave's 128x64 state tile (32 x 16-byte loads per lane). With the
    // tokens in one chunk (modes 0 and 1) it is loaded before phase A, whose
    // conv, gate and silu math then runs under the loads (186 VGPRs with up
    // to KT tokens, no spills at two waves per SIMD; loading it after phase
    // A cost 7 us per config-4 layer). With several chunks (mode 2) it is
    // loaded after phase A of the first. (The descriptor is made where si
    // and h are known uniform.)
    constexpr bool kEarlyTile = MODE != 2;
    auto load_tile = [&]() {
        const int tix = __builtin_amdgcn_readfirstlane(si * hv + h);
        const auto Sr = buf_rsrc(S + (size_t)tix * DK * DV, DK * DV * 4);
#pragma unroll
        for (int q = 0; q < DK / 4; q++) {
            const f32x4_t v = buf_ld4(Sr, voff, q * 1024);
            sr[4 * q + 0] = v[0];
            sr[4 * q + 1] = v[1];
            sr[4 * q + 2] = v[2];
            sr[4 * q + 3] = v[3];
        }
    };
    if (kEarlyTile) {
        // small loads stay in front of the tile loads: the memory counter
        // retires in order, so a small load behind the tile would make the
        // phase-A math wait for the whole tile
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        load_tile();
        asm volatile("" : "+v"(c0x), "+v"(c0y), "+v"(c1x), "+v"(c1y), "+v"(w0), "+v"(w1),
                     "+v"(w2), "+v"(u0), "+v"(u1), "+v"(u2), "+v"(wo_b), "+v"(alog_b),
                     "+v"(dtb_b), "+v"(ag), "+v"(bg));
        asm volatile("" : "+v"(xq[0]), "+v"(xv[0]), "+v"(zc[0]));
    }
    const float wq[4] = {__uint_as_float(c0x << 16), __uint_as_float(c0x & 0xffff0000u),
                         __uint_as_float(c0y << 16), __uint_as_float(c0y & 0xffff0000u)};
    const float wvv[4] = {__uint_as_float(c1x << 16), __uint_as_float(c1x & 0xffff0000u),
                          __uint_as_float(c1y << 16), __uint_as_float(c1y & 0xffff0000u)};
    const float wo = bf2f((uint16_t)wo_b);

    // modes 0 and 1 hold one chunk (the host checked the token counts)
    const int cend = MODE == 2 ? nt : 1;
    for (int c0 = 0; c0 < cend; c0 += KTT) {
        const int n = MODE == 0 ? 1 : min(KTT, nt - c0);
        if (MODE == 2 && c0 > 0) {                 // a later chunk's inputs
#pragma unroll
            for (int k = 0; k < KTT; k++) {
                if (k < n) {
                    const size_t t = (size_t)(t0 + c0 + k);
                    xq[k] = qkv[t * cd + cqk];
                    xv[k] = qkv[t * cd + cvg];
                    zc[k] = z[t * vd + kh * REP * DV + tid];
                }
            }
            if (gk < n) {
                ag = a[(size_t)(t0 + c0 + gk) * hv + gh];
                bg = b[(size_t)(t0 + c0 + gk) * hv + gh];
            }
        }
        // ---- A: token-parallel pieces
        #pragma unroll
        for (int k = 0; k < KTT; k++) {
            if (k < n) {
                const uint16_t cq = conv_tap4(wq, bf2f(w0), bf2f(w1), bf2f(w2), bf2f(xq[k]));
                const uint16_t cvv = conv_tap4(wvv, bf2f(u0), bf2f(u1), bf2f(u2), bf2f(xv[k]));
                w0 = w1; w1 = w2; w2 = xq[k];
                u0 = u1; u1 = u2; u2 = xv[k];   // (16-bit codes held in 32-bit registers)
                raw[k][tid] = bf2f(cq);
                cvs[k][tid] = bf2f(cvv);
                const float zf = bf2f(zc[k]);
                zgs[k][tid] = zf * sigmoid_cr(zf);     // silu(z), fp32
            }
        }
        __syncthreads();
        if (wv_ == 0 && lane < 2 * n) {                // l2-norm sums, one per lane
            const int k = lane >> 1, qk = lane & 1;
            rsq[k][qk] = 1.0f / sqrtf(sumsq128(&raw[k][qk * DK]) + kEps);
        } else if (wv_ == 1 && lane < 2 * n) {         // gates, one pair per lane
            const float g = decay_of((uint16_t)ag, __uint_as_float(alog_b), __uint_as_float(dtb_b));
            gt[gk][grr] = make_float2(exp_cr(g), rndf(sigmoid_cr(bf2f((uint16_t)bg))));
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < KTT; k++)
            if (k < n)
                raw[k][tid] = tid < DK ? (raw[k][tid] * rsq[k][0]) * qscale
                                       : raw[k][tid] * rsq[k][1];
        __syncthreads();
        if (!kEarlyTile && c0 == 0) load_tile();
        // ---- B: the recurrence on this wave's columns
        recur_chunk(sr, raw, gt, cvs, ob, n, r, j, tid,
                    tr_ob ? tr_ob + (size_t)(t0 + c0) * vd + h * DV + j : nullptr, vd);
        if (c0 + KTT >= cend) {
            // the last chunk: the tile is final; storing it here frees its
            // registers for phase C
            const int tox = __builtin_amdgcn_readfirstlane(so * hv + h);
            const auto Sw = buf_rsrc(S_out + (size_t)tox * DK * DV, DK * DV * 4);
#pragma unroll
            for (int q = 0; q < DK / 4; q++)
                buf_st4(Sw, voff, q * 1024,
                        f32x4_t{sr[4 * q + 0], sr[4 * q + 1], sr[4 * q + 2], sr[4 * q + 3]});
        }

        // ---- C: output norms, then y
        __syncthreads();
        if (wv_ == 2 && lane < 2 * n) {
            const int k = lane >> 1, rr = lane & 1;
            rso[k][rr] = 1.0f / sqrtf(sumsq128(&ob[k][rr][0]) / (float)DV + kEps);
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < KTT; k++) {
            if (k < n) {
                const float x1 = rndf(ob[k][r][j] * rso[k][r]);
                const float x2 = rndf(x1 * wo);
                y[(size_t)(t0 + c0 + k) * vd + h * DV + j] = f2bf(x2 * zgs[k][tid]);
            }
        }
    }
    uint16_t *otq = conv_out + (size_t)so * cd * 3 + (size_t)cqk * 3;
    uint16_t *otv = conv_out + (size_t)so * cd * 3 + (size_t)cvg * 3;
    otq[0] = w0; otq[1] = w1; otq[2] = w2;
    otv[0] = u0; otv[1] = u1; otv[2] = u2;
}

// ---- token-parallel pieces for the chunked prefill ------------------------
constexpr int PT = 16;       // tokens per k_gdn_prep tile
constexpr int PR = 64;       // (token, v-head) rows per k_gdn_post tile
constexpr int RS = DK + 4;   // LDS row stride: 16-byte aligned rows on distinct banks
constexpr int PC = 4 * DK;   // pre-conv channels of one K head: q, k, 2 x v

// Ascending sum of squares of one 128-float LDS row, one rounding per mul
// and add, with 16-byte reads kept in flight ahead of the add chain (over a
// row of 128 bf16 codes: gdn_dev.h). The row holds bf16 values, so the
// fused form is exact as there.
__device__ __forceinline__ float row_sumsq(const float *row) {
    const float4 *x4 = reinterpret_cast<const float4 *>(row);
    float ss = 0.0f;
#pragma unroll 8
    for (int j = 0; j < DK / 4; j++) {
        const float4 v = x4[j];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    return ss;
}

constexpr int RSC = DV + 8;  // LDS row stride in bf16 codes: 16-byte aligned rows

// k_gdn_prep: per (tile of 16 tokens, K head), 256 threads. The tile's
// pre-conv inputs of the head (q, k and its two v-heads' channels) plus
// three halo tokens are staged in LDS with 16-byte loads; thread c then
// owns one q/k channel and one v channel and walks the tokens (a
// sequence's first three tokens take their window from the old conv
// state). The q/k codes go out as they are, and one lane per (token, q|k)
// takes the ordered sum of squares for the l2norm (c/gdn.h:402-416) and
// writes the row's factor 1/sqrt(ss + eps) (the normalised row is code x
// factor, rounded once, as the chunk kernels form it); 32 lanes evaluate
// the (exp(g), beta) gates of the two v-heads, optionally with the raw g.
__global__ __launch_bounds__(256) void k_gdn_prep(
    GdnCu ci, const int32_t *__restrict__ dcu, int B, int Ttot, const uint16_t *__restrict__ qkv,
    const uint16_t *__restrict__ a, const uint16_t *__restrict__ b,
    const uint16_t *__restrict__ conv_w, const float *__restrict__ A_log,
    const float *__restrict__ dt_bias, const uint16_t *__restrict__ conv_state,
    uint16_t *__restrict__ qk, float *__restrict__ qkr, uint16_t *__restrict__ vconv,
    float2 *__restrict__ gate, float *__restrict__ graw, int hk,
    const uint16_t *__restrict__ silu_bf, const uint16_t *__restrict__ sig_bf,
    const int32_t *__restrict__ slots, uint16_t *__restrict__ tr_conv,
    uint16_t *__restrict__ tr_beta) {
    typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
    const int32_t *cu = dcu ? dcu : ci.cu;
    const int tile = blockIdx.x / hk, kh = blockIdx.x % hk;
    const int tb = tile * PT, nt = min(PT, Ttot - tb);
    const int tid = threadIdx.x;
    const int hv = hk * REP;
    const size_t kd = (size_t)hk * DK, vd = (size_t)hv * DV, cd = 2 * kd + vd;
    // The staged inputs, then (once every conv tap has been read) the conv
    // outputs of q and k for the ordered sums: q rows at 0, k rows at PT*RS
    // (rows 16-byte aligned). Sharing the space keeps 8 blocks per CU.
    constexpr int XIN_B = (PT + 3) * PC * 2, RAW_B = 2 * PT * RS * 4;
    __shared__ __attribute__((aligned(16))) char prep_lds[XIN_B > RAW_B ? XIN_B : RAW_B];
    uint16_t *xin = reinterpret_cast<uint16_t *>(prep_lds);
    float *raw = reinterpret_cast<float *>(prep_lds);
    __shared__ int2 tseq[PT];                 // (sequence, its first token) per tile token

    // stage rows tb-3 .. tb+nt-1 (those that exist); LDS channel order
    // [q(128) | k(128) | v(256)]. Every load of the tile is issued before
    // the first LDS store (a store right after its load would wait for it).
    constexpr int NPC = ((PT + 3) * PC / 8 + 255) / 256;
    u16x8 pc[NPC];
#pragma unroll
    for (int k = 0; k < NPC; k++) {
        const int e = tid + 256 * k, r = e / (PC / 8), c8 = (e % (PC / 8)) * 8;
        const int t = tb - 3 + r;
        if (e < (PT + 3) * PC / 8 && t >= 0 && r < nt + 3) {
            const size_t gc = c8 < DK ? (size_t)kh * DK + c8
                            : c8 < 2 * DK ? kd + (size_t)kh * DK + (c8 - DK)
                                          : 2 * kd + (size_t)kh * 2 * DV + (c8 - 2 * DK);
            pc[k] = *reinterpret_cast<const u16x8 *>(qkv + (size_t)t * cd + gc);
        }
    }
#pragma unroll
    for (int k = 0; k < NPC; k++) {
        const int e = tid + 256 * k, r = e / (PC / 8), c8 = (e % (PC / 8)) * 8;
        const int t = tb - 3 + r;
        if (e < (PT + 3) * PC / 8 && t >= 0 && r < nt + 3)
            *reinterpret_cast<u16x8 *>(xin + r * PC + c8) = pc[k];
    }
    if (tid < nt) {
        const int sq = seq_of(cu, B, tb + tid);
        tseq[tid] = make_int2(sq, cu[sq]);
    }
    const size_t cqk = tid < DK ? (size_t)kh * DK + tid : kd + (size_t)kh * DK + (tid - DK);
    const int h = kh * REP + tid / DV, j = tid % DV;
    const size_t cv = 2 * kd + (size_t)h * DV + j;
    float wq[4], wv[4];
    for (int i = 0; i < 4; i++) {
        wq[i] = bf2f(conv_w[cqk * 4 + i]);
        wv[i] = bf2f(conv_w[cv * 4 + i]);
    }
    __syncthreads();

    float *rrow = raw + (tid < DK ? 0 : PT * RS) + (tid & (DK - 1));
    // The tile's conv sums (bf16 codes) first, then SiLU, then the stores.
    // Tokens past the tile's end use code 0.
    uint16_t sq[PT], sv[PT];
    const int2 ts0 = tseq[0], tsl = tseq[nt - 1];
    if (ts0.y <= tb - 3 && ts0.x == tsl.x) {
        // (tile-uniform) one sequence, its 3 preceding tokens staged too:
        // every tap comes from the staged rows, read once, all in flight
        // (rows past the tile's tokens give unused codes)
        float xq[PT + 3], xv[PT + 3];
#pragma unroll
        for (int r = 0; r < PT + 3; r++) {
            xq[r] = bf2f(xin[r * PC + tid]);
            xv[r] = bf2f(xin[r * PC + 2 * DK + tid]);
        }
#pragma unroll
        for (int i = 0; i < PT; i++) {
            sq[i] = conv_sum4_code(wq, xq[i], xq[i + 1], xq[i + 2], xq[i + 3]);
            sv[i] = conv_sum4_code(wv, xv[i], xv[i + 1], xv[i + 2], xv[i + 3]);
        }
    } else {
#pragma unroll
    for (int i = 0; i < PT; i++) {
        sq[i] = sv[i] = 0;
        if (i < nt) {
            const int2 ts = tseq[i];
            const int t = tb + i, t0 = ts.y;
            const uint16_t *cst = conv_state + (size_t)(slots ? slots[ts.x] : ts.x) * cd * 3;
            float xq[4], xv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int ti = t - 3 + u;
                if (ti >= t0) {
                    xq[u] = bf2f(xin[(i + u) * PC + tid]);
                    xv[u] = bf2f(xin[(i + u) * PC + 2 * DK + tid]);
                } else {
                    xq[u] = bf2f(cst[cqk * 3 + (ti - t0 + 3)]);
                    xv[u] = bf2f(cst[cv * 3 + (ti - t0 + 3)]);
                }
            }
            sq[i] = conv_sum4_code(wq, xq[0], xq[1], xq[2], xq[3]);
            sv[i] = conv_sum4_code(wv, xv[0], xv[1], xv[2], xv[3]);
        }
    }
    }
    // SiLU through the fp32 fast path; the few results it cannot vouch for
    // come from the bf16-code table (gathers with few lanes active), all
    // issued before the first use (code 0 past the tile's tokens)
    uint32_t redo = 0;
#pragma unroll
    for (int i = 0; i < PT; i++) {
        bool okq, okv;
        const uint16_t rq = silu_fast(bf2f(sq[i]), okq), rv = silu_fast(bf2f(sv[i]), okv);
        redo |= (okq ? 0u : 1u << i) | (okv ? 0u : 1u << (PT + i));
        if (okq) sq[i] = rq;
        if (okv) sv[i] = rv;
    }
    if (redo) {
#pragma unroll
        for (int i = 0; i < PT; i++) {
            if (redo >> i & 1u) sq[i] = silu_bf[sq[i]];
            if (redo >> (PT + i) & 1u) sv[i] = silu_bf[sv[i]];
        }
    }
    __syncthreads();                          // every tap read: raw may overwrite xin
#pragma unroll
    for (int i = 0; i < PT; i++) {
        if (i < nt) {
            rrow[i * RS] = bf2f(sq[i]);
            qk[(size_t)(tb + i) * 2 * kd + cqk] = sq[i];
            vconv[(size_t)(tb + i) * vd + (size_t)h * DV + j] = sv[i];
            if (tr_conv) {                    // (trace) conv+SiLU codes, c/layer.h:178
                tr_conv[(size_t)(tb + i) * cd + cqk] = sq[i];
                tr_conv[(size_t)(tb + i) * cd + cv] = sv[i];
            }
        }
    }
    __syncthreads();
    if (tid < 2 * PT) {                      // ordered sums, one lane per row
        const int r = tid & (PT - 1), w = tid / PT;
        if (r < nt)
            qkr[(size_t)(tb + r) * 2 * hk + w * hk + kh] =
                1.0f / sqrtf(row_sumsq(raw + w * PT * RS + r * RS) + kEps);
    } else if (tid >= 64 && tid < 64 + REP * PT) {   // gates of the two v-heads
        const int r = (tid - 64) & (PT - 1), hh = kh * REP + (tid - 64) / PT;
        if (r < nt) {
            const size_t t = (size_t)(tb + r);
            const float g = decay_of(a[t * hv + hh], A_log[hh], dt_bias[hh]);
            const uint16_t btc = sig_bf[b[t * hv + hh]];
            const float bt = bf2f(btc);
            gate[t * hv + hh] = make_float2(exp_cr(g), bt);
            if (graw) graw[t * hv + hh] = g;
            if (tr_beta) tr_beta[t * hv + hh] = btc;
        }
    }
}

// k_gdn_post: blocks [0, ceil(Ttot*hv/64)) apply the gated RMSNorm
// (c/gdn.h:639-661) to 64 consecutive (token, v-head) rows of ob: 16-byte
// loads, the rows parked in LDS as codes (17 KiB a block, 8 blocks per CU
// to hide the serial sums), one lane per row for the ordered sum of
// squares, then elementwise from the registers with 16-byte z loads and
// y stores. The rows, z and y are each touched once: streaming
// (non-temporal) loads and stores keep them from displacing the next
// kernels' operands in L2 (T=4096 layer step 0.217 -> 0.212 ms). The
// remaining blocks
// write each sequence's new conv state (the last three pre-conv inputs of
// [old state | tokens]) after every reader of the old one has finished.
__global__ __launch_bounds__(256) void k_gdn_post(
    GdnCu ci, const int32_t *__restrict__ dcu, int B, int Ttot,
    const uint16_t *__restrict__ ob, const uint16_t *__restrict__ z,
    const uint16_t *__restrict__ onorm_w, uint16_t *__restrict__ y,
    const uint16_t *__restrict__ qkv, uint16_t *__restrict__ conv_state,
    int hk, const float *__restrict__ silu_f, const int32_t *__restrict__ slots) {
    const int32_t *cu = dcu ? dcu : ci.cu;
    const int hv = hk * REP;
    const size_t kd = (size_t)hk * DK, vd = (size_t)hv * DV, cd = 2 * kd + vd;
    const int tid = threadIdx.x;
    const size_t nrows = (size_t)Ttot * hv;
    const size_t nnorm = (nrows + PR - 1) / PR;
    typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
    if ((size_t)blockIdx.x < nnorm) {
        const size_t r0 = (size_t)blockIdx.x * PR;
        const int nr = (int)min((size_t)PR, nrows - r0);
        __shared__ __attribute__((aligned(16))) uint16_t os[PR * RSC];
        __shared__ float rs[PR];
        // every load of the block (the rows and their z) in flight at once
        constexpr int NPC = PR * DV / 8 / 256;
        u16x8 ov[NPC], zv8[NPC];
#pragma unroll
        for (int k = 0; k < NPC; k++) {
            const int e = tid + 256 * k, row = e / (DV / 8), c8 = (e % (DV / 8)) * 8;
            if (row < nr) {
                ov[k] = __builtin_nontemporal_load(reinterpret_cast<const u16x8 *>(ob + (r0 + row) * DV + c8));
                zv8[k] = __builtin_nontemporal_load(reinterpret_cast<const u16x8 *>(z + (r0 + row) * DV + c8));
            }
        }
#pragma unroll
        for (int k = 0; k < NPC; k++) {
            const int e = tid + 256 * k, row = e / (DV / 8), c8 = (e % (DV / 8)) * 8;
            if (row < nr) *reinterpret_cast<u16x8 *>(os + row * RSC + c8) = ov[k];
        }
        __syncthreads();
        if (tid < nr) {
            rs[tid] = 1.0f / sqrtf(apus::row_sumsq(os + tid * RSC) / (float)DV + kEps);
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < NPC; k++) {
            const int e = tid + 256 * k, row = e / (DV / 8), c8 = (e % (DV / 8)) * 8;
            if (row < nr) {
                const size_t off = (r0 + row) * DV + c8;
                const u16x8 zv = zv8[k];
                const u16x8 wv = *reinterpret_cast<const u16x8 *>(onorm_w + c8);
                u16x8 out;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float x1 = rndf(bf2f(ov[k][i]) * rs[row]);
                    const float x2 = rndf(x1 * bf2f(wv[i]));
                    out[i] = f2bf(x2 * silu_f[zv[i]]);     // silu(z), fp32
                }
                __builtin_nontemporal_store(out, reinterpret_cast<u16x8 *>(y + off));
            }
        }
        return;
    }
    const size_t bb = blockIdx.x - nnorm;
    const size_t per = cd / 256;
    const size_t s = bb / per, c = (bb % per) * 256 + tid;
    const int t0 = cu[s], n = cu[s + 1] - t0;
    if (n == 0) return;
    uint16_t *st = conv_state + (size_t)(slots ? slots[s] : (int32_t)s) * cd * 3 + c * 3;
    uint16_t w3[3];
    for (int jj = 0; jj < 3; jj++) {
        int idx = n - 3 + jj;          // position in the token span
        w3[jj] = idx >= 0 ? qkv[(size_t)(t0 + idx) * cd + c] : st[idx + 3];
    }
    st[0] = w3[0];
    st[1] = w3[1];
    st[2] = w3[2];
}

}  // namespace

namespace apus {

int gdn_check_layer(const ApusHipGdnLayer *L) {
    if (!L) return set_error(kErrArgument, "NULL layer");
    if (L->dk != DK || L->dv != DV || L->hv != REP * L->hk || L->hk == 0)
        return set_error(kErrUnsupported,
                         "GDN mixer supports dk=dv=128, hv=2*hk (got hk=%zu hv=%zu "
                         "dk=%zu dv=%zu)", L->hk, L->hv, L->dk, L->dv);
    return kOk;
}

int gdn_check_offsets(size_t B, const int32_t *cu) {
    if (!cu || cu[0] != 0) return set_error(kErrArgument, "cu must start at 0");
    for (size_t s = 0; s < B; s++)
        if (cu[s + 1] < cu[s])
            return set_error(kErrArgument, "token offsets must ascend");
    return kOk;
}

// the offsets by value when they fit, else the device copy
static bool gdn_cu_arg(size_t B, const int32_t *cu, const int32_t *dcu, GdnCu *ci) {
    if (dcu) return true;
    if (B > (size_t)kGdnCuInline || !cu) return false;
    memcpy(ci->cu, cu, (B + 1) * 4);
    return true;
}

int gdn_prep(const ApusHipGdnLayer *L, size_t B, const int32_t *cu, const int32_t *dcu,
             size_t Ttot, const uint16_t *qkv, const uint16_t *a,
             const uint16_t *b, const uint16_t *conv_state, GdnScratch *w,
             bool want_graw, const int32_t *slots, const ApusHipGdnTrace *tr) {
    const size_t kd = L->hk * DK, vd = L->hv * DV;
    if (!w->qk) {                              // else the caller's workspace
        w->qk = (uint16_t *)scratch(kScratchGdnQK, Ttot * 2 * kd * 2);
        w->qkr = (float *)scratch(kScratchGdnQKR, Ttot * 2 * L->hk * 4);
        w->vconv = (uint16_t *)scratch(kScratchGdnV, Ttot * vd * 2);
        w->gate = (float2 *)scratch(kScratchGdnGate, Ttot * L->hv * 8);
        w->ob = (uint16_t *)scratch(kScratchGdnOB, Ttot * vd * 2);
        w->graw = want_graw ? (float *)scratch(kScratchGdnChunk3, Ttot * L->hv * 4) : nullptr;
    }
    if (!w->qk || !w->qkr || !w->vconv || !w->gate || !w->ob || (want_graw && !w->graw))
        return kErrHip;
    // a traced call without the raw gates for WY writes them straight to
    // the trace
    float *graw = w->graw ? w->graw : (tr ? tr->gdecay : nullptr);
    const ActTables *tabs = act_tables();
    if (!tabs) return kErrHip;
    GdnCu ci;
    if (!gdn_cu_arg(B, cu, dcu, &ci)) return set_error(kErrArgument, "no token offsets");
    APUS_TIMED("k_gdn_prep",
               k_gdn_prep<<<(unsigned)(cdiv(Ttot, PT) * L->hk), 256, 0, stream()>>>(
        ci, dcu, (int)B, (int)Ttot, qkv, a, b, L->conv_w, L->A_log, L->dt_bias, conv_state,
        w->qk, w->qkr, w->vconv, w->gate, graw, (int)L->hk, tabs->silu_bf, tabs->sig_bf,
        slots, tr ? tr->qkv_conv : nullptr, tr ? tr->beta : nullptr));
    return launch_check("k_gdn_prep");
}

int gdn_post(const ApusHipGdnLayer *L, size_t B, const int32_t *cu, const int32_t *dcu,
             size_t Ttot, const GdnScratch *w, const uint16_t *z,
             const uint16_t *qkv, uint16_t *conv_state, uint16_t *y, const int32_t *slots) {
    const size_t cd = 2 * L->hk * DK + L->hv * DV;
    const size_t nblk = cdiv(Ttot * L->hv, PR) + B * (cd / 256);
    const ActTables *tabs = act_tables();
    if (!tabs) return kErrHip;
    GdnCu ci;
    if (!gdn_cu_arg(B, cu, dcu, &ci)) return set_error(kErrArgument, "no token offsets");
    APUS_TIMED("k_gdn_post",
               k_gdn_post<<<(unsigned)nblk, 256, 0, stream()>>>(
        ci, dcu, (int)B, (int)Ttot, w->ob, z, L->onorm_w, y, qkv, conv_state,
        (int)L->hk, tabs->silu_f, slots));
    return launch_check("k_gdn_post");
}

}  // namespace apus

extern "C" {

}  // extern "C"

namespace apus {

// Decode / verify with optional state slot maps (host arrays; nullptr:
// sequence s uses slot s).
static int gdn_decode_run(const ApusHipGdnLayer *L, size_t B, const int32_t *cu,
                          const uint16_t *qkv, const uint16_t *z, const uint16_t *a,
                          const uint16_t *b, const uint16_t *conv_in, const float *S_in,
                          uint16_t *conv_out, float *S_out, uint16_t *y, const int32_t *sin_h,
                          const int32_t *sout_h) {
    if (int r = gdn_check_layer(L)) return r;
    if (B == 0) return kOk;
    if (int r = gdn_check_offsets(B, cu)) return r;
    if (cu[B] == 0) return kOk;
    CuArgs ca;
    const int32_t *dcu = nullptr;
    if (B <= (size_t)kInlineSeqs) {
        memcpy(ca.cu, cu, (B + 1) * sizeof(int32_t));
    } else {
        dcu = (const int32_t *)upload_async(cu, (B + 1) * 4);
        if (!dcu) return kErrHip;
    }
    const ApusHipGdnTrace *tr = gdn_trace();
    const bool traced = tr && (tr->qkv_conv || tr->beta || tr->gdecay);
    const int32_t *dsin = nullptr, *dsout = nullptr;
    const bool slots_inline = sin_h && !dcu && 3 * B + 1 <= (size_t)kInlineWords;
    if (slots_inline) {
        memcpy(ca.cu + B + 1, sin_h, B * 4);
        memcpy(ca.cu + 2 * B + 1, sout_h, B * 4);
    }
    if (sin_h && (!slots_inline || traced)) {     // the trace's prep pass reads them on device
        std::vector<int32_t> m(2 * B);
        memcpy(m.data(), sin_h, B * 4);
        memcpy(m.data() + B, sout_h, B * 4);
        dsin = (const int32_t *)upload_async(m.data(), m.size() * 4);
        if (!dsin) return kErrHip;
        dsout = dsin + B;
    }
    if (traced) {
        // the token-parallel intermediates from the same inputs and the
        // old conv state, before the decode rewrites it
        const int32_t *pcu = dcu;
        if (!pcu && B > (size_t)kGdnCuInline) {
            pcu = (const int32_t *)upload_async(cu, (B + 1) * 4);
            if (!pcu) return kErrHip;
        }
        GdnScratch w{};
        if (int r = gdn_prep(L, B, cu, pcu, (size_t)cu[B], qkv, a, b, conv_in, &w, false, dsin, tr))
            return r;
    }
    const float qscale = (float)pow((double)L->dk, -0.5);
    int max_tok = 0;                           // the most tokens of one sequence
    for (size_t s = 0; s < B; s++) max_tok = std::max(max_tok, cu[s + 1] - cu[s]);
    auto launch = [&](auto args) {
        constexpr int NW = sizeof(args.cu) / sizeof(int32_t);
        auto kern = max_tok <= 1 ? k_gdn_decode<0, NW>
                                 : max_tok <= KT ? k_gdn_decode<1, NW> : k_gdn_decode<2, NW>;
        APUS_TIMED("k_gdn_decode",
                   kern<<<(unsigned)(B * L->hk), 256, 0, stream()>>>(
            args, dcu, (int)B, qkv, z, a, b, L->conv_w, L->A_log, L->dt_bias, L->onorm_w,
            conv_in, S_in, conv_out, S_out, y, (int)L->hk, qscale, dsin, dsout,
            (int)slots_inline, tr ? tr->rec_o : nullptr));
    };
    // the words the kernel reads: cu[0..B], then the inline slot maps
    const size_t used = dcu ? 0 : (slots_inline ? 3 * B + 1 : B + 1);
    if (used <= (size_t)kSmallWords) {
        CuArgsN<kSmallWords> sa;
        memcpy(sa.cu, ca.cu, sizeof(sa.cu));
        launch(sa);
    } else {
        launch(ca);
    }
    APUS_LAUNCHED("k_gdn_decode");
    if (tr && tr->onorm)                       // the gated norm's output is y
        APUS_HIP_TRY(hipMemcpyAsync(tr->onorm, y, (size_t)cu[B] * L->hv * DV * 2,
                                    hipMemcpyDeviceToDevice, stream()));
    return kOk;
}

// Slot maps must not let one sequence's writes land in another's reads or
// writes: the output slots of the sequences with tokens are distinct, and
// none is another sequence's input slot.
static int check_slot_maps(size_t B, const int32_t *cu, const int32_t *sin, const int32_t *sout,
                           size_t nslots) {
    std::vector<std::pair<int32_t, int32_t>> outs, ins;
    for (size_t s = 0; s < B; s++) {
        if (sin[s] < 0 || sout[s] < 0 || (nslots && ((size_t)sin[s] >= nslots ||
                                                      (size_t)sout[s] >= nslots)))
            return set_error(kErrArgument, "state slot of sequence %zu out of range", s);
        if (cu[s + 1] == cu[s]) continue;
        outs.emplace_back(sout[s], (int32_t)s);
        ins.emplace_back(sin[s], (int32_t)s);
    }
    std::sort(outs.begin(), outs.end());
    std::sort(ins.begin(), ins.end());
    for (size_t i = 1; i < outs.size(); i++)
        if (outs[i].first == outs[i - 1].first)
            return set_error(kErrArgument, "two sequences write state slot %d", outs[i].first);
    for (auto &o : outs) {
        auto it = std::lower_bound(ins.begin(), ins.end(), std::make_pair(o.first, INT32_MIN));
        for (; it != ins.end() && it->first == o.first; ++it)
            if (it->second != o.second)
                return set_error(kErrArgument,
                                 "state slot %d is written by sequence %d and read by %d",
                                 o.first, o.second, it->second);
    }
    return kOk;
}

}  // namespace apus

extern "C" {

int apus_hip_gdn_decode_into(const ApusHipGdnLayer *L, size_t B, const int32_t *cu,
                             const uint16_t *qkv, const uint16_t *z,
                             const uint16_t *a, const uint16_t *b,
                             const uint16_t *conv_in, const float *S_in,
                             uint16_t *conv_out, float *S_out, uint16_t *y) {
    APUS_READY();
    if (!L) return set_error(kErrArgument, "NULL layer");
    // in place, or two disjoint state sets: a partial overlap would let one
    // workgroup's writes land in another's inputs
    const size_t nS = B * L->hv * DK * DV * 4, nC = B * (2 * L->hk * DK + L->hv * DV) * 3 * 2;
    auto overlap = [](const void *p, const void *q, size_t n) {
        const char *x = (const char *)p, *w = (const char *)q;
        return x != w && x < w + n && w < x + n;
    };
    if (overlap(S_in, S_out, nS) || overlap(conv_in, conv_out, nC))
        return set_error(kErrArgument, "state in/out must be the same buffer or disjoint");
    return gdn_decode_run(L, B, cu, qkv, z, a, b, conv_in, S_in, conv_out, S_out, y, nullptr,
                          nullptr);
}

int apus_hip_gdn_decode(const ApusHipGdnLayer *L, size_t B, const int32_t *cu,
                        const uint16_t *qkv, const uint16_t *z,
                        const uint16_t *a, const uint16_t *b,
                        uint16_t *conv_state, float *S, uint16_t *y) {
    return apus_hip_gdn_decode_into(L, B, cu, qkv, z, a, b, conv_state, S,
                                    conv_state, S, y);
}

int apus_hip_gdn_decode_slots(const ApusHipGdnLayer *L, size_t B, const int32_t *slot_in,
                              const int32_t *slot_out, const int32_t *cu, const uint16_t *qkv,
                              const uint16_t *z, const uint16_t *a, const uint16_t *b,
                              uint16_t *conv, float *S, uint16_t *y) {
    APUS_READY();
    if (B == 0) return kOk;
    if (!slot_in || !slot_out) return set_error(kErrArgument, "NULL slot map");
    if (int r = gdn_check_offsets(B, cu)) return r;
    if (int r = check_slot_maps(B, cu, slot_in, slot_out, 0)) return r;
    return gdn_decode_run(L, B, cu, qkv, z, a, b, conv, S, conv, S, y, slot_in, slot_out);
}

int apus_hip_gdn_state_pack(const float *S_ref, float *S_dev, size_t nmat) {
    APUS_READY();
    if (nmat == 0) return kOk;
    k_gdn_pack<<<cdiv(nmat * DK * DV, 256), 256, 0, stream()>>>(S_ref, S_dev, nmat);
    APUS_LAUNCHED("k_gdn_pack");
    return kOk;
}

int apus_hip_gdn_state_unpack(const float *S_dev, float *S_ref, size_t nmat) {
    APUS_READY();
    if (nmat == 0) return kOk;
    k_gdn_unpack<<<cdiv(nmat * DK * DV, 256), 256, 0, stream()>>>(S_dev, S_ref, nmat);
    APUS_LAUNCHED("k_gdn_unpack");
    return kOk;
}

}  // extern "C"
