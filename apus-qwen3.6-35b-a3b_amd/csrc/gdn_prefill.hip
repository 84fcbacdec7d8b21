// gdn_prefill.hip -- chunked Gated DeltaNet prefill for gfx950: the op
// sequence of c/layer.h:427-492 (conv, l2norm, gates, delta-rule
// recurrence, gated RMSNorm for every prompt token) with the recurrence
// evaluated chunk-parallel instead of token by token.
//
// Recurrence (c/gdn.h:471-504), per v-head, a_t = exp(g_t):
//     S_t = a_t S_{t-1} + k_t d_t^T,   d_t = b_t (v_t - a_t S_{t-1}^T k_t),
//     o_t = S_t^T q_t.
// Over a chunk of C = 64 tokens with gamma_t = g_1 + .. + g_t (within the
// chunk) and G_t = exp(gamma_t), the deltas of the chunk satisfy the unit
// lower-triangular system (the WY / UT form)
//     (I + L) D = diag(b) V - diag(b G) K S0,
//     L[t][s] = b_t exp(gamma_t - gamma_s) (k_t . k_s)   (s < t),
// so D = U - W S0 with U = (I+L)^-1 diag(b) V and W = (I+L)^-1 diag(b G) K
// -- quantities of the chunk alone -- and
//     O  = diag(G) Q S0 + A D,   A[t][s] = exp(gamma_t - gamma_s)(q_t . k_s)
//                                (s <= t),
//     S1 = G_C S0 + K^T diag(exp(gamma_C - gamma_s)) D.
// Padding a chunk with tokens of g = 0, b = 0, k = q = 0 leaves S and the
// real rows unchanged, so ragged sequences need no special case.
//
// Kernels (before k_gdn_post of gdn_mixer.hip):
//   k_gdn_chunk_wy    one workgroup per (chunk, K head), all chunks in
//                     parallel: the q, k, v conv codes, gates and l2norm
//                     factors, K K^T and Q K^T once for the K head's two
//                     v-heads, then per v-head L and A with their decay
//                     factors and U and W as T [b V | b G K] with
//                     T = (I+L)^-1 built in 32x32 blocks.
//   k_gdn_chunk_scan  one workgroup per (sequence, v-head, 16-column block
//                     of S): the delta rule is separable by value column,
//                     so the chunk-to-chunk carry of S runs in 8 independent
//                     column slices per head, each walking its sequence's
//                     chunks in order (D, O, S1 above).
// The recurrent state must stay within 1e-4 of the sequential fp32
// recurrence, which bf16 operands (8-bit mantissa) cannot hold: products
// run on the bf16 MFMA with each fp32 operand split into bf16 parts (two
// parts, hi + lo, for 16 bits; three for Q K^T, which cancels and feeds the
// outputs directly) and fp32 accumulation. The chunk form sums in a
// different order from the reference's token loop -- a tolerance class,
// checked against the sequential oracle.
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
constexpr int C = 64;                  // chunk length (tokens)
constexpr int CB = 16;                 // S columns per scan workgroup
constexpr int NCB = DV / CB;
constexpr int KP = DK + 4;             // padded LDS row (floats)
constexpr int CP = C + 4;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Per-call sequence metadata by value (no upload for small batches).
constexpr int kPrefillInline = 400;
struct ChunkSeqs {
    int32_t n;
    int32_t cu[kPrefillInline + 1];    // token offsets
    int32_t coff[kPrefillInline + 1];  // chunk offsets
};

__device__ __forceinline__ int seq_of(const int32_t *off, int n, int x) {
    int lo = 0, hi = n - 1;            // largest s with off[s] <= x
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= x) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// 16 steps of the reduction dimension on the 16x16x4 fp32 MFMA. Lane l
// holds row l%16 of the A tile and column l%16 of the B tile at reduction
// indices k0 + 4*(l/16) + 0..3 (a 16-byte read each); step j feeds index
// 4*(l/16) + j, so A and B see the same permutation of k and the sum is
// the plain 16-term dot product per output element.

__device__ __forceinline__ float4 lds4(const float *p) {
    return *reinterpret_cast<const float4 *>(p);
}

__device__ __forceinline__ float4 ld4(const float *p) {
    return *reinterpret_cast<const float4 *>(p);
}

// Device copy of by-value metadata, written on the stream (no host sync).
__global__ void k_prefill_meta(ChunkSeqs sq, int32_t *__restrict__ dst) {
    for (int i = threadIdx.x; i <= sq.n; i += blockDim.x) {
        dst[i] = sq.cu[i];
        dst[sq.n + 1 + i] = sq.coff[i];
    }
}

struct ChunkPos {
    int s, t0, nt;
};

__device__ __forceinline__ ChunkPos chunk_pos(const int32_t *cu, const int32_t *coff, int n,
                                              int c) {
    ChunkPos p;
    p.s = seq_of(coff, n, c);
    p.t0 = cu[p.s] + (c - coff[p.s]) * C;
    p.nt = min(C, cu[p.s + 1] - p.t0);
    return p;
}

// Per (chunk, v-head) buffers written by k_gdn_chunk_wy, stored in the
// order k_gdn_chunk_scan's MFMA lanes consume them, so that every scan load
// instruction reads 1 KiB of contiguous memory. The scan multiplies on
// the 16x16x32 bf16 MFMA in split precision: every fp32 operand x is held
// as hi = rnd(x) and lo = rnd(x - hi) (bf16), and a product is
// hi.hi + hi.lo + lo.hi with fp32 accumulation (about 2^-16 relative per
// product; the dropped lo.lo term is below 2^-17). Matrix operands are
// stored per 16 rows x 32 reduction columns: lane g*16 + r of block
// (row block, 32-column block) holds row r, columns 8g..8g+7 as 8 hi then
// 8 lo codes (32 bytes).
//   W  [4 row blocks][4 column blocks][64 lanes][16] (rows t, columns c);
//   A  [4 row blocks][2 column blocks][64][16] (rows t, columns s; zero for
//      s > t inside the blocks the scan reads);
//   U  fp32 [8 column slices][4 row blocks][64][4]: element (t, j) at lane
//      (j%16) + 16*((t%16)/4) of (j/16, t/16), slot t%4 -- the
//      accumulator layout of the scan's D tile;
//   F  fp32 [3][C]: F[0][t] = G_t rq_t qscale (the scale of row t of
//      Q S0, Q as codes), F[1][s] = exp(gamma_C - gamma_s) rk_s (the scale
//      of key s in the state update, K as codes), F[2][0] = G_C.
__device__ __forceinline__ size_t bx_a_index(int t, int c, int nkb) {
    return ((size_t)((t >> 4) * nkb + (c >> 5)) * 64 + ((c & 31) >> 3) * 16 + (t & 15)) * 16 + (c & 7);
}
__device__ __forceinline__ size_t wy_u_index(int t, int j) {
    return ((size_t)((j >> 4) * 4 + (t >> 4)) * 64 + ((t & 15) >> 2) * 16 + (j & 15)) * 4 + (t & 3);
}

// Per (chunk, K head), written by the v-head of even index (both v-heads
// of a K head hold the same q and k), q and k travel to the scan as the
// conv codes themselves (exact in bf16, so one MFMA per product against a
// split operand's two parts), as code planes in the same lane order, 1 KiB
// blocks of 64 lanes x 8 codes:
//   Q  [4 row blocks][4 column blocks][64][8], W's lane order (the A
//      operand of Q S0);
//   K  [8 state-row blocks][2 key blocks][64][8], a B operand: lane
//      g*16 + i%16 holds key rows s = 8g..8g+7 of state row i.
__device__ __forceinline__ size_t bx1_a_index(int t, int c, int nkb) {
    return ((size_t)((t >> 4) * nkb + (c >> 5)) * 64 + ((c & 31) >> 3) * 16 + (t & 15)) * 8 + (c & 7);
}
__device__ __forceinline__ size_t bx1_b_index(int s, int i) {
    return ((size_t)((i >> 4) * 2 + (s >> 5)) * 64 + ((s & 31) >> 3) * 16 + (i & 15)) * 8 + (s & 7);
}

// hi = rnd(x), lo = rnd(x - hi), as bf16 codes (hardware round to nearest
// even)
__device__ __forceinline__ void split_bf(float x, uint16_t &hi, uint16_t &lo) {
    const __bf16 h = (__bf16)x;
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (__bf16)(x - (float)h));
}
// the 8 hi codes then the 8 lo codes of x[0..7]: one 32-byte unit of the
// packed operand layouts, written with two 16-byte stores
__device__ __forceinline__ void put_split8(uint16_t *p, const float (&x)[8]) {
    typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));
    u16x8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint16_t h, l;
        split_bf(x[i], h, l);
        hi[i] = h;
        lo[i] = l;
    }
    *reinterpret_cast<u16x8_t *>(p) = hi;
    *reinterpret_cast<u16x8_t *>(p + 8) = lo;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf(u16x8 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ u16x8 ld8(const uint16_t *p) {
    return *reinterpret_cast<const u16x8 *>(p);
}
// acc += a.b in split precision: (ah, al) and (bh, bl) the hi/lo operands
__device__ __forceinline__ f32x4 mfma_x3(u16x8 ah, u16x8 al, u16x8 bh, u16x8 bl, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(al), as_bf(bh), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah), as_bf(bl), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah), as_bf(bh), c, 0, 0, 0);
    return c;
}

// acc += c.x with c exact bf16 codes and x = xh + xl split: c.xl then
// c.xh. code_is_b: the codes are the B operand (x the A operand).
__device__ __forceinline__ f32x4 mfma_x2a(u16x8 c, u16x8 xh, u16x8 xl, f32x4 acc, bool code_is_b) {
    if (code_is_b) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(xl), as_bf(c), acc, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(xh), as_bf(c), acc, 0, 0, 0);
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(c), as_bf(xl), acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(c), as_bf(xh), acc, 0, 0, 0);
}

// hi/lo bf16 codes of 8 fp32 values: one split-precision MFMA operand
__device__ __forceinline__ void split8(const float (&x)[8], u16x8 &hi, u16x8 &lo) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint16_t h, l;
        split_bf(x[i], h, l);
        hi[i] = h;
        lo[i] = l;
    }
}

// The normalised rows are q_t = rq_t qscale cq_t and k_s = rk_s ck_s with
// cq, ck the conv codes, so q.k and k.k are the factors times the exact
// dot products of the codes: one bf16 MFMA per product, fp32
// accumulation, no operand splitting. k_gdn_chunk_wy forms the codes of a
// (chunk, K head) and their products once; per (chunk, v-head) work runs on
// half of its wavefronts each.
constexpr int CKP = DK + 8;            // bf16 row stride of the code copies

// Two channels' 4-tap conv sums (tap order, one rounding per mul and add,
// c/gdn.h:19-33), rounded to bf16 codes by one hardware round-to-nearest-
// even conversion (v_cvt_pk_bf16_f32): the codes conv_sum4_code gives for
// finite sums.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t conv_sum4_pair(const float (&w0)[4], const float (&w1)[4],
                                                   uint32_t x0, uint32_t x1, uint32_t x2,
                                                   uint32_t x3) {
    auto lo = [](uint32_t v) { return __uint_as_float(v << 16); };
    auto hi = [](uint32_t v) { return __uint_as_float(v & 0xffff0000u); };
    float a = 0.0f, c = 0.0f;
    a = a + w0[0] * lo(x0);
    c = c + w1[0] * hi(x0);
    a = a + w0[1] * lo(x1);
    c = c + w1[1] * hi(x1);
    a = a + w0[2] * lo(x2);
    c = c + w1[2] * hi(x2);
    a = a + w0[3] * lo(x3);
    c = c + w1[3] * hi(x3);
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, c}, bf16x2_t));
}
constexpr int TG = 16;                         // tokens per conv work item

// The conv+SiLU codes of channels gcol and gcol + 1 (c/gdn.h:19-33,
// 220-228) for the 16 tokens tg .. tg+15 of chunk P, in two parts so that
// a thread's two items have their loads in flight together:
// conv_rows16 reads the item's tokens' inputs and the 3 before them (from
// the sequence's old conv state in its first chunk) and the two channels'
// taps; conv_codes16 forms the codes. Loads are unconditional (rows
// clamped into the chunk); the codes of padding rows (t >= nt) are 0.
struct ConvRows {
    uint32_t x[TG + 3];                         // inputs, two channels a word
    float w0[4], w1[4];                         // the two channels' taps
};
__device__ __forceinline__ void conv_rows16(const uint16_t *__restrict__ qkv, size_t cd,
                                            size_t gcol, const ChunkPos &P, int tg, bool first,
                                            const uint16_t *__restrict__ cst,
                                            const uint16_t *__restrict__ conv_w, ConvRows &R) {
    // (tg, P and first are wave-uniform: the row addresses are scalar)
    const uint32_t cofs = (uint32_t)gcol * 2;   // the lane's byte offset in a row
    const int t0 = __builtin_amdgcn_readfirstlane(P.t0), nt = __builtin_amdgcn_readfirstlane(P.nt);
#pragma unroll
    for (int r = 0; r < TG + 3; r++) {
        const int t = tg - 3 + r;               // chunk-relative token
        const int row = t0 + max(min(t, nt - 1), first ? 0 : -3);
        const char *rowp = reinterpret_cast<const char *>(qkv) + (size_t)row * cd * 2;
        const uint32_t vq = *reinterpret_cast<const uint32_t *>(rowp + cofs);
        if (r < 3 && tg == 0) {
            const uint32_t vs = (uint32_t)cst[gcol * 3 + r] | ((uint32_t)cst[(gcol + 1) * 3 + r] << 16);
            R.x[r] = first ? vs : vq;
        } else {
            R.x[r] = vq;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        R.w0[i] = bf2f(conv_w[gcol * 4 + i]);
        R.w1[i] = bf2f(conv_w[(gcol + 1) * 4 + i]);
    }
}
// conv sums, then the SiLU of each code from the bf16-code table
// (rnd(co sigmoid(co)) is a function of the code co; the table holds the
// reference's value for every code). Gathering it costs less than the fp32
// fast path with its exponential and reciprocal (config 1: WY 95 -> 90 us).
__device__ __forceinline__ void conv_codes16(const ConvRows &R, int tg, int nt,
                                             const uint16_t *__restrict__ silu_bf,
                                             uint16_t (&c0)[TG], uint16_t (&c1)[TG]) {
#pragma unroll
    for (int j = 0; j < TG; j++) {
        const uint32_t cc = conv_sum4_pair(R.w0, R.w1, R.x[j], R.x[j + 1], R.x[j + 2], R.x[j + 3]);
        c0[j] = silu_bf[cc & 0xffffu];
        c1[j] = silu_bf[cc >> 16];
    }
#pragma unroll
    for (int j = 0; j < TG; j++)
        if (tg + j >= nt) c0[j] = c1[j] = 0;
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void k_gdn_chunk_wy(
    ChunkSeqs sq, const int32_t *__restrict__ dmeta, const uint16_t *__restrict__ qkv,
    const uint16_t *__restrict__ a, const uint16_t *__restrict__ b,
    const uint16_t *__restrict__ conv_w, const float *__restrict__ A_log,
    const float *__restrict__ dt_bias, const uint16_t *__restrict__ conv_state,
    const int32_t *__restrict__ slots, const uint16_t *__restrict__ silu_bf,
    const uint16_t *__restrict__ sig_bf, float *__restrict__ Ub,
    uint16_t *__restrict__ Wb, uint16_t *__restrict__ Ab, float *__restrict__ Fb,
    uint16_t *__restrict__ Qp, uint16_t *__restrict__ Kp, int hk, float qscale) {
    const int hv = hk * REP;
    const size_t kd = (size_t)hk * DK, vd = (size_t)hv * DV, cd = 2 * kd + vd;
    const int ku = blockIdx.x, ci = ku / hk, kh = ku % hk;
    const int32_t *cu = dmeta ? dmeta : sq.cu;
    const int32_t *coff = dmeta ? dmeta + sq.n + 1 : sq.coff;
    const ChunkPos P = chunk_pos(cu, coff, sq.n, ci);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // wavefronts 4 grp .. 4 grp + 3 work on v-head 2 kh + grp (unit unitg)
    // once the q, k work is done
    const int grp = wave >> 2, gw = wave & 3, gtid = tid & 255;
    const int unitg = ci * hv + kh * REP + grp;

    // LDS (two workgroups per CU): the q and k codes (rows t, CKP pitch),
    // then the V codes of each v-head transposed ([column][token]: the B
    // operand of T R; the 16-byte pieces of row n XOR-swizzled by n % 8, so
    // the MFMA operand reads spread over the banks). L of each v-head
    // replaces the codes once the products are formed; W's staging of each
    // v-head replaces L and V once T R is done.
    constexpr int QC_B = C * CKP * 2, L_B = C * CP * 4, W_B = C * KP * 4, V_B = DV * C * 2;
    static_assert(L_B <= QC_B, "L does not fit over the codes");
    static_assert(2 * W_B <= 2 * QC_B + 2 * V_B, "W's staging does not fit over L and V");
    __shared__ __attribute__((aligned(16))) char wy_lds[2 * QC_B + 2 * V_B];
    uint16_t *Qc = reinterpret_cast<uint16_t *>(wy_lds);
    uint16_t *Kc = reinterpret_cast<uint16_t *>(wy_lds + QC_B);
    float *Lg = reinterpret_cast<float *>(wy_lds + grp * QC_B);
    uint16_t *Vg = reinterpret_cast<uint16_t *>(wy_lds + 2 * QC_B + grp * V_B);
    __shared__ float graw_s[REP][C], gam[REP][C], bet[REP][C], Gs[REP][C], rq[C], rk[C];
    const float *betg = bet[grp], *Gsg = Gs[grp];

    // ---- the token-parallel front (c/layer.h:427-492 up to the
    // recurrence) for this chunk and K head: causal conv1d k=4 + SiLU
    // (c/gdn.h:19-33, 220-228) of the q, k channels of K head kh and the v
    // channels of its two v-heads, the l2norm factors (c/gdn.h:402-416) and
    // the gates (c/gdn.h:34-40). Work items are (two adjacent channels, 16
    // tokens): 512 of q|k, then 256 of v per v-head, two per thread. The
    // gates of padding rows (t >= nt) are 0.
    const bool first = __builtin_amdgcn_readfirstlane(ci == coff[P.s] ? 1 : 0) != 0;
    const uint16_t *cst = conv_state + (size_t)(slots ? slots[P.s] : P.s) * cd * 3;
    if (tid < REP * C) {                        // the gates of token t, v-head 2 kh + g
        const int g = tid / C, t = tid % C, h = kh * REP + g;
        float gg = 0.0f, bt = 0.0f;
        if (t < P.nt) {
            const size_t i = (size_t)(P.t0 + t) * hv + h;
            gg = decay_of(a[i], A_log[h], dt_bias[h]);
            bt = bf2f(sig_bf[b[i]]);
        }
        graw_s[g][t] = gg;
        bet[g][t] = bt;
    }
    static_assert(2 * DK * (C / TG) / 2 == 512 && REP * (DV / 2) * (C / TG) == 512,
                  "two conv items per thread");
    {
        // item A: q | k channels 2 lc, 2 lc + 1, tokens tgA ..; item B: v
        // channels n0, n0 + 1 of v-head 2 kh + g, tokens tgB .. (both
        // items' inputs are loaded before either's codes are formed)
        const int lc = 2 * (tid % DK), tgA = __builtin_amdgcn_readfirstlane((tid / DK) * TG);
        const size_t gA = lc < DK ? (size_t)kh * DK + lc : kd + (size_t)kh * DK + (lc - DK);
        const int g = tid / ((DV / 2) * (C / TG)), jv = tid % ((DV / 2) * (C / TG));
        const int n0 = 2 * (jv % (DV / 2)), tgB = __builtin_amdgcn_readfirstlane((jv / (DV / 2)) * TG);
        const size_t gB = 2 * kd + (size_t)(kh * REP + g) * DV + n0;
        ConvRows RA, RB;
        conv_rows16(qkv, cd, gA, P, tgA, first, cst, conv_w, RA);
        conv_rows16(qkv, cd, gB, P, tgB, first, cst, conv_w, RB);
        const int nt = __builtin_amdgcn_readfirstlane(P.nt);
        uint16_t c0[TG], c1[TG];
        conv_codes16(RA, tgA, nt, silu_bf, c0, c1);
        uint16_t *dst = (lc < DK ? Qc : Kc) + (lc & (DK - 1));
#pragma unroll
        for (int j = 0; j < TG; j++)
            *reinterpret_cast<uint32_t *>(dst + (tgA + j) * CKP) = (uint32_t)c0[j] | ((uint32_t)c1[j] << 16);
        conv_codes16(RB, tgB, nt, silu_bf, c0, c1);
        uint16_t *V = reinterpret_cast<uint16_t *>(wy_lds + 2 * QC_B + g * V_B);
#pragma unroll
        for (int h8 = 0; h8 < TG / 8; h8++) {
            u16x8 a0, a1;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                a0[j] = c0[h8 * 8 + j];
                a1[j] = c1[h8 * 8 + j];
            }
            const int t8 = tgB / 8 + h8;
            *reinterpret_cast<u16x8 *>(V + n0 * C + ((t8 ^ (n0 & 7)) << 3)) = a0;
            *reinterpret_cast<u16x8 *>(V + (n0 + 1) * C + ((t8 ^ ((n0 + 1) & 7)) << 3)) = a1;
        }
    }
    __syncthreads();
    if (tid < 2 * C) {                          // l2norm factors, one lane per row
        const int t = tid & (C - 1);
        const float f = t < P.nt ? 1.0f / sqrtf(row_sumsq((tid < C ? Qc : Kc) + t * CKP) + kL2Eps) : 0.0f;
        if (tid < C) rq[t] = f * qscale;
        else rk[t] = f;
    } else if (tid >= 256 && tid < 256 + REP * C) {   // gamma_t = g_0 + .. + g_t, in token order
        const int g = (tid - 256) / C, t = (tid - 256) % C;
        float acc = 0.0f;
        for (int u = 0; u <= t; u++) acc = acc + graw_s[g][u];
        gam[g][t] = acc;
    }
    // the scan's Q (rows t, 8 consecutive dims a piece) and K (dim i, 8
    // consecutive keys a piece) as code planes
    uint16_t *Qpu = Qp + (size_t)ku * C * DK, *Kpu = Kp + (size_t)ku * C * DK;
#pragma unroll
    for (int u = 0; u < C * DK / 8 / 512; u++) {
        const int e = tid + 512 * u;
        {
            const int t = e / (DK / 8), c0 = (e % (DK / 8)) * 8;
            *reinterpret_cast<u16x8 *>(Qpu + bx1_a_index(t, c0, DK / 32)) =
                *reinterpret_cast<const u16x8 *>(Qc + t * CKP + c0);
        }
        {
            const int i = e % DK, s0 = (e / DK) * 8;
            u16x8 x;
#pragma unroll
            for (int j = 0; j < 8; j++) x[j] = Kc[(s0 + j) * CKP + i];
            *reinterpret_cast<u16x8 *>(Kpu + bx1_b_index(s0, i)) = x;
        }
    }
    __syncthreads();
    // F of each v-head: the output scale G_t rq_t, the state-update scale
    // exp(gamma_C - gamma_s) rk_s, and G_C
    if (tid < REP * C) {
        const int g = tid / C, t = tid % C;
        float *F = Fb + (size_t)(ci * hv + kh * REP + g) * 3 * C;
        Gs[g][t] = exp_fast(gam[g][t]);
        F[t] = Gs[g][t] * rq[t];
        F[C + t] = exp_fast(gam[g][C - 1] - gam[g][t]) * rk[t];
        F[2 * C + t] = t == 0 ? exp_fast(gam[g][C - 1]) : 0.0f;
    }

    // products on the bf16 MFMA 16x16x32 on the codes (lane: row / column
    // r16, reduction indices g8 .. g8+7; result rows kq .. kq+3). Each
    // group of four wavefronts forms them for its v-head: wavefront gw takes
    // row block 3 - gw of Q K^T and row block gw of K K^T (5 tiles each; the
    // MFMAs are repeated per group, the decay and gate factors differ).
    const int r16 = lane & 15, kq = (lane >> 4) * 4, g8 = (lane >> 4) * 8;
    {
        // Q K^T: A = decayed lower triangle, to global. The product is
        // formed transposed (K Q^T) so each lane holds 4 consecutive key
        // columns s of one row t: 4 hi and 4 lo codes, two 8-byte stores.
        typedef unsigned short u16x4_t __attribute__((ext_vector_type(4)));
        const int rb = 3 - gw;
        const int t = rb * 16 + r16;
        uint16_t *A = Ab + (size_t)unitg * C * C * 2;
        auto put4 = [&](int s0, const float (&v)[4]) {
            u16x4_t hi, lo;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint16_t h, l;
                split_bf(v[i], h, l);
                hi[i] = h;
                lo[i] = l;
            }
            uint16_t *p = A + bx_a_index(t, s0, C / 32);
            *reinterpret_cast<u16x4_t *>(p) = hi;
            *reinterpret_cast<u16x4_t *>(p + 8) = lo;
        };
        if ((rb & 1) == 0) {           // the upper tile the scan's 32-column block covers
            const float z[4] = {0.f, 0.f, 0.f, 0.f};
            put4((rb + 1) * 16 + kq, z);
        }
        u16x8 qf[DK / 32];
#pragma unroll
        for (int ks = 0; ks < DK / 32; ks++) qf[ks] = ld8(Qc + t * CKP + ks * 32 + g8);
        const float qt = rq[t];
        const float *gm = gam[grp];
        for (int cb = 0; cb <= rb; cb++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < DK / 32; ks++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf(ld8(Kc + (cb * 16 + r16) * CKP + ks * 32 + g8)), as_bf(qf[ks]), acc, 0, 0, 0);
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int s = cb * 16 + kq + i;
                v[i] = s <= t ? exp_fast(gm[t] - gm[s]) * ((qt * rk[s]) * acc[i]) : 0.0f;
            }
            put4(cb * 16 + kq, v);
        }
    }
    // K K^T, row block gw: L, kept in registers until every reader of the
    // codes is done, then written over them
    float lv[4][4];
    {
        const float *gm = gam[grp];
        u16x8 kw[DK / 32];
#pragma unroll
        for (int ks = 0; ks < DK / 32; ks++) kw[ks] = ld8(Kc + (gw * 16 + r16) * CKP + ks * 32 + g8);
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            if (cb <= gw) {
                f32x4 gk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < DK / 32; ks++)
                    gk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        as_bf(kw[ks]), as_bf(ld8(Kc + (cb * 16 + r16) * CKP + ks * 32 + g8)), gk, 0, 0, 0);
                const int s = cb * 16 + r16;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = gw * 16 + kq + i;
                    lv[cb][i] = s < t ? betg[t] * (exp_fast(gm[t] - gm[s]) * ((rk[t] * rk[s]) * gk[i])) : 0.0f;
                }
            }
        }
    }
    __syncthreads();                   // every reader of the codes is done
#pragma unroll
    for (int cb = 0; cb < 4; cb++)
        if (cb <= gw)
#pragma unroll
            for (int i = 0; i < 4; i++) Lg[(gw * 16 + kq + i) * CP + cb * 16 + r16] = lv[cb][i];
    __syncthreads();

    // ---- per v-head (wavefronts 4 grp .. 4 grp + 3)
    constexpr int H = C / 2;
    if (gw < 2) {
        const int o = gw * H;                  // this diagonal block's first row / column
        float x[H];
#pragma unroll
        for (int t = 0; t < H; t++) x[t] = t == lane ? 1.0f : 0.0f;
#pragma unroll
        for (int t = 1; t < H; t++) {
            float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
            for (int s0 = 0; s0 < t; s0 += 4) {
                const float4 l4 = lds4(Lg + (o + t) * CP + o + s0);
                p0 = fmaf(l4.x, x[s0], p0);
                if (s0 + 1 < t) p1 = fmaf(l4.y, x[s0 + 1], p1);
                if (s0 + 2 < t) p2 = fmaf(l4.z, x[s0 + 2], p2);
                if (s0 + 3 < t) p3 = fmaf(l4.w, x[s0 + 3], p3);
            }
            x[t] = x[t] - ((p0 + p1) + (p2 + p3));
        }
        // (this wavefront's reads of L are all issued: DS operations run in order)
        if (lane < H) {
#pragma unroll
            for (int t = 0; t < H; t++) Lg[(o + t) * CP + o + lane] = x[t];
        }
    }
    __syncthreads();
    {
        // wavefront w: output tile (w / 2, w % 2) of the 32x32 products
        const int tr = (gw >> 1) * 16, tc = (gw & 1) * 16;
        const int rr = lane & 15, kk = (lane >> 4) * 8;
        // Y = L10 T00: A = L rows H + tr + rr, k = kk..; B = T00 column tc + rr
        u16x8 ah, al, bh, bl;
        {
            const float4 a0 = lds4(Lg + (H + tr + rr) * CP + kk), a1 = lds4(Lg + (H + tr + rr) * CP + kk + 4);
            const float va[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            split8(va, ah, al);
            float vb[8];
#pragma unroll
            for (int j = 0; j < 8; j++) vb[j] = Lg[(kk + j) * CP + tc + rr];
            split8(vb, bh, bl);
        }
        f32x4 y = mfma_x3(ah, al, bh, bl, f32x4{0.f, 0.f, 0.f, 0.f});
        // Y to the upper-right block [k = row][n]: rows tr + 4(l/16) + i, column tc + rr
#pragma unroll
        for (int i = 0; i < 4; i++) Lg[(tr + (lane >> 4) * 4 + i) * CP + H + tc + rr] = y[i];
        __syncthreads();
        // T10 = -T11 Y: A = T11 rows H + tr + rr, k = H + kk..; B = Y column tc + rr
        {
            const float4 a0 = lds4(Lg + (H + tr + rr) * CP + H + kk), a1 = lds4(Lg + (H + tr + rr) * CP + H + kk + 4);
            const float va[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            split8(va, ah, al);
            float vb[8];
#pragma unroll
            for (int j = 0; j < 8; j++) vb[j] = Lg[(kk + j) * CP + H + tc + rr];
            split8(vb, bh, bl);
        }
        const f32x4 t10 = mfma_x3(ah, al, bh, bl, f32x4{0.f, 0.f, 0.f, 0.f});
        __syncthreads();                         // every read of L10 and Y is done
#pragma unroll
        for (int i = 0; i < 4; i++) Lg[(H + tr + (lane >> 4) * 4 + i) * CP + tc + rr] = -t10[i];
        // the upper-right block back to zero (T is lower triangular; T R reads
        // only k below its row block, but keep the matrix clean)
#pragma unroll
        for (int i = 0; i < 4; i++) Lg[(tr + (lane >> 4) * 4 + i) * CP + H + tc + rr] = 0.0f;
    }
    __syncthreads();
    const int g4 = kq;
    const int cbase = gw * 64;                // this wavefront's 64 columns of R
    const bool isv = cbase < DV;
    f32x4 xacc[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; rt++)
#pragma unroll
        for (int ct = 0; ct < 4; ct++) xacc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    // R = [diag(b) V | diag(b G rk) K] with V and K exact codes: a
    // wavefront's 64 columns are of one kind, so its T operand carries that
    // kind's row factors (T diag(f), split hi/lo) and the codes are the B
    // operand as they are: two MFMAs per product
#pragma unroll
    for (int ks = 0; ks < C / 32; ks++) {
        const int k0 = ks * 32 + g8;             // this lane's 8 reduction indices
        float f[8];
#pragma unroll
        for (int j = 0; j < 8; j++) f[j] = isv ? betg[k0 + j] : (betg[k0 + j] * Gsg[k0 + j]) * rk[k0 + j];
        u16x8 ah[4], al[4], bc[4];
#pragma unroll
        for (int rt = 2 * ks; rt < 4; rt++) {    // T rows 16 rt + r16
            const float4 a0 = lds4(Lg + (rt * 16 + r16) * CP + k0);
            const float4 a1 = lds4(Lg + (rt * 16 + r16) * CP + k0 + 4);
            const float v[8] = {a0.x * f[0], a0.y * f[1], a0.z * f[2], a0.w * f[3],
                                a1.x * f[4], a1.y * f[5], a1.z * f[6], a1.w * f[7]};
            split8(v, ah[rt], al[rt]);
        }
#pragma unroll
        for (int ct = 0; ct < 4; ct++) {         // R column n, rows k0 .. k0 + 7
            const int n = cbase + ct * 16 + r16;
            if (isv) {
                bc[ct] = ld8(Vg + n * C + (((k0 >> 3) ^ (n & 7)) << 3));
            } else {
                bc[ct] = ld8(Kpu + bx1_b_index(k0, n - DV));   // keys k0 .. k0+7 of dim n - DV
            }
        }
#pragma unroll
        for (int rt = 2 * ks; rt < 4; rt++)
#pragma unroll
            for (int ct = 0; ct < 4; ct++) {
                xacc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(al[rt]), as_bf(bc[ct]), xacc[rt][ct], 0, 0, 0);
                xacc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(ah[rt]), as_bf(bc[ct]), xacc[rt][ct], 0, 0, 0);
            }
    }
    const size_t ub = (size_t)unitg * C * DV;
    if (isv) {                         // U: the accumulator order is U's layout
#pragma unroll
        for (int rt = 0; rt < 4; rt++)
#pragma unroll
            for (int ct = 0; ct < 4; ct++)
                *reinterpret_cast<float4 *>(Ub + ub + wy_u_index(rt * 16 + g4, cbase + ct * 16 + r16)) =
                    make_float4(xacc[rt][ct][0], xacc[rt][ct][1], xacc[rt][ct][2], xacc[rt][ct][3]);
    }
    // W through LDS (L is no longer read): column tid - DV of every row in,
    // then 32-byte units of 8 consecutive columns of one row out
    __syncthreads();                   // every reader of T, V and the k codes is done
    float *Wl = reinterpret_cast<float *>(wy_lds + grp * W_B);   // over both Ls and Vs
    if (!isv) {
#pragma unroll
        for (int rt = 0; rt < 4; rt++)
#pragma unroll
            for (int ct = 0; ct < 4; ct++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    Wl[(rt * 16 + g4 + i) * KP + (cbase - DV + ct * 16 + r16)] = xacc[rt][ct][i];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < C * DK / 8 / 256; u++) {
        const int e = gtid + 256 * u, t = e / (DK / 8), c0 = (e % (DK / 8)) * 8;
        float w8[8];
        const float4 a0 = lds4(Wl + t * KP + c0), a1 = lds4(Wl + t * KP + c0 + 4);
        w8[0] = a0.x; w8[1] = a0.y; w8[2] = a0.z; w8[3] = a0.w;
        w8[4] = a1.x; w8[5] = a1.y; w8[6] = a1.z; w8[7] = a1.w;
        put_split8(Wb + 2 * ub + bx_a_index(t, c0, DK / 32), w8);
    }
}

// Chunk-to-chunk scan of one 16-column slice of one head's state.
// Block index = cb * (B*hv) + (s*hv + h): the 8 slices of a head share
// their operand reads, and with B*hv a multiple of 8 they land on the same
// XCD (blocks are dealt round-robin over the 8 XCDs) and so share its L2.
// 512 threads in two roles, two wavefronts per SIMD:
//   waves 0-3 carry the recurrence: D = U - W S0 (rows 16w..), then
//             S1^T = G_C S0^T + Dp^T K (state rows 32w..);
//   waves 4-7 produce the chunk's outputs meanwhile: G_t (Q S0), then
//             + A D once D is complete, rnd(o) to ob.
// Products run on the 16x16x32 bf16 MFMA in split precision (hi.hi +
// hi.lo + lo.hi); the state slice is kept in fp32 and, for the MFMA, as
// hi/lo codes made once when it is written. Each wavefront loads the next
// chunk's operands it consumes into registers as soon as the current copy
// is used.
constexpr int SB = DK + 8;     // bf16 row stride of the state slice copies
constexpr int DB = C + 8;      // bf16 row stride of the D copies

// One chunk step's operands in registers. A wavefront uses one role's
// fields only, so the two roles share the storage:
//   recurrence: ScanOps b = W (row block w: 4 column blocks x hi/lo), u = U;
//               ScanOps2 b = K (2 state-row blocks x 2 key blocks x hi/lo);
//   output:     ScanOps b = Q (row block w); ScanOps2 b[0..3] = A (causal part).
// The operands a step needs first (W / Q, U, the decay factors) form a
// two-slot ring: step ci reads slot ci % 2 and, once they are consumed,
// reloads them with step ci + 2's, so those loads have two chunk steps to
// arrive; K / A (needed late in a step) are loaded one step ahead.
struct ScanOps {
    u16x8 b[8];
    float4 u;
    float f;                        // decay factors (threads < 2C)
};
struct ScanOps2 {
    u16x8 b[8];                     // K (recurrence) or A (output), one step ahead
};

__device__ __forceinline__ void scan_load_wu(ScanOps &nx, const uint16_t *__restrict__ Wb,
                                             const float *__restrict__ Ub, size_t u, int wave,
                                             int lane, int cb) {
    const uint16_t *W = Wb + u * C * DK * 2 + ((size_t)wave * (DK / 32) * 64 + lane) * 16;
#pragma unroll
    for (int kb = 0; kb < DK / 32; kb++) {
        nx.b[2 * kb] = ld8(W + kb * 64 * 16);
        nx.b[2 * kb + 1] = ld8(W + kb * 64 * 16 + 8);
    }
    nx.u = ld4(Ub + u * C * DV + ((size_t)(cb * 4 + wave) * 64 + lane) * 4);
}

__device__ __forceinline__ void scan_load_k(ScanOps2 &nx, const uint16_t *__restrict__ Kp,
                                            size_t uk, int wave, int lane) {
    const uint16_t *K = Kp + uk * C * DK + ((size_t)wave * 2 * (C / 32) * 64 + lane) * 8;
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int kb = 0; kb < C / 32; kb++) nx.b[2 * r + kb] = ld8(K + (r * (C / 32) + kb) * 64 * 8);
}

__device__ __forceinline__ void scan_load_q(ScanOps &nx, const uint16_t *__restrict__ Qp,
                                            size_t uk, int ow, int lane) {
    const uint16_t *Q = Qp + uk * C * DK + ((size_t)ow * (DK / 32) * 64 + lane) * 8;
#pragma unroll
    for (int kb = 0; kb < DK / 32; kb++) nx.b[kb] = ld8(Q + kb * 64 * 8);
}

__device__ __forceinline__ void scan_load_a(ScanOps2 &nx, const uint16_t *__restrict__ Ab,
                                            size_t u, int ow, int lane) {
    const uint16_t *Ar = Ab + u * C * C * 2 + ((size_t)ow * (C / 32) * 64 + lane) * 16;
#pragma unroll
    for (int kb = 0; kb < C / 32; kb++) {      // (the block past the diagonal is unused)
        nx.b[2 * kb] = ld8(Ar + kb * 64 * 16);
        nx.b[2 * kb + 1] = ld8(Ar + kb * 64 * 16 + 8);
    }
}

__global__ __launch_bounds__(512) void k_gdn_chunk_scan(
    ChunkSeqs sq, const int32_t *__restrict__ dmeta, const uint16_t *__restrict__ Qp,
    const uint16_t *__restrict__ Kp, const float *__restrict__ Ub,
    const uint16_t *__restrict__ Wb, const uint16_t *__restrict__ Ab,
    const float *__restrict__ Fb, float *__restrict__ S, uint16_t *__restrict__ ob, int hk,
    const int32_t *__restrict__ slots) {
    const int hv = hk * REP;
    const size_t vd = (size_t)hv * DV;
    const int nsh = sq.n * hv;
    const int cb = blockIdx.x / nsh, sh = blockIdx.x % nsh;
    const int s = sh / hv, h = sh % hv, kh = h / REP;
    const int32_t *cu = dmeta ? dmeta : sq.cu;
    const int32_t *coff = dmeta ? dmeta + sq.n + 1 : sq.coff;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool rec = wave < 4;                  // recurrence or output role
    const int wr = wave & 3;
    const int rw = wr * 16;                     // the role's 16-row block
    const int r16 = lane & 15, g4 = lane >> 4;  // MFMA row / column, lane group
    const int kq = g4 * 4;

    // The state slice and the decay factors are double-buffered by chunk
    // parity: step ci reads copy ci & 1 and writes step ci + 1's into the
    // other, so a step needs two barriers (state in place; D complete).
    __shared__ __attribute__((aligned(16))) float S0Tb[2][CB * KP];    // S slice [col][row]
    __shared__ __attribute__((aligned(16))) uint16_t S0hb[2][CB * SB]; // its hi / lo codes
    __shared__ __attribute__((aligned(16))) uint16_t S0lb[2][CB * SB];
    __shared__ __attribute__((aligned(16))) uint16_t Dh[CB * DB];      // D [col][t], hi / lo
    __shared__ __attribute__((aligned(16))) uint16_t Dl[CB * DB];
    __shared__ __attribute__((aligned(16))) uint16_t Dph[CB * DB];     // decayed D
    __shared__ __attribute__((aligned(16))) uint16_t Dpl[CB * DB];
    __shared__ float Fsb[2][3 * C];
    __shared__ __attribute__((aligned(16))) uint16_t Ost[4][16 * CB];   // output role: rnd(o) tiles

    // state slice in: packed layout ((j/64*32 + i/4)*64 + j%64)*4 + i%4
    float *Sm = S + ((size_t)(slots ? slots[s] : s) * hv + h) * DK * DV;
    const int jb = (cb * CB) / 64 * 32, jl = (cb * CB) % 64;
    const int c0 = coff[s], c1 = coff[s + 1];
    {
        const int p0 = c0 & 1;
        for (int e = tid; e < CB * DK; e += 512) {
            const int q = e / 64, rem = e % 64, jj = rem / 4, r = rem % 4;
            const float x = Sm[((size_t)(jb + q) * 64 + jl + jj) * 4 + r];
            S0Tb[p0][jj * KP + 4 * q + r] = x;
            split_bf(x, S0hb[p0][jj * SB + 4 * q + r], S0lb[p0][jj * SB + 4 * q + r]);
        }
    }

    const int tS = cu[s], tE = cu[s + 1];
    // Prefetches are unconditional, their chunk clamped to the sequence's
    // last (re-read, unused): with no branch around them, and the two roles
    // in loops of their own, every wait on a prefetch counts exactly the
    // loads and stores issued after it instead of draining them all.
    auto cl = [&](int ci) { return (size_t)min(ci, c1 - 1); };
    if (c0 < c1 && rec) {
        // ---- recurrence role: D = U - W S0 and S1 = G_C S0 + Dp^T K
        ScanOps ring0, ring1;
        ScanOps2 kf;
        auto load_wu = [&](ScanOps &nx, int ci) {
            const size_t u = cl(ci) * hv + h;
            if (tid < 3 * C) nx.f = Fb[u * 3 * C + tid];
            scan_load_wu(nx, Wb, Ub, u, wr, lane, cb);
        };
        load_wu(ring0, c0);
        if (tid < 3 * C) Fsb[c0 & 1][tid] = ring0.f;
        scan_load_k(kf, Kp, cl(c0) * hk + kh, wr, lane);
        load_wu(ring1, c0 + 1);
        auto step = [&](ScanOps &cur, const ScanOps &oth, int ci) {
            const bool more = ci + 1 < c1;
            const float *S0T = S0Tb[ci & 1], *Fs = Fsb[ci & 1];
            const uint16_t *S0h = S0hb[ci & 1], *S0l = S0lb[ci & 1];
            if (tid < 3 * C) cur.f = Fb[(cl(ci + 2) * hv + h) * 3 * C + tid];
            __syncthreads();           // the state slice and Fs of this chunk are in place;
                                       // every reader of the last step's D is done
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < DK / 32; kb++)
                acc = mfma_x3(cur.b[2 * kb], cur.b[2 * kb + 1],
                              ld8(S0h + r16 * SB + kb * 32 + g4 * 8),
                              ld8(S0l + r16 * SB + kb * 32 + g4 * 8), acc);
            const float uu[4] = {cur.u.x, cur.u.y, cur.u.z, cur.u.w};
            {
                // tokens rw + kq .. + 3 of column r16: 8-byte pieces
                u16x4 dh, dl, ph, pl;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = rw + kq + i;
                    const float d = uu[i] - acc[i];
                    uint16_t a0, a1, b0, b1;
                    split_bf(d, a0, a1);
                    split_bf(Fs[C + t] * d, b0, b1);
                    dh[i] = a0; dl[i] = a1; ph[i] = b0; pl[i] = b1;
                }
                const int o = r16 * DB + rw + kq;
                *reinterpret_cast<u16x4 *>(Dh + o) = dh;
                *reinterpret_cast<u16x4 *>(Dl + o) = dl;
                *reinterpret_cast<u16x4 *>(Dph + o) = ph;
                *reinterpret_cast<u16x4 *>(Dpl + o) = pl;
            }
            scan_load_wu(cur, Wb, Ub, cl(ci + 2) * hv + h, wr, lane, cb);
            __syncthreads();           // D complete
            // S1 = G_C S0 + K^T Dp, formed as [state row][column] (the codes
            // as the A operand): a lane holds rows i0 + kq .. + 3 of column
            // r16, so its S0 reads and S1 writes are 16- and 8-byte pieces
            f32x4 sn[2];
            const float gc = Fs[2 * C];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int i0 = wr * 32 + r * 16;
                const f32x4 s0 = *reinterpret_cast<const f32x4 *>(S0T + r16 * KP + i0 + kq);
#pragma unroll
                for (int i = 0; i < 4; i++) sn[r][i] = gc * s0[i];
#pragma unroll
                for (int kb = 0; kb < C / 32; kb++)
                    sn[r] = mfma_x2a(kf.b[2 * r + kb], ld8(Dph + r16 * DB + kb * 32 + g4 * 8),
                                     ld8(Dpl + r16 * DB + kb * 32 + g4 * 8), sn[r], false);
            }
            scan_load_k(kf, Kp, cl(ci + 1) * hk + kh, wr, lane);
            // the next step's state and factors go to the other copies
            // (their last readers were in step ci - 1, before this step's
            // first barrier)
            float *S1T = S0Tb[(ci + 1) & 1];
            uint16_t *S1h = S0hb[(ci + 1) & 1], *S1l = S0lb[(ci + 1) & 1];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int o = wr * 32 + r * 16 + kq;
                u16x4 h4, l4;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint16_t a0, a1;
                    split_bf(sn[r][i], a0, a1);
                    h4[i] = a0;
                    l4[i] = a1;
                }
                *reinterpret_cast<f32x4 *>(S1T + r16 * KP + o) = sn[r];
                *reinterpret_cast<u16x4 *>(S1h + r16 * SB + o) = h4;
                *reinterpret_cast<u16x4 *>(S1l + r16 * SB + o) = l4;
            }
            if (more && tid < 3 * C) Fsb[(ci + 1) & 1][tid] = oth.f;
        };
        for (int ci = c0; ci < c1; ci += 2) {
            step(ring0, ring1, ci);
            if (ci + 1 < c1) step(ring1, ring0, ci + 1);
        }
    } else if (c0 < c1) {
        // ---- output role: O = G Q S0 + A D, then rnd(o) out
        // Q and A both in two-slot rings (two steps ahead): the first wait
        // issued behind a step's output stores then comes three steps later
        ScanOps ring0, ring1;
        ScanOps2 af0, af1;
        scan_load_q(ring0, Qp, cl(c0) * hk + kh, wr, lane);
        scan_load_a(af0, Ab, cl(c0) * hv + h, wr, lane);
        scan_load_q(ring1, Qp, cl(c0 + 1) * hk + kh, wr, lane);
        scan_load_a(af1, Ab, cl(c0 + 1) * hv + h, wr, lane);
        auto step = [&](ScanOps &cur, ScanOps2 &af, int ci) {
            const int t0 = tS + (ci - c0) * C, nt = min(C, tE - t0);
            const float *Fs = Fsb[ci & 1];
            const uint16_t *S0h = S0hb[ci & 1], *S0l = S0lb[ci & 1];
            __syncthreads();           // the state slice and Fs of this chunk are in place
            f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < DK / 32; kb++)
                o = mfma_x2a(cur.b[kb], ld8(S0h + r16 * SB + kb * 32 + g4 * 8),
                             ld8(S0l + r16 * SB + kb * 32 + g4 * 8), o, false);
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = Fs[rw + kq + i] * o[i];
            scan_load_q(cur, Qp, cl(ci + 2) * hk + kh, wr, lane);
            __syncthreads();           // D complete
            // ... + A D over the causal part s < rw + 16
#pragma unroll
            for (int kb = 0; kb < C / 32; kb++)
                if (kb <= wr / 2)
                    o = mfma_x3(af.b[2 * kb], af.b[2 * kb + 1],
                                ld8(Dh + r16 * DB + kb * 32 + g4 * 8),
                                ld8(Dl + r16 * DB + kb * 32 + g4 * 8), o);
            scan_load_a(af, Ab, cl(ci + 2) * hv + h, wr, lane);
            // rnd(o) through a wave-private LDS tile, so that 32 lanes store
            // the 16 rows as 16-byte pieces (2-byte stores run ~20x slower)
            uint16_t *Ow = Ost[wr];
#pragma unroll
            for (int i = 0; i < 4; i++) Ow[(kq + i) * CB + r16] = f2bf(o[i]);
            __builtin_amdgcn_wave_barrier();
            if (lane < 32) {
                const int rr = lane >> 1, half = lane & 1, t = rw + rr;
                const u16x8 v8 = *reinterpret_cast<const u16x8 *>(Ow + rr * CB + half * 8);
                if (t < nt)
                    *reinterpret_cast<u16x8 *>(ob + (size_t)(t0 + t) * vd + (size_t)h * DV +
                                               cb * CB + half * 8) = v8;
            }
        };
        for (int ci = c0; ci < c1; ci += 2) {
            step(ring0, af0, ci);
            if (ci + 1 < c1) step(ring1, af1, ci + 1);
        }
    }
    __syncthreads();
    const float *S1T = S0Tb[c1 & 1];   // the state after the last chunk
    for (int e = tid; e < CB * DK; e += 512) {
        const int q = e / 64, rem = e % 64, jj = rem / 4, r = rem % 4;
        Sm[((size_t)(jb + q) * 64 + jl + jj) * 4 + r] = S1T[jj * KP + 4 * q + r];
    }
}

}  // namespace

namespace apus {

// Chunked prefill; slots_h (host, nullable): the state slot of each
// sequence in conv_state / S (identity when null).
// The buffers of one prefill call carved from a workspace (256-byte
// aligned pieces): the token-parallel intermediates, the per (chunk,
// v-head) WY operands and the device metadata. bytes: the total.
struct PrefillWs {
    GdnScratch w;
    float *Ub = nullptr, *Fb = nullptr;
    uint16_t *Wb = nullptr, *Ab = nullptr, *Qp = nullptr, *Kp = nullptr;
    int32_t *meta = nullptr;
    size_t bytes = 0;
};
static PrefillWs prefill_ws_carve(char *base, size_t Ttot, size_t nch, size_t B, size_t hk,
                                  size_t hv) {
    PrefillWs p;
    size_t off = 0;
    auto take = [&](size_t n) {
        char *q = base ? base + off : nullptr;
        off += (n + 255) / 256 * 256;
        return q;
    };
    const size_t vd = hv * DV, units = nch * hv;
    p.w.ob = (uint16_t *)take(Ttot * vd * 2);
    p.Ub = (float *)take(units * C * DV * 4);
    p.Wb = (uint16_t *)take(units * C * DK * 4);
    p.Ab = (uint16_t *)take(units * C * C * 4);
    p.Fb = (float *)take(units * 3 * C * 4);
    p.Qp = (uint16_t *)take(nch * hk * C * DK * 2);
    p.Kp = (uint16_t *)take(nch * hk * C * DK * 2);
    p.meta = (int32_t *)take(2 * (B + 1) * 4);
    p.bytes = off;
    return p;
}

// ws: a workspace of ws_bytes bytes the whole call works in (nothing is
// allocated; then B <= kPrefillInline and no slot map), or nullptr for
// library scratch.
static int gdn_prefill_run(const ApusHipGdnLayer *L, size_t B, const int32_t *cu,
                           const uint16_t *qkv, const uint16_t *z, const uint16_t *a,
                           const uint16_t *b, uint16_t *conv_state, float *S, uint16_t *y,
                           const int32_t *slots_h, char *ws = nullptr, size_t ws_bytes = 0) {
    if (int r = gdn_check_layer(L)) return r;
    if (B == 0) return kOk;
    if (int r = gdn_check_offsets(B, cu)) return r;
    const size_t Ttot = (size_t)cu[B];
    if (Ttot == 0) return kOk;
    if (B * L->hv * NCB > 0x7fffffffu) return set_error(kErrArgument, "batch too large");

    // metadata [cu | chunk offsets]: by value for small batches (k_gdn_prep
    // and k_gdn_post take cu for up to kGdnCuInline sequences, WY and the
    // scan both arrays for up to kPrefillInline), else a device copy
    // (a stack array for the batches whose metadata travels by value: the
    // allocation-free entry allocates nothing, host memory included)
    int32_t meta_small[2 * (kPrefillInline + 1)];
    std::vector<int32_t> meta_big;
    if (B > (size_t)kPrefillInline) meta_big.resize(2 * (B + 1));
    int32_t *meta = B > (size_t)kPrefillInline ? meta_big.data() : meta_small;
    const size_t nmeta = 2 * (B + 1);
    memcpy(meta, cu, (B + 1) * 4);
    int32_t *coff = meta + B + 1;
    coff[0] = 0;
    for (size_t s = 0; s < B; s++) coff[s + 1] = coff[s] + (cu[s + 1] - cu[s] + C - 1) / C;
    const size_t nch = (size_t)coff[B];
    PrefillWs pw;
    if (ws) {
        if (B > (size_t)kPrefillInline || slots_h)
            return set_error(kErrUnsupported,
                             "the allocation-free prefill takes up to %d sequences, no slot map",
                             kPrefillInline);
        pw = prefill_ws_carve(nullptr, Ttot, nch, B, L->hk, L->hv);
        if (pw.bytes > ws_bytes)
            return set_error(kErrUnsupported,
                             "prefill of %zu tokens in %zu chunks needs %zu bytes of scratch; the "
                             "allocation-free entry has %zu",
                             Ttot, nch, pw.bytes, ws_bytes);
        pw = prefill_ws_carve(ws, Ttot, nch, B, L->hk, L->hv);
    }
    ChunkSeqs sq;
    sq.n = (int32_t)B;
    const int32_t *dmeta, *kmeta;
    if (B <= (size_t)kPrefillInline) {
        memcpy(sq.cu, cu, (B + 1) * 4);
        memcpy(sq.coff, coff, (B + 1) * 4);
        dmeta = nullptr;                       // prep / post take cu by value
        if (B > (size_t)kGdnCuInline) {
            int32_t *m = ws ? pw.meta : (int32_t *)scratch(kScratchMeta3, nmeta * 4);
            if (!m) return kErrHip;
            k_prefill_meta<<<1, 256, 0, stream()>>>(sq, m);
            APUS_LAUNCHED("k_prefill_meta");
            dmeta = m;
        }
        kmeta = nullptr;
    } else {
        dmeta = (const int32_t *)upload_async(meta, nmeta * 4);
        if (!dmeta) return kErrHip;
        kmeta = dmeta;
    }

    const int32_t *slots = nullptr;
    if (slots_h) {
        slots = (const int32_t *)upload_async(slots_h, B * 4);
        if (!slots) return kErrHip;
    }
    GdnScratch w = pw.w;                       // workspace buffers, or null: scratch
    if (!ws) w.ob = (uint16_t *)scratch(kScratchGdnOB, Ttot * L->hv * DV * 2);
    if (!w.ob) return kErrHip;
    const ApusHipGdnTrace *tr = gdn_trace();
    if (tr && (tr->qkv_conv || tr->beta || tr->gdecay)) {
        // the trace's token-parallel intermediates (the chunk kernel forms
        // its own copies of them)
        GdnScratch tw{};
        if (int r = gdn_prep(L, B, cu, dmeta, Ttot, qkv, a, b, conv_state, &tw, false, slots, tr))
            return r;
    }
    const ActTables *tabs = act_tables();
    if (!tabs) return kErrHip;
    const size_t units = nch * L->hv;
    float *Ub = ws ? pw.Ub : (float *)scratch(kScratchGdnChunk, units * C * DV * 4);
    uint16_t *Wb = ws ? pw.Wb : (uint16_t *)scratch(kScratchGdnChunk2, units * C * DK * 4);
    uint16_t *Ab = ws ? pw.Ab : (uint16_t *)scratch(kScratchGdnChunk4, units * C * C * 4);
    float *Fb = ws ? pw.Fb : (float *)scratch(kScratchGdnChunk5, units * 3 * C * 4);
    uint16_t *Qp = ws ? pw.Qp : (uint16_t *)scratch(kScratchGdnChunk6, nch * L->hk * C * DK * 2);
    uint16_t *Kp = ws ? pw.Kp : (uint16_t *)scratch(kScratchGdnChunk7, nch * L->hk * C * DK * 2);
    if (!Ub || !Wb || !Ab || !Fb || !Qp || !Kp) return kErrHip;
    APUS_TIMED("k_gdn_chunk_wy",
               k_gdn_chunk_wy<<<(unsigned)(nch * L->hk), 512, 0, stream()>>>(
        sq, kmeta, qkv, a, b, L->conv_w, L->A_log, L->dt_bias, conv_state, slots,
        tabs->silu_bf, tabs->sig_bf, Ub, Wb, Ab, Fb, Qp, Kp, (int)L->hk,
        (float)pow((double)L->dk, -0.5)));
    APUS_LAUNCHED("k_gdn_chunk_wy");
    APUS_TIMED("k_gdn_chunk_scan",
               k_gdn_chunk_scan<<<(unsigned)(B * L->hv * NCB), 512, 0, stream()>>>(
        sq, kmeta, Qp, Kp, Ub, Wb, Ab, Fb, S, w.ob, (int)L->hk, slots));
    APUS_LAUNCHED("k_gdn_chunk_scan");
    if (tr && tr->rec_o)                       // rnd(o) of every token, as the scan left it
        APUS_HIP_TRY(hipMemcpyAsync(tr->rec_o, w.ob, Ttot * L->hv * DV * 2,
                                    hipMemcpyDeviceToDevice, stream()));
    if (int r = gdn_post(L, B, cu, dmeta, Ttot, &w, z, qkv, conv_state, y, slots)) return r;
    if (tr && tr->onorm)
        APUS_HIP_TRY(hipMemcpyAsync(tr->onorm, y, Ttot * L->hv * DV * 2, hipMemcpyDeviceToDevice,
                                    stream()));
    return kOk;
}

}  // namespace apus

extern "C" {

int apus_hip_gdn_prefill(const ApusHipGdnLayer *L, size_t B, const int32_t *cu,
                         const uint16_t *qkv, const uint16_t *z, const uint16_t *a,
                         const uint16_t *b, uint16_t *conv_state, float *S, uint16_t *y) {
    APUS_READY();
    return gdn_prefill_run(L, B, cu, qkv, z, a, b, conv_state, S, y, nullptr);
}

int apus_hip_gdn_prefill_noalloc(const ApusHipGdnLayer *L, size_t B, const int32_t *cu,
                                 const uint16_t *qkv, const uint16_t *z, const uint16_t *a,
                                 const uint16_t *b, uint16_t *conv_state, float *S, uint16_t *y) {
    APUS_READY();
    char *ws = (char *)noalloc_scratch();
    if (!ws) return set_error(kErrHip, "the allocation-free scratch of this device is not set up");
    // a trace's intermediates would need library scratch (an allocation)
    if (gdn_trace())
        return set_error(kErrUnsupported,
                         "the allocation-free prefill does not capture traces (clear the trace "
                         "with apus_hip_trace_set first)");
    return gdn_prefill_run(L, B, cu, qkv, z, a, b, conv_state, S, y, nullptr, ws,
                           kNoAllocScratchBytes);
}

int apus_hip_gdn_prefill_slots(const ApusHipGdnLayer *L, size_t B, const int32_t *slots,
                               const int32_t *cu, const uint16_t *qkv, const uint16_t *z,
                               const uint16_t *a, const uint16_t *b, uint16_t *conv,
                               float *S, uint16_t *y) {
    APUS_READY();
    if (B == 0) return kOk;
    if (!slots) return set_error(kErrArgument, "NULL slot map");
    if (int r = gdn_check_offsets(B, cu)) return r;
    std::vector<int32_t> sorted;
    for (size_t s = 0; s < B; s++) {
        if (slots[s] < 0) return set_error(kErrArgument, "negative state slot");
        if (cu[s + 1] > cu[s]) sorted.push_back(slots[s]);
    }
    std::sort(sorted.begin(), sorted.end());
    for (size_t i = 1; i < sorted.size(); i++)
        if (sorted[i] == sorted[i - 1])
            return set_error(kErrArgument, "two sequences use state slot %d", sorted[i]);
    return gdn_prefill_run(L, B, cu, qkv, z, a, b, conv, S, y, slots);
}

}  // extern "C"
