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
// Kernels (after k_gdn_prep, before k_gdn_post of gdn_mixer.hip):
//   k_gdn_chunk_wy    one workgroup per (chunk, v-head), all chunks in
//                     parallel: K K^T and Q K^T on fp32 MFMA, L and A with
//                     their decay factors, then U and W by forward
//                     substitution (one thread per right-hand-side column).
//   k_gdn_chunk_scan  one workgroup per (sequence, v-head, 16-column block
//                     of S): the delta rule is separable by value column,
//                     so the chunk-to-chunk carry of S runs in 8 independent
//                     column slices per head, each walking its sequence's
//                     chunks in order on fp32 MFMA (D, O, S1 above).
// All products run on fp32 MFMA with fp32 accumulation: the recurrent
// state must stay within 1e-4 of the sequential fp32 recurrence, which
// bf16 operands (8-bit mantissa) cannot hold. The chunk form sums in a
// different order from the reference's token loop -- a tolerance class,
// checked against the sequential oracle.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"
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
__device__ __forceinline__ f32x4 mfma_k16(float4 a, float4 b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
    return c;
}

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

// Per (chunk, v-head) buffers written by k_gdn_chunk_wy:
//   U [C][DV], W [C][DK], A [C][C] (rows t, lower triangle incl. diagonal
//   valid), F [2][C]: F[0][t] = G_t, F[1][s] = exp(gamma_C - gamma_s).
__global__ __launch_bounds__(256) void k_gdn_chunk_wy(
    ChunkSeqs sq, const int32_t *__restrict__ dmeta, const float *__restrict__ qk,
    const uint16_t *__restrict__ vconv, const float2 *__restrict__ gate,
    const float *__restrict__ graw, float *__restrict__ Ub, float *__restrict__ Wb,
    float *__restrict__ Ab, float *__restrict__ Fb, int hk) {
    const int hv = hk * REP;
    const size_t kd = (size_t)hk * DK, vd = (size_t)hv * DV;
    const int ci = blockIdx.x / hv, h = blockIdx.x % hv, kh = h / REP;
    const int32_t *cu = dmeta ? dmeta : sq.cu;
    const int32_t *coff = dmeta ? dmeta + sq.n + 1 : sq.coff;
    const ChunkPos P = chunk_pos(cu, coff, sq.n, ci);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    __shared__ __attribute__((aligned(16))) float Ks[C * KP];
    __shared__ __attribute__((aligned(16))) float Qs[C * KP];
    __shared__ __attribute__((aligned(16))) float Ls[C * CP];
    __shared__ float gam[C], bet[C], Gs[C];

    // rows t >= nt are padding: q = k = 0, g = 0, beta = 0
    for (int e = tid; e < C * DK / 4; e += 256) {
        const int t = e / (DK / 4), q4 = (e % (DK / 4)) * 4;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f), k = q;
        if (t < P.nt) {
            const float *row = qk + (size_t)(P.t0 + t) * 2 * kd + (size_t)kh * DK + q4;
            q = ld4(row);
            k = ld4(row + kd);
        }
        *reinterpret_cast<float4 *>(Qs + t * KP + q4) = q;
        *reinterpret_cast<float4 *>(Ks + t * KP + q4) = k;
    }
    if (tid < C) {
        const bool ok = tid < P.nt;
        gam[tid] = ok ? graw[(size_t)(P.t0 + tid) * hv + h] : 0.0f;
        bet[tid] = ok ? gate[(size_t)(P.t0 + tid) * hv + h].y : 0.0f;
    }
    __syncthreads();
    if (tid == 0) {                    // cumulative log decay, in token order
        float acc = 0.0f;
        for (int t = 0; t < C; t++) {
            acc = acc + gam[t];
            gam[t] = acc;
        }
    }
    __syncthreads();
    float *F = Fb + (size_t)blockIdx.x * 2 * C;
    if (tid < C) {
        Gs[tid] = exp_fast(gam[tid]);
        F[tid] = Gs[tid];
        F[C + tid] = exp_fast(gam[C - 1] - gam[tid]);
    }

    // K K^T (row block w) and Q K^T (row block 3-w): lower-triangle tiles
    const int r16 = lane & 15, kq = (lane >> 4) * 4;
    float *A = Ab + (size_t)blockIdx.x * C * C;
    for (int pass = 0; pass < 2; pass++) {
        const int rb = pass == 0 ? wave : 3 - wave;
        const float *X = pass == 0 ? Ks : Qs;
        for (int cb = 0; cb <= rb; cb++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k0 = 0; k0 < DK; k0 += 16)
                acc = mfma_k16(lds4(X + (rb * 16 + r16) * KP + k0 + kq),
                               lds4(Ks + (cb * 16 + r16) * KP + k0 + kq), acc);
            const int s = cb * 16 + r16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = rb * 16 + kq + i;
                if (pass == 0) {
                    Ls[t * CP + s] = s < t ? bet[t] * (exp_fast(gam[t] - gam[s]) * acc[i]) : 0.0f;
                } else {
                    A[t * C + s] = s <= t ? exp_fast(gam[t] - gam[s]) * acc[i] : 0.0f;
                }
            }
        }
    }
    __syncthreads();

    // forward substitution: X_t = R_t - sum_{s<t} L[t][s] X_s for the 256
    // right-hand-side columns [b V | b G K], one per thread
    float x[C];
    if (tid < DV) {
        const uint16_t *vp = vconv + (size_t)P.t0 * vd + (size_t)h * DV + tid;
#pragma unroll
        for (int t = 0; t < C; t++)
            x[t] = t < P.nt ? bet[t] * bf2f(vp[(size_t)t * vd]) : 0.0f;
    } else {
#pragma unroll
        for (int t = 0; t < C; t++)
            x[t] = (bet[t] * Gs[t]) * Ks[t * KP + (tid - DV)];
    }
#pragma unroll
    for (int t = 1; t < C; t++) {
        float acc = x[t];
#pragma unroll
        for (int s0 = 0; s0 < t; s0 += 4) {
            const float4 l4 = lds4(Ls + t * CP + s0);
            acc = fmaf(-l4.x, x[s0], acc);
            if (s0 + 1 < t) acc = fmaf(-l4.y, x[s0 + 1], acc);
            if (s0 + 2 < t) acc = fmaf(-l4.z, x[s0 + 2], acc);
            if (s0 + 3 < t) acc = fmaf(-l4.w, x[s0 + 3], acc);
        }
        x[t] = acc;
    }
    float *out = (tid < DV ? Ub : Wb) + (size_t)blockIdx.x * C * DV + (tid & (DV - 1));
#pragma unroll
    for (int t = 0; t < C; t++) out[t * DV] = x[t];
}

// Chunk-to-chunk scan of one 16-column slice of one head's state.
// Block index = cb * (B*hv) + (s*hv + h): the 8 slices of a head share
// their U/W/A/Q/K reads, and with B*hv a multiple of 8 they land on the
// same XCD (blocks are dealt round-robin over the 8 XCDs) and so share
// its L2.
__global__ __launch_bounds__(256) void k_gdn_chunk_scan(
    ChunkSeqs sq, const int32_t *__restrict__ dmeta, const float *__restrict__ qk,
    const float *__restrict__ Ub, const float *__restrict__ Wb,
    const float *__restrict__ Ab, const float *__restrict__ Fb, float *__restrict__ S,
    uint16_t *__restrict__ ob, int hk) {
    const int hv = hk * REP;
    const size_t kd = (size_t)hk * DK, vd = (size_t)hv * DV;
    const int nsh = sq.n * hv;
    const int cb = blockIdx.x / nsh, sh = blockIdx.x % nsh;
    const int s = sh / hv, h = sh % hv, kh = h / REP;
    const int32_t *cu = dmeta ? dmeta : sq.cu;
    const int32_t *coff = dmeta ? dmeta + sq.n + 1 : sq.coff;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, kq = (lane >> 4) * 4;

    __shared__ __attribute__((aligned(16))) float KT[DK * CP];     // K^T of the chunk
    __shared__ __attribute__((aligned(16))) float S0T[CB * KP];    // S slice, [col][row]
    __shared__ __attribute__((aligned(16))) float DT[CB * CP];     // D slice, [col][t]
    __shared__ __attribute__((aligned(16))) float DpT[CB * CP];    // decayed D
    __shared__ float Fs[2 * C];

    // state slice in: packed layout ((j/64*32 + i/4)*64 + j%64)*4 + i%4
    float *Sm = S + (size_t)sh * DK * DV;
    const int jb = (cb * CB) / 64 * 32, jl = (cb * CB) % 64;
    for (int e = tid; e < CB * DK; e += 256) {
        const int q = e / 64, rem = e % 64, jj = rem / 4, r = rem % 4;
        S0T[jj * KP + 4 * q + r] = Sm[((size_t)(jb + q) * 64 + jl + jj) * 4 + r];
    }

    const int c0 = coff[s], c1 = coff[s + 1];
    for (int ci = c0; ci < c1; ci++) {
        const int t0 = cu[s] + (ci - c0) * C, nt = min(C, cu[s + 1] - t0);
        const size_t u = (size_t)ci * hv + h;
        __syncthreads();               // previous step done with KT/Fs/S0T
        for (int e = tid; e < C * DK / 4; e += 256) {
            const int t = e % C, q4 = (e / C) * 4;
            float4 k = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < nt) k = ld4(qk + (size_t)(t0 + t) * 2 * kd + kd + (size_t)kh * DK + q4);
            KT[(q4 + 0) * CP + t] = k.x;
            KT[(q4 + 1) * CP + t] = k.y;
            KT[(q4 + 2) * CP + t] = k.z;
            KT[(q4 + 3) * CP + t] = k.w;
        }
        if (tid < 2 * C) Fs[tid] = Fb[u * 2 * C + tid];
        __syncthreads();

        // D rows [16w, 16w+16) of this slice: U - W S0
        const int rw = wave * 16;
        const float *W = Wb + (u * C + rw + r16) * DK;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < DK; k0 += 16)
            acc = mfma_k16(ld4(W + k0 + kq), lds4(S0T + r16 * KP + k0 + kq), acc);
        const float *U = Ub + u * C * DV + cb * CB + r16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = rw + kq + i;
            const float d = U[(size_t)t * DV] - acc[i];
            DT[r16 * CP + t] = d;
            DpT[r16 * CP + t] = Fs[C + t] * d;
        }
        // O rows: G_t (Q S0) ...
        const int tq = rw + r16;
        const float *Q = qk + (size_t)(t0 + tq) * 2 * kd + (size_t)kh * DK;
        // (MFMA is a whole-wave operation: padding rows get zero operands,
        // never a branch around the instruction)
        float4 qa[DK / 16];
#pragma unroll
        for (int k = 0; k < DK / 16; k++)
            qa[k] = tq < nt ? ld4(Q + k * 16 + kq) : make_float4(0.f, 0.f, 0.f, 0.f);
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < DK / 16; k++)
            o = mfma_k16(qa[k], lds4(S0T + r16 * KP + k * 16 + kq), o);
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = Fs[rw + kq + i] * o[i];
        __syncthreads();               // D complete

        // ... + A D over the causal part s < 16(w+1)
        const float *Ar = Ab + (u * C + rw + r16) * C;
        for (int k0 = 0; k0 < rw + 16; k0 += 16)
            o = mfma_k16(ld4(Ar + k0 + kq), lds4(DT + r16 * CP + k0 + kq), o);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = rw + kq + i;
            if (t < nt) ob[(size_t)(t0 + t) * vd + (size_t)h * DV + cb * CB + r16] = f2bf(o[i]);
        }

        // S1 rows [32w, 32w+32): G_C S0 + K^T Dp
        const float gc = Fs[C - 1];
        f32x4 sn[2];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i0 = wave * 32 + r * 16;
#pragma unroll
            for (int i = 0; i < 4; i++) sn[r][i] = gc * S0T[r16 * KP + i0 + kq + i];
#pragma unroll
            for (int k0 = 0; k0 < C; k0 += 16)
                sn[r] = mfma_k16(lds4(KT + (i0 + r16) * CP + k0 + kq),
                                 lds4(DpT + r16 * CP + k0 + kq), sn[r]);
        }
        __syncthreads();               // every reader of S0T is done
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int i0 = wave * 32 + r * 16;
#pragma unroll
            for (int i = 0; i < 4; i++) S0T[r16 * KP + i0 + kq + i] = sn[r][i];
        }
    }
    __syncthreads();
    for (int e = tid; e < CB * DK; e += 256) {
        const int q = e / 64, rem = e % 64, jj = rem / 4, r = rem % 4;
        Sm[((size_t)(jb + q) * 64 + jl + jj) * 4 + r] = S0T[jj * KP + 4 * q + r];
    }
}

}  // namespace

extern "C" {

int apus_hip_gdn_prefill(const ApusHipGdnLayer *L, size_t B, const int32_t *cu,
                         const uint16_t *qkv, const uint16_t *z, const uint16_t *a,
                         const uint16_t *b, uint16_t *conv_state, float *S, uint16_t *y) {
    APUS_READY();
    if (int r = gdn_check_layer(L)) return r;
    if (B == 0) return kOk;
    if (int r = gdn_check_offsets(B, cu)) return r;
    const size_t Ttot = (size_t)cu[B];
    if (Ttot == 0) return kOk;
    if (B * L->hv * NCB > 0x7fffffffu) return set_error(kErrArgument, "batch too large");

    // metadata: [cu | chunk offsets], uploaded (k_gdn_prep/post read the
    // device copy) and, for small batches, also passed by value
    std::vector<int32_t> meta(2 * (B + 1));
    memcpy(meta.data(), cu, (B + 1) * 4);
    int32_t *coff = meta.data() + B + 1;
    coff[0] = 0;
    for (size_t s = 0; s < B; s++) coff[s + 1] = coff[s] + (cu[s + 1] - cu[s] + C - 1) / C;
    const size_t nch = (size_t)coff[B];
    ChunkSeqs sq;
    sq.n = (int32_t)B;
    const int32_t *dmeta, *kmeta;
    if (B <= (size_t)kPrefillInline) {
        memcpy(sq.cu, cu, (B + 1) * 4);
        memcpy(sq.coff, coff, (B + 1) * 4);
        int32_t *m = (int32_t *)scratch(kScratchMeta3, meta.size() * 4);
        if (!m) return kErrHip;
        k_prefill_meta<<<1, 256, 0, stream()>>>(sq, m);
        APUS_LAUNCHED("k_prefill_meta");
        dmeta = m;
        kmeta = nullptr;
    } else {
        dmeta = (const int32_t *)upload_small(kScratchMeta, meta.data(), meta.size() * 4);
        if (!dmeta) return kErrHip;
        kmeta = dmeta;
    }

    GdnScratch w;
    if (int r = gdn_prep(L, B, dmeta, Ttot, qkv, a, b, conv_state, &w, true)) return r;
    const size_t units = nch * L->hv;
    float *Ub = (float *)scratch(kScratchGdnChunk, units * C * DV * 4);
    float *Wb = (float *)scratch(kScratchGdnChunk2, units * C * DK * 4);
    float *Ab = (float *)scratch(kScratchGdnChunk4, units * C * C * 4);
    float *Fb = (float *)scratch(kScratchGdnChunk5, units * 2 * C * 4);
    if (!Ub || !Wb || !Ab || !Fb) return kErrHip;
    APUS_TIMED("k_gdn_chunk_wy",
               k_gdn_chunk_wy<<<(unsigned)units, 256, 0, stream()>>>(
        sq, kmeta, w.qk, w.vconv, w.gate, w.graw, Ub, Wb, Ab, Fb, (int)L->hk));
    APUS_LAUNCHED("k_gdn_chunk_wy");
    APUS_TIMED("k_gdn_chunk_scan",
               k_gdn_chunk_scan<<<(unsigned)(B * L->hv * NCB), 256, 0, stream()>>>(
        sq, kmeta, w.qk, Ub, Wb, Ab, Fb, S, w.ob, (int)L->hk));
    APUS_LAUNCHED("k_gdn_chunk_scan");
    return gdn_post(L, B, dmeta, Ttot, &w, z, qkv, conv_state, y);
}

}  // extern "C"
