// attn_prefill.hip -- gated-GQA causal prefill for gfx950: the op sequence
// of c/layer.h:498-564 (q/k (1+w) RMSNorm, partial RoPE, KV-cache append,
// causal GQA over the cache, sigmoid output gate) for B sequences of any
// length, with the attention as an MFMA flash-attention kernel.
//
// k_attn_fa: one workgroup of 8 wavefronts (two per SIMD) per (32-token
// query tile, kv head), tiles dealt longest first. The 8 q heads of the
// kv head x 32 tokens are 256 query rows; wavefront w owns tokens
// 4w..4w+3 (32 rows: one MFMA N-tile), its Q rows held in registers.
// Key tiles of 64 (K rows and the cache's two 32-key transposed V blocks)
// are copied global -> LDS by the DMA path (global_load_lds, 16 bytes a
// lane), the next tile's copy in flight while the current one is used;
// one barrier per tile. Two passes over the keys:
//   pass 1: S^T = K Q^T on MFMA 32x32x16 bf16 (fp32 accumulation); with
//           keys on the M side each lane holds 16 keys of ONE query, so
//           the row max / sum need one exchange between the lane halves
//           (v_permlane32_swap). A = rnd(rnd(q.k) * scale) as the
//           reference rounds it (c/attn.h:340-347), causal mask key <=
//           query; running max m and sum s = sum_j e^{A_j - m} per query;
//   pass 2: S^T again, then the reference's normalised probabilities
//           P = rnd(e^{A-m} / s) (c/attn.h:354-360) in bf16, straight from
//           the S^T accumulator registers into O^T += V^T P^T on MFMA.
// The A-operand row m of S^T is key pi(m) = 16(m/16) + 8((m/4)%2) +
// 4((m/8)%2) + m%4 of the 32-key step, chosen so that the 8 probabilities
// a lane feeds to each P.V MFMA are 8 consecutive keys: the V^T operand
// is then one 16-byte piece of the V block.
// LDS pieces are XOR-swizzled (16-byte piece c of K row r at c ^ (r%16);
// of V^T row r at c ^ ((r/4)%4)) so that the MFMA operand reads of 16
// lanes hit 16 distinct 16-byte bank groups.
// Epilogue: o = rnd(O), y = rnd(o * rnd(sigmoid(gate))) (c/attn.h:524-531).
//
// Numerics: P is the reference's rounding point, so only the MFMA
// summation order of q.k and P.V and libm ulps in e^x differ (the
// tolerance class of the decode kernel): |c - r| <= 2e-3 (|r| + esc),
// esc = sum_j |P_j V_j| (the reference's own form, tests/m4a/README.md).
// A single-pass online softmax rounds e^{A - m_running} before the final
// normalisation instead, which measurably exceeds that bound.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"
#include "attn_mixer.h"

using namespace apus;

namespace {

constexpr int D = 256, GRP = 8;
constexpr int NW = 8;                  // wavefronts per workgroup
constexpr int TQ = 4 * NW;             // query tokens per workgroup
constexpr int KT = 64;                 // keys per tile
constexpr int VB = 32;                 // keys per V^T block of the cache

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kFaInline = 300;
struct FaSeqs {
    int32_t n;
    int32_t cu[kFaInline + 1];
    int32_t pos0[kFaInline];
    int32_t toff[kFaInline + 1];       // query-tile offsets
};

__device__ __forceinline__ int seq_of(const int32_t *off, int n, int x) {
    int lo = 0, hi = n - 1;            // largest s with off[s] <= x
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= x) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Hardware round-to-nearest-even to bf16 (v_cvt_pk_bf16_f32): the same
// rounding as the reference's apus_bf16_bits for finite values.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}
__device__ __forceinline__ float rnd_hw(float x) { return (float)(__bf16)x; }

// max / sum of x over lanes l and l ^ 32, in both (v_permlane32_swap
// exchanges one half of its two operands; with both = x the two results
// hold x's two halves in some order, and max / + commute)
__device__ __forceinline__ float max32(float x) {
    const uint32_t u = __float_as_uint(x);
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float sum32(float x) {
    const uint32_t u = __float_as_uint(x);
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// one 16-byte global -> LDS copy per lane through a buffer resource:
// byte offset voff (per lane) + soff (uniform), LDS address = the
// wave-uniform base plus 16 * lane. Offsets past the resource's size read
// as zero.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, int voff, int soff,
                                      uint16_t *lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds_base, 16, voff, soff, 0, 0);
}

// K rows of tile kb -> Kb: wavefront w copies rows 8w..8w+7, two rows of
// 32 pieces per instruction. The resource ends at the last key, so rows
// past it are zero (and their scores masked).
__device__ __forceinline__ void fa_dma_k(uint16_t *Kb, __amdgpu_buffer_rsrc_t kr, int kb,
                                         int wave, int lane) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r0 = 8 * wave + 2 * j, r = r0 + (lane >> 5);
        const int c = (lane & 31) ^ (r & 15);
        dma16(kr, (r * D + c * 8) * 2, kb * KT * D * 2, Kb + r0 * D);
    }
}

// V^T blocks 2kb, 2kb+1 -> Vb ([block][d][32 keys]): wavefront w copies
// the 1 KiB groups 4w..4w+3 (16 d-rows of 4 pieces each). The resource
// ends at the last key's block; keys past the last one inside that block
// are zeroed in LDS before use.
__device__ __forceinline__ void fa_dma_v(uint16_t *Vb, __amdgpu_buffer_rsrc_t vr, int kb,
                                         int wave, int lane) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q = 4 * wave + j, bb = q >> 4, g = q & 15;
        const int r = 16 * g + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        dma16(vr, (bb * D * VB + r * VB + c * 8) * 2, kb * KT * D * 2,
              Vb + bb * D * VB + g * 16 * VB);
    }
}

// Per-lane LDS byte offsets of the MFMA operands. K operand of S^T step
// ks: row pi(l32) of the 32-key step, piece (2ks + h) ^ (row % 16), i.e.
// kbase ^ (ks << 5): the ks bits (5..8) are disjoint from the row bits
// (9..) and the h bit (4), so one base and one XOR per read suffice.
__device__ __forceinline__ int fa_kbase(int l32, int h) {
    const int m = l32;
    const int row = 16 * (m >> 4) + 8 * ((m >> 2) & 1) + 4 * ((m >> 3) & 1) + (m & 3);
    const int sw = row & 15;
    return row * D * 2 + (((h ^ sw) & 1) << 4) + ((sw & 14) << 4);
}
// V^T operand of P.V step st, d-tile mt: row 32mt + l32, piece
// (2st + h) ^ ((row / 4) % 4): vbase ^ (st << 5), plus mt * 2 KiB
__device__ __forceinline__ int fa_vbase(int l32, int h) {
    const int sw = (l32 >> 2) & 3;
    return l32 * VB * 2 + (((h ^ sw) & 1) << 4) + ((sw & 2) << 4);
}

// S^T of the 32 keys at byte offset koff of the K tile for this lane's
// query (element i <-> key 16(i/8) + 8h + i%8 of the step).
__device__ __forceinline__ f32x16 fa_qk(const char *Kb, int kbase, const bf16x8 (&qb)[D / 16]) {
    f32x16 sc;
#pragma unroll
    for (int i = 0; i < 16; i++) sc[i] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < D / 16; ks++) {
        const bf16x8 k =
            __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(Kb + (kbase ^ (ks << 5))));
        sc = mfma32(k, qb[ks], sc);
    }
    return sc;
}

// rnd(q.k) with the causal mask (-inf past the query), keys
// k0 + 16(i/8) + 8h + i%8; the compare only on steps that reach the
// wavefront's first query
__device__ __forceinline__ void fa_round(float (&r)[16], const f32x16 &sc, int k0, int qpos,
                                         int qmin, int h) {
    if (k0 + 31 <= qmin) {             // wave-uniform: no key of the step is masked
#pragma unroll
        for (int i = 0; i < 16; i++) r[i] = rnd_hw(sc[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int key = k0 + 16 * (i >> 3) + 8 * h + (i & 7);
            r[i] = key <= qpos ? rnd_hw(sc[i]) : -INFINITY;
        }
    }
}

// End of a step: this wavefront's copies have landed, then the barrier
// that publishes them. When the tile just copied is the last one (`last`)
// and the keys end inside a V block, its V entries past the last key are
// zeroed (P is 0 there, but 0 * NaN from unwritten cache memory would not
// be), behind a second barrier.
__device__ __forceinline__ void fa_sync(uint16_t *Vn, bool last, int nkeys, int tid) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (last && nkeys % VB != 0) {
        const int kbase = (nkeys - 1) / KT * KT;
        for (int e = tid; e < KT * D; e += 64 * NW) {
            const int bb = e / (D * VB), rem = e % (D * VB), row = rem / VB, kk = rem % VB;
            if (kbase + bb * VB + kk >= nkeys) {
                const int c = (kk >> 3) ^ ((row >> 2) & 3);
                Vn[bb * D * VB + row * VB + c * 8 + (kk & 7)] = 0;
            }
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(64 * NW) void k_attn_fa(
    FaSeqs sq, const int32_t *__restrict__ dmeta, const uint16_t *__restrict__ qn,
    const uint16_t *__restrict__ qg, const uint16_t *__restrict__ kcache,
    const uint16_t *__restrict__ vcache, size_t max_seq, int nh, int nkv, float scale,
    uint16_t *__restrict__ y, const uint16_t *__restrict__ sig_bf) {
    const int n = sq.n;
    const int32_t *cu = dmeta ? dmeta : sq.cu;
    const int32_t *pos0 = dmeta ? dmeta + n + 1 : sq.pos0;
    const int32_t *toff = dmeta ? dmeta + 2 * n + 1 : sq.toff;
    const int ntiles = toff[n];
    const int g = ntiles - 1 - (int)(blockIdx.x / nkv);
    const int kvh = blockIdx.x % nkv;
    // workgroup-uniform (loaded values are not provably so: readfirstlane
    // keeps the buffer resources in SGPRs)
    const int s = __builtin_amdgcn_readfirstlane(seq_of(toff, n, g));
    const int tb = __builtin_amdgcn_readfirstlane(cu[s] + (g - toff[s]) * TQ);  // first token
    const int nt = __builtin_amdgcn_readfirstlane(min(TQ, cu[s + 1] - tb));
    const int qpos0 = __builtin_amdgcn_readfirstlane(pos0[s] + (tb - cu[s]));  // its position
    const int nkeys = qpos0 + nt;
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][KT * D];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[2][KT * D];

    const uint16_t *kc = kcache + ((size_t)s * nkv + kvh) * max_seq * D;
    const uint16_t *vc = vcache + ((size_t)s * nkv + kvh) * D * max_seq;
    const int nkt = (nkeys + KT - 1) / KT;
    const int nblk = (nkeys + VB - 1) / VB;
    const __amdgpu_buffer_rsrc_t kr = buf_rsrc(kc, (uint32_t)nkeys * D * 2);
    const __amdgpu_buffer_rsrc_t vr = buf_rsrc(vc, (uint32_t)nblk * D * VB * 2);

    // first K tile in flight while Q is loaded
    fa_dma_k(Ks[0], kr, 0, wave, lane);

    // query row of this lane: token 4w + l32/8, head l32%8 of the kv head
    const int tk = wave * 4 + l32 / GRP, head = kvh * GRP + l32 % GRP;
    const bool qok = tk < nt;
    const int qtok = tb + min(tk, nt - 1);
    const int qpos = qpos0 + tk;
    const int qmin = qpos0 + wave * 4;          // the wavefront's first / last query position
    const int qmax = qmin + 3;
    bf16x8 qb[D / 16];
    {
        const uint16_t *qr = qn + ((size_t)qtok * nh + head) * D + h * 8;
#pragma unroll
        for (int ks = 0; ks < D / 16; ks++)
            qb[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(qr + ks * 16));
    }
    // (A - m) log2(e) = (rnd(q.k) - M) * scale * log2(e) with M = m / scale:
    // scale is a power of two, so this is the reference's A - m scaled
    const float c2 = scale * 1.44269504088896341f;

    f32x16 o[D / 32];
#pragma unroll
    for (int mt = 0; mt < D / 32; mt++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[mt][i] = 0.0f;
    float M = -INFINITY, lsum = 0.0f;

    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // pass 1: per-query max M (in units of rnd(q.k)) and sum s over all
    // keys; the last step also starts the copy of pass 2's first tile
    for (int kb = 0; kb < nkt; kb++) {
        const int buf = kb & 1;
        fa_dma_k(Ks[buf ^ 1], kr, kb + 1 < nkt ? kb + 1 : 0, wave, lane);
        if (kb + 1 == nkt) fa_dma_v(Vs[buf ^ 1], vr, 0, wave, lane);
        const char *Kb = reinterpret_cast<const char *>(Ks[buf]);
#pragma unroll
        for (int sub = 0; sub < KT / 32; sub++) {
            const int k0 = kb * KT + sub * 32;
            if (k0 <= qmax) {                  // wave-uniform: else every key is masked
                int kbase = fa_kbase(l32, h);
                asm volatile("" : "+v"(kbase));
                const f32x16 sc = fa_qk(Kb + sub * 32 * D * 2, kbase, qb);
                float r[16];
                fa_round(r, sc, k0, qpos, qmin, h);
                float mx = r[0];
#pragma unroll
                for (int i = 1; i < 16; i++) mx = fmaxf(mx, r[i]);
                mx = max32(mx);
                const float mn = fmaxf(M, mx);
                float ps = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; i++) ps += __builtin_amdgcn_exp2f((r[i] - mn) * c2);
                ps = sum32(ps);
                // first step: M = -inf, lsum = 0 (exp2(-inf) = 0)
                lsum = lsum * __builtin_amdgcn_exp2f((M - mn) * c2) + ps;
                M = mn;
            }
        }
        fa_sync(Vs[buf ^ 1], kb + 1 == nkt && nkt == 1, nkeys, tid);
    }
    const float inv_s = 1.0f / lsum;

    // pass 2: P = rnd(e^{A-m} / s), O^T += V^T P^T
    for (int kb = 0; kb < nkt; kb++) {
        const int buf = (nkt + kb) & 1;
        if (kb + 1 < nkt) {
            fa_dma_k(Ks[buf ^ 1], kr, kb + 1, wave, lane);
            fa_dma_v(Vs[buf ^ 1], vr, kb + 1, wave, lane);
        }
        const char *Kb = reinterpret_cast<const char *>(Ks[buf]);
        const char *Vb = reinterpret_cast<const char *>(Vs[buf]);
#pragma unroll
        for (int sub = 0; sub < KT / 32; sub++) {
            const int k0 = kb * KT + sub * 32;
            int kbase = fa_kbase(l32, h), vbase = fa_vbase(l32, h);
            asm volatile("" : "+v"(kbase), "+v"(vbase));
            const f32x16 sc = fa_qk(Kb + sub * 32 * D * 2, kbase, qb);
            float r[16];
            fa_round(r, sc, k0, qpos, qmin, h);
            uint32_t pp[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                pp[i] = pack2(__builtin_amdgcn_exp2f((r[2 * i] - M) * c2) * inv_s,
                              __builtin_amdgcn_exp2f((r[2 * i + 1] - M) * c2) * inv_s);
            const char *Vsub = Vb + sub * D * VB * 2;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const uint32_t w4[4] = {pp[4 * st], pp[4 * st + 1], pp[4 * st + 2],
                                        pp[4 * st + 3]};
                const bf16x8 pb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(w4));
                const char *Vst = Vsub + (vbase ^ (st << 5));
#pragma unroll
                for (int mt = 0; mt < D / 32; mt++) {
                    const bf16x8 va = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const u16x8 *>(Vst + mt * 32 * VB * 2));
                    o[mt] = mfma32(va, pb, o[mt]);
                }
            }
        }
        if (kb + 1 < nkt) fa_sync(Vs[buf ^ 1], kb + 2 == nkt, nkeys, tid);
    }

    // epilogue: o = rnd(O); y = rnd(o * rnd(sigmoid(gate)))
    if (qok) {
        const size_t row = (size_t)qtok * nh + head;
        const uint16_t *gr = qg + row * 2 * D + D;
        uint16_t *yr = y + row * D;
#pragma unroll
        for (int mt = 0; mt < D / 32; mt++) {
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const int d0 = mt * 32 + 8 * q4 + 4 * h;
                const u16x4 gv = *reinterpret_cast<const u16x4 *>(gr + d0);
                u16x4 out;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float ov = rndf(o[mt][4 * q4 + i]);
                    const float gs = bf2f(sig_bf[gv[i]]);     // rnd(sigmoid(gate))
                    out[i] = f2bf(ov * gs);
                }
                *reinterpret_cast<u16x4 *>(yr + d0) = out;
            }
        }
    }
}

}  // namespace

extern "C" {

int apus_hip_attn_prefill(const ApusHipAttnLayer *L, size_t B, const int32_t *cu,
                          const int32_t *pos0, const uint16_t *qg, const uint16_t *k,
                          const uint16_t *v, uint16_t *kcache, uint16_t *vcache,
                          size_t max_seq, uint16_t *y) {
    APUS_READY();
    if (int r = attn_check_layer(L)) return r;
    if (B == 0) return kOk;
    if (!cu || !pos0 || cu[0] != 0) return set_error(kErrArgument, "bad offsets");
    if (max_seq % VB != 0) return set_error(kErrArgument, "max_seq must be a multiple of %d", VB);
    if (L->nh != GRP * L->nkv)
        return set_error(kErrUnsupported, "prefill supports nh = %d * nkv", GRP);
    size_t max_pos = 0;
    std::vector<int32_t> meta(3 * B + 2);
    int32_t *mcu = meta.data(), *mpos = mcu + B + 1, *mtoff = mpos + B;
    mtoff[0] = 0;
    for (size_t s = 0; s < B; s++) {
        const int32_t ns = cu[s + 1] - cu[s];
        if (ns < 0) return set_error(kErrArgument, "token offsets must ascend");
        if (pos0[s] < 0 || (size_t)pos0[s] + (size_t)ns > max_seq)
            return set_error(kErrArgument, "sequence %zu overflows the cache (%d+%d > %zu)", s,
                             pos0[s], ns, max_seq);
        max_pos = std::max(max_pos, (size_t)pos0[s] + (size_t)ns);
        mtoff[s + 1] = mtoff[s] + (ns + TQ - 1) / TQ;
    }
    memcpy(mcu, cu, (B + 1) * 4);
    memcpy(mpos, pos0, B * 4);
    const size_t Ttot = (size_t)cu[B];
    if (Ttot == 0) return kOk;
    const size_t ntiles = (size_t)mtoff[B];

    // q/k norm + RoPE + cache append (shared with decode)
    AttnSeqs as;
    as.n = (int32_t)B;
    as.ks1 = as.ks2 = 0;
    const int32_t *adm = nullptr;
    FaSeqs fs;
    fs.n = (int32_t)B;
    const int32_t *fdm = nullptr;
    if (B <= (size_t)kAttnInlineSeqs) {
        memcpy(as.cu, cu, (B + 1) * 4);
        memcpy(as.pos0, pos0, B * 4);
    }
    if (B <= (size_t)kFaInline) {
        memcpy(fs.cu, cu, (B + 1) * 4);
        memcpy(fs.pos0, pos0, B * 4);
        memcpy(fs.toff, mtoff, (B + 1) * 4);
    }
    if (B > (size_t)kAttnInlineSeqs || B > (size_t)kFaInline) {
        // [cu | pos0 | toff] serves both (attn_prep reads cu and pos0 at the
        // same offsets)
        fdm = (const int32_t *)upload_small(kScratchMeta2, meta.data(), meta.size() * 4);
        if (!fdm) return kErrHip;
        if (B > (size_t)kAttnInlineSeqs) adm = fdm;
        if (B <= (size_t)kFaInline) fdm = nullptr;
    }
    uint16_t *qn = (uint16_t *)scratch(kScratchAttnQ, Ttot * L->nh * D * 2);
    if (!qn) return kErrHip;
    if (int r = attn_prep(L, as, adm, Ttot, max_pos, qg, k, v, kcache, vcache, max_seq, qn))
        return r;
    const float scale = (float)(1.0 / sqrt((double)L->d));
    const ActTables *tabs = act_tables();
    if (!tabs) return kErrHip;
    APUS_TIMED("k_attn_fa",
               k_attn_fa<<<(unsigned)(ntiles * L->nkv), 64 * NW, 0, stream()>>>(
                   fs, fdm, qn, qg, kcache, vcache, max_seq, (int)L->nh, (int)L->nkv, scale, y,
                   tabs->sig_bf));
    APUS_LAUNCHED("k_attn_fa");
    return kOk;
}

}  // extern "C"
