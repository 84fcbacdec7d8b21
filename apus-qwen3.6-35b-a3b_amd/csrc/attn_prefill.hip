// attn_prefill.hip -- gated-GQA causal prefill for gfx950: the op sequence
// of c/layer.h:498-564 (q/k (1+w) RMSNorm, partial RoPE, KV-cache append,
// causal GQA over the cache, sigmoid output gate) for B sequences of any
// length, with the attention as an MFMA flash-attention kernel.
//
// k_attn_fa: one workgroup per (16-token query tile, kv head), tiles
// dealt longest first. The 8 q heads of the kv head x 16 tokens are 128
// query rows; wavefront w owns tokens 4w..4w+3 (32 rows: one MFMA N-tile).
// Key tiles of 32 (K rows and the cache's 32-key transposed V block) are
// staged in LDS, the next one prefetched into registers. Two passes over
// the keys:
//   pass 1: S^T = K Q^T on MFMA 32x32x16 bf16 (fp32 accumulation); with
//           keys on the M side each lane holds 16 keys of ONE query, so
//           the row max / sum need one exchange between the lane halves.
//           A = rnd(rnd(q.k) * scale) as the reference rounds it
//           (c/attn.h:340-347), causal mask key <= query; running max m
//           and sum s = sum_j e^{A_j - m} per query;
//   pass 2: S^T again, then the reference's normalised probabilities
//           P = rnd(e^{A-m} / s) (c/attn.h:354-360) in bf16, straight from
//           the S^T accumulator registers into O^T += V^T P^T on MFMA (the
//           key order each lane half holds is the reduction order both
//           operands use).
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
constexpr int TQ = 16;                 // query tokens per workgroup
constexpr int KT = 32;                 // keys per tile
constexpr int KSTR = D + 8;            // K tile row stride (bf16)
constexpr int VSTR = KT + 4;           // V^T tile row stride (bf16)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

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

// e^x for the softmax, x <= 0: the hardware exp2 of x*log2(e) (about two
// ulp; the result is rounded to a bf16 probability, so this stays inside
// the tolerance class; exp2(-inf) = 0)
__device__ __forceinline__ float exp_sm(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// Key-tile staging: 16-byte pieces e = r*256 + tid, K rows (key e/32,
// dims (e%32)*8..) and the V^T block ([d][32 keys], contiguous in the
// cache: piece e is d = e/4, keys (e%4)*8..). Keys at or past nkeys are
// zeroed in LDS (never read unwritten cache memory into the sums).
__device__ __forceinline__ void fa_load_k(u16x8 (&pk)[4], const uint16_t *__restrict__ kc,
                                          int kb, int tid) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = r * 256 + tid;
        const int key = e / (D / 8), c8 = (e % (D / 8)) * 8;
        pk[r] = *reinterpret_cast<const u16x8 *>(kc + (size_t)(kb * KT + key) * D + c8);
    }
}

__device__ __forceinline__ void fa_load_v(u16x8 (&pv)[4], const uint16_t *__restrict__ vc,
                                          int kb, int tid) {
#pragma unroll
    for (int r = 0; r < 4; r++)
        pv[r] = *reinterpret_cast<const u16x8 *>(vc + (size_t)kb * D * KT + (size_t)(r * 256 + tid) * 8);
}

__device__ __forceinline__ void fa_store_k(uint16_t *Ks, const u16x8 (&pk)[4], int kbase,
                                           int nkeys, int tid) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = r * 256 + tid;
        const int key = e / (D / 8), c8 = (e % (D / 8)) * 8;
        u16x8 kv = pk[r];
        if (kbase + key >= nkeys) kv = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        *reinterpret_cast<u16x8 *>(Ks + key * KSTR + c8) = kv;
    }
}

__device__ __forceinline__ void fa_store_v(uint16_t *Vs, const u16x8 (&pv)[4], int kbase,
                                           int nkeys, int tid) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = r * 256 + tid;
        const int d = e / 4, k8 = (e % 4) * 8;
        u16x8 vv = pv[r];
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (kbase + k8 + i >= nkeys) vv[i] = 0;
        uint32_t *dst = reinterpret_cast<uint32_t *>(Vs + d * VSTR + k8);
        *reinterpret_cast<uint2 *>(dst) = make_uint2((uint32_t)vv[0] | ((uint32_t)vv[1] << 16),
                                                     (uint32_t)vv[2] | ((uint32_t)vv[3] << 16));
        *reinterpret_cast<uint2 *>(dst + 2) =
            make_uint2((uint32_t)vv[4] | ((uint32_t)vv[5] << 16),
                       (uint32_t)vv[6] | ((uint32_t)vv[7] << 16));
    }
}

// Scores of one key tile for this lane's query, in two parts so the
// callers can interleave them with other work: fa_qk runs S^T = K Q^T on
// MFMA (two accumulation chains, even / odd 16-dim steps, the K operands
// of step pair p+1 read while pair p is on the MFMA pipe), fa_round turns
// it into A = rnd(rnd(q.k) * scale) for keys kbase + 8*(i/4) + 4h + i%4
// <= qpos, -inf beyond (the compare only on tiles that reach the diagonal
// of the wavefront's queries).
__device__ __forceinline__ void fa_qk(f32x16 &sc0, f32x16 &sc1, const uint16_t *Ks,
                                      const bf16x8 (&qb)[D / 16], int l32, int h) {
#pragma unroll
    for (int i = 0; i < 16; i++) { sc0[i] = 0.0f; sc1[i] = 0.0f; }
    const uint16_t *kr = Ks + l32 * KSTR + h * 8;
    bf16x8 k0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(kr));
    bf16x8 k1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(kr + 16));
#pragma unroll
    for (int ks = 0; ks < D / 16; ks += 2) {
        bf16x8 n0 = k0, n1 = k1;
        if (ks + 2 < D / 16) {
            n0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(kr + (ks + 2) * 16));
            n1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(kr + (ks + 3) * 16));
        }
        sc0 = mfma32(k0, qb[ks], sc0);
        sc1 = mfma32(k1, qb[ks + 1], sc1);
        k0 = n0;
        k1 = n1;
    }
}

__device__ __forceinline__ void fa_round(float (&a)[16], const f32x16 &sc0, const f32x16 &sc1,
                                         int kbase, int qpos, int qmin, float scale, int h) {
    if (kbase + KT - 1 <= qmin) {      // wave-uniform: no key of the tile is masked
#pragma unroll
        for (int i = 0; i < 16; i++) a[i] = rnd_hw(rnd_hw(sc0[i] + sc1[i]) * scale);
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int key = kbase + 8 * (i / 4) + 4 * h + (i % 4);
            a[i] = key <= qpos ? rnd_hw(rnd_hw(sc0[i] + sc1[i]) * scale) : -INFINITY;
        }
    }
}

// order of one S^T computation: reads of pairs 0 and 1, then (MFMA pair p,
// VALU from the caller, reads of pair p+2)
template <int VALU_PER_PAIR>
__device__ __forceinline__ void fa_qk_schedule() {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);       // LDS reads
#pragma unroll
    for (int g = 0; g < D / 32 - 2; g++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, VALU_PER_PAIR, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // LDS reads
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, VALU_PER_PAIR, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
}

__global__ __launch_bounds__(256) void k_attn_fa(
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
    const int s = seq_of(toff, n, g);
    const int tb = cu[s] + (g - toff[s]) * TQ;             // first token of the tile
    const int nt = min(TQ, cu[s + 1] - tb);
    const int qpos0 = pos0[s] + (tb - cu[s]);              // its position
    const int nkeys = qpos0 + nt;
    const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // K tiles double buffered, V tiles triple buffered: with one barrier
    // per key tile (after the staging writes), a buffer is rewritten only
    // after every wavefront has passed a later barrier than its last reader
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][KT * KSTR];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[3][D * VSTR];

    const uint16_t *kc = kcache + ((size_t)s * nkv + kvh) * max_seq * D;
    const uint16_t *vc = vcache + ((size_t)s * nkv + kvh) * D * max_seq;

    // query row of this lane: token 4w + l32/8, head l32%8 of the kv head
    const int tk = wave * 4 + l32 / GRP, head = kvh * GRP + l32 % GRP;
    const bool qok = tk < nt;
    const int qtok = tb + min(tk, nt - 1);
    const int qpos = qpos0 + tk;
    const int qmin = qpos0 + wave * 4;          // smallest query position of the wavefront
    bf16x8 qb[D / 16];
    {
        const uint16_t *qr = qn + ((size_t)qtok * nh + head) * D + h * 8;
#pragma unroll
        for (int ks = 0; ks < D / 16; ks++)
            qb[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(qr + ks * 16));
    }
    const int nkt = (nkeys + KT - 1) / KT;
    u16x8 pk[4], pv[4];

    // ---- pass 1: per-query max m and sum s over all keys. Iteration kb
    // stages tile kb+1, then scores it on MFMA while the VALU folds tile
    // kb into (m, s).
    float m = -INFINITY, lsum = 0.0f;
    float a[16];
    fa_load_k(pk, kc, 0, tid);
    fa_store_k(Ks[0], pk, 0, nkeys, tid);
    if (nkt > 1) fa_load_k(pk, kc, 1, tid);
    __syncthreads();
    {
        f32x16 s0, s1;
        fa_qk(s0, s1, Ks[0], qb, l32, h);
        fa_round(a, s0, s1, 0, qpos, qmin, scale, h);
    }
    for (int kb = 0; kb < nkt; kb++) {
        const bool more = kb + 1 < nkt;
        if (more) {
            fa_store_k(Ks[(kb + 1) & 1], pk, (kb + 1) * KT, nkeys, tid);
            if (kb + 2 < nkt) fa_load_k(pk, kc, kb + 2, tid);
        }
        __syncthreads();
        // next tile's S^T (past the last tile it reads a stale buffer and is
        // discarded) interleaved with folding tile kb into (m, s)
        f32x16 s0, s1;
        fa_qk(s0, s1, Ks[(kb + 1) & 1], qb, l32, h);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) mx = fmaxf(mx, a[i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) ps += exp_sm(a[i] - mn);
        ps += __shfl_xor(ps, 32);
        lsum = lsum * exp_sm(m - mn) + ps;     // exp(-inf) = 0 on the first tile
        m = mn;
        fa_round(a, s0, s1, (kb + 1) * KT, qpos, qmin, scale, h);
        fa_qk_schedule<10>();
    }

    // ---- pass 2: P = rnd(e^{A-m} / s), O^T += V^T P^T (e times 1/s: a
    // different fp32 quotient only when the two straddle a bf16 rounding
    // boundary). Iteration kb stages tile kb+1, scores it, and turns tile
    // kb's scores into P for the P.V MFMAs.
    const float inv_s = 1.0f / lsum;
    f32x16 o[D / 32];
#pragma unroll
    for (int mt = 0; mt < D / 32; mt++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[mt][i] = 0.0f;
    __syncthreads();                   // pass 1 is done with Ks
    fa_load_k(pk, kc, 0, tid);
    fa_load_v(pv, vc, 0, tid);
    fa_store_k(Ks[0], pk, 0, nkeys, tid);
    fa_store_v(Vs[0], pv, 0, nkeys, tid);
    if (nkt > 1) {
        fa_load_k(pk, kc, 1, tid);
        fa_load_v(pv, vc, 1, tid);
    }
    __syncthreads();
    {
        f32x16 s0, s1;
        fa_qk(s0, s1, Ks[0], qb, l32, h);
        fa_round(a, s0, s1, 0, qpos, qmin, scale, h);
    }
    for (int kb = 0; kb < nkt; kb++) {
        const bool more = kb + 1 < nkt;
        if (more) {
            fa_store_k(Ks[(kb + 1) & 1], pk, (kb + 1) * KT, nkeys, tid);
            fa_store_v(Vs[(kb + 1) % 3], pv, (kb + 1) * KT, nkeys, tid);
            if (kb + 2 < nkt) {
                fa_load_k(pk, kc, kb + 2, tid);
                fa_load_v(pv, vc, kb + 2, tid);
            }
        }
        __syncthreads();
        // next tile's S^T interleaved with tile kb's probabilities, then
        // tile kb's P.V interleaved with the next tile's score rounding
        f32x16 s0, s1;
        fa_qk(s0, s1, Ks[(kb + 1) & 1], qb, l32, h);
        uint32_t pp[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            pp[i] = pack2(exp_sm(a[2 * i] - m) * inv_s, exp_sm(a[2 * i + 1] - m) * inv_s);
        fa_qk_schedule<8>();
        const uint16_t *Vb = Vs[kb % 3];
        // step st covers keys st*16 + {4h..4h+3, 8+4h..8+4h+3}; the V^T
        // operand of MFMA j+1 is read while MFMA j runs
        const uint16_t *vr0 = Vb + l32 * VSTR + 4 * h;
        uint2 vlo = *reinterpret_cast<const uint2 *>(vr0);
        uint2 vhi = *reinterpret_cast<const uint2 *>(vr0 + 8);
#pragma unroll
        for (int j = 0; j < 2 * (D / 32); j++) {
            const int st = j / (D / 32), mt = j % (D / 32);
            uint2 nlo = vlo, nhi = vhi;
            if (j + 1 < 2 * (D / 32)) {
                const int st1 = (j + 1) / (D / 32), mt1 = (j + 1) % (D / 32);
                const uint16_t *vr = vr0 + mt1 * 32 * VSTR + st1 * 16;
                nlo = *reinterpret_cast<const uint2 *>(vr);
                nhi = *reinterpret_cast<const uint2 *>(vr + 8);
            }
            const uint32_t w4[4] = {pp[4 * st], pp[4 * st + 1], pp[4 * st + 2], pp[4 * st + 3]};
            const bf16x8 pb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(w4));
            const uint32_t v4[4] = {vlo.x, vlo.y, vhi.x, vhi.y};
            const bf16x8 va = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(v4));
            o[mt] = mfma32(va, pb, o[mt]);
            vlo = nlo;
            vhi = nhi;
        }
        fa_round(a, s0, s1, (kb + 1) * KT, qpos, qmin, scale, h);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // LDS reads
#pragma unroll
        for (int j = 0; j < 2 * (D / 32) - 2; j++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // LDS reads
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
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
    if (max_seq % KT != 0) return set_error(kErrArgument, "max_seq must be a multiple of %d", KT);
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
               k_attn_fa<<<(unsigned)(ntiles * L->nkv), 256, 0, stream()>>>(
                   fs, fdm, qn, qg, kcache, vcache, max_seq, (int)L->nh, (int)L->nkv, scale, y,
                   tabs->sig_bf));
    APUS_LAUNCHED("k_attn_fa");
    return kOk;
}

}  // extern "C"
