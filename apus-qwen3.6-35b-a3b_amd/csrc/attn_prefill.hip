// attn_prefill.hip -- gated-GQA causal prefill for gfx950: the op sequence
// of c/layer.h:498-564 (q/k (1+w) RMSNorm, partial RoPE, KV-cache append,
// causal GQA over the cache, sigmoid output gate) for B sequences of any
// length, with the attention as an MFMA flash-attention kernel.
//
// k_attn_fa: one workgroup of 8 wavefronts (two per SIMD) per (32-token
// query tile, kv head), tiles dealt longest first. The 8 q heads of the
// kv head x 32 tokens are 256 query rows; wavefront w owns tokens
// 4w..4w+3 (32 rows: one MFMA N-tile), its Q rows held in registers. It
// forms those rows itself from the layer input ((1+w) RMSNorm, RoPE);
// k_attn_prep forms the k rows and appends k and v to the cache.
//
// The attention runs over the keys twice:
//   pass 1: S^T = K Q^T on MFMA 32x32x16 bf16 (fp32 accumulation); with
//           keys on the M side each lane holds 16 keys of ONE query, so
//           the row max / sum need one exchange between the lane halves
//           (v_permlane32_swap). A = rnd(rnd(q.k) * scale) as the
//           reference rounds it (c/attn.h:340-347), causal mask key <=
//           query; a reference point m and sum s = sum_j e^{A_j - m} per
//           query, m a running max that is raised only when the sum would
//           leave the fp32 range (s e^{m} and so P do not depend on m);
//   pass 2: S^T again, then the reference's normalised probabilities
//           P = rnd(e^{A-m} / s) (c/attn.h:354-360) in bf16, straight from
//           the S^T accumulator registers into O^T += V^T P^T on MFMA.
// Each pass is a software pipeline over 32-key steps that keeps the MFMA
// pipe fed while the softmax runs on the VALU: in pass 1 step j issues
// the MFMAs of S(j+1) interleaved with the sum fold of S(j); in
// pass 2 step j computes S(j), then the MFMAs of P(j-1).V(j-1)
// interleaved with forming P(j) (one set of scores and one of packed
// probabilities live at a time: the O^T accumulators take half of the
// wavefront's 256 registers).
//
// Keys arrive in tiles of 64 (K rows and the cache's two 32-key
// transposed V blocks), copied global -> LDS by buffer DMA (16 bytes a
// lane), one tile ahead, with one barrier per tile. A pass-2 tile's steps
// read its K and V and the previous tile's V, so K is double and V triple
// buffered (5 x 32 KiB, all of LDS). The DMA is issued as inline assembly
// with explicit waits: the compiler would otherwise make every LDS read
// wait for the copy in flight into another buffer.
//
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
constexpr int NW = 8;                  // wavefronts per workgroup, two per SIMD
constexpr int TQ = 4 * NW;             // query tokens per workgroup
constexpr int KT = 64;                 // keys per tile
constexpr int VB = 32;                 // keys per V^T block of the cache
constexpr int KROW = D * 2 + 16;       // K row pitch in LDS (one 16-byte pad)
constexpr int KBUF = KT * KROW;        // one K tile in LDS
constexpr int KHALF = 32 * KROW;       // its second 32 keys
constexpr int VHALF = 32 * D * 2;      // one 32-key V^T block in LDS

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));

constexpr int kFaInline = 224;
struct FaSeqs {
    int32_t n;
    int32_t cu[kFaInline + 1];
    int32_t pos0[kFaInline];
    int32_t toff[kFaInline + 1];       // query-tile offsets
    int32_t hd[kFaInline];             // block-table rows
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

// the lane index, opaque to the compiler: values derived from it are
// formed where they are used rather than hoisted and held in registers
// across the key loop (registers are the binding resource here)
__device__ __forceinline__ int fa_lane() {
    int l = __lane_id();
    asm volatile("" : "+v"(l));
    return l;
}

// K rows of key tile kt -> the K buffer at LDS address kb (row pitch
// KROW): copy part p is tile rows 8p..8p+7, one row (32 pieces, lanes
// 0..31) per instruction, from cache block 2kt + p/4 (its rows
// 8(p%4)..+7) at byte offset soff of the resource kr, which ends at the
// last key: rows past it read zero (and their scores are masked).
__device__ __forceinline__ void fa_dma_k(uint32_t kb, i32x4 kr, int soff, int part) {
    const int lane = fa_lane();
    if (lane < 32) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int r = 8 * part + j, rb = 8 * (part & 3) + j;
            dma16(kr, (rb * D + lane * 8) * 2, soff, kb + r * KROW);
        }
    }
}

// V^T blocks 2kt, 2kt+1 -> the LDS blocks at vb0, vb1 ([d][32 keys]):
// copy part p is the 1 KiB groups 4p..4p+3 of block p / 4 (16 d-rows
// of 4 pieces each) from the cache block at byte offset soff of vr (a
// block past the last key lies past the resource's end: it reads zero). Keys past the last one inside its
// block are zeroed in LDS before use.
__device__ __forceinline__ void fa_dma_v(uint32_t vb0, uint32_t vb1, i32x4 vr, int soff, int part) {
    const int lane = fa_lane();
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q = 4 * part + j, bb = q >> 4, g = q & 15;
        const int r = 16 * g + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        dma16(vr, (r * VB + c * 8) * 2, soff, (bb ? vb1 : vb0) + g * 16 * VB * 2);
    }
}

// Per-lane LDS byte offsets of the MFMA operands. K operand of S^T step
// ks: row pi(l32) of the 32-key step, piece 2ks + h: kbase + 32 ks (an
// immediate offset). The 16-byte pad per K row puts the 16 rows one read
// covers in 16 distinct 16-byte bank groups.
__device__ __forceinline__ int fa_kbase() {
    const int lane = fa_lane(), l32 = lane & 31, h = lane >> 5;
    const int m = l32;
    const int row = 16 * (m >> 4) + 8 * ((m >> 2) & 1) + 4 * ((m >> 3) & 1) + (m & 3);
    return row * KROW + h * 16;
}
// V^T operand of P.V step st, d-tile mt: row 32mt + l32, piece
// (2st + h) ^ ((row / 4) % 4): vbase ^ (st << 5), plus mt * 2 KiB
__device__ __forceinline__ int fa_vbase() {
    const int lane = fa_lane(), l32 = lane & 31, h = lane >> 5;
    const int sw = (l32 >> 2) & 3;
    return l32 * VB * 2 + (((h ^ sw) & 1) << 4) + ((sw & 2) << 4);
}

__device__ __forceinline__ u16x8 lds16(const char *p) {
    return *reinterpret_cast<const u16x8 *>(p);
}

// the LDS tile buffers: K tiles 0..1, then a ring of five 32-key V^T
// blocks (tile u's block h in slot (2u + h) % 5: a step reads the block of
// the step before it, so at most five are live or in flight)
__shared__ __attribute__((aligned(16))) char fa_lds[2 * KBUF + 5 * VHALF];

struct FaCtx {
    KvRef kv;                          // the cache
    int hd, kvh, nkv, nblk;            // block-table row, kv head, kv heads, cache blocks used
    int nkt, nkeys;                    // key tiles, keys
    int tid, wave, lane, l32, h;
    float c2;                          // scale * log2(e)
    uint32_t lds;                      // LDS address of fa_lds
};

// Cache block 2 kt + half of key tile kt (clamped to the last block
// holding keys), its id (a block-table load for a paged cache), and the
// buffer resources of its K rows and V^T block.
// The id is read by a vector load (the address is uniform; the value is
// taken with readfirstlane a tile later, after the tile barrier's wait for
// the vector memory counter). A scalar load would be counted by lgkmcnt,
// which LDS reads share and which does not retire scalar loads in order:
// with one pending, every LDS operand read would have to wait for all
// reads in flight (lgkmcnt(0)) instead of just its own.
__device__ __forceinline__ int fa_block(const FaCtx &c, int kt, int half) {
    return min(2 * kt + half, c.nblk - 1);
}
__device__ __forceinline__ int fa_block_id(const FaCtx &c, int b) {
    if (!c.kv.btab) return (int)kv_block_id_u(c.kv, c.hd, b);
    typedef const __attribute__((address_space(1))) int32_t *gi32p;
    return *(gi32p)(c.kv.btab + (size_t)c.hd * c.kv.bstride + b);
}
__device__ __forceinline__ i32x4 fa_krsrc(const FaCtx &c, int kt, int half, int id) {
    const int b = 2 * kt + half;
    const int valid = max(0, min(KVB, c.nkeys - KVB * b));
    return dma_rsrc(c.kv.k + ((size_t)id * c.nkv + c.kvh) * KVB * D, (uint32_t)valid * D * 2);
}
__device__ __forceinline__ i32x4 fa_vrsrc(const FaCtx &c, int kt, int half, int id) {
    const int b = 2 * kt + half;
    return dma_rsrc(c.kv.v + ((size_t)id * c.nkv + c.kvh) * D * KVB,
                   b < c.nblk ? (uint32_t)(D * KVB * 2) : 0u);
}

// running softmax state of one query row (per lane)
struct FaRow {
    int qpos;                          // query position
    float M, lsum;                     // reference point (a running max), sum of e^{A - M}
    float K2;                          // pass 2: M * scale * log2(e) + log2(sum)
};

// Instruction order. Each phase below is its own basic block (fa_split:
// a uniform branch on a runtime value the compiler cannot fold), so the
// scheduler cannot mix the K reads of an S block with the V reads of a
// P.V block or pull a later step's reads forward. Inside the pass-1 step
// and the P.V half of a pass-2 step, each (operand read DEPTH ahead, MFMA,
// softmax work of one score) slice is fenced by a scheduling barrier:
// under this register pressure the scheduler otherwise moves every
// operand read to just before its MFMA (each MFMA then waits for its
// read) and the softmax work after the last MFMA, and scheduling-group
// barriers did not keep the slices. The S-only block (fa_s) keeps
// scheduling-group barriers, which it follows.
__device__ __forceinline__ void fa_split(int opaque) {
    if (__builtin_expect(opaque == -12345, 0)) asm volatile("s_nop 0");
}

// DEPTH LDS reads, then (1 MFMA, NVALU VALU, 1 read) x (16 - DEPTH), then
// (1 MFMA, NVALU VALU) x DEPTH
template <int DEPTH, int NVALU>
__device__ __forceinline__ void fa_groups16() {
    __builtin_amdgcn_sched_group_barrier(0x100, DEPTH, 0);   // LDS reads
#pragma unroll
    for (int i = 0; i < 16 - DEPTH; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        if (NVALU) __builtin_amdgcn_sched_group_barrier(0x002, NVALU, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < DEPTH; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (NVALU) __builtin_amdgcn_sched_group_barrier(0x002, NVALU, 0);
    }
}

// The softmax arithmetic per score, on the VALU, kept to a few
// instructions because it is only partly hidden under the MFMAs:
//   r   = rnd(q.k)                       v_cvt_pk_bf16_f32 (two scores),
//                                        then a shift / mask to fp32
//   arg = r * c2 - K                     v_fma_f32 (c2 = scale * log2(e),
//                                        a power of two times log2(e))
//   e   = exp2(arg)                      v_exp_f32
// pass 1 (K = m * c2): the running sum of e; the row max is taken on the
// unrounded scores (rnd is monotone: max rnd(x) = rnd(max x));
// pass 2 (K = m * c2 + log2(s)): P = rnd(e) = rnd(e^{A-m} / s), the
// reference's normalised probability (c/attn.h:354-360) with the division
// folded into the exponent: a relative difference of a few 1e-7 from the
// quotient, which moves P by one bf16 ulp only when e / s lies that close
// to a rounding boundary -- the tolerance class of the hardware exp2.
// Scores past the query (key kj + 16(i/8) + 8h + i%8 > qpos) are masked
// only on steps that reach the diagonal (MASK).
__device__ __forceinline__ bool fa_keep(int i, int lim) {
    return 16 * (i >> 3) + (i & 7) <= lim;
}
// e_i = exp2(rnd(sc_i) * c2 - K), 0 where masked
template <bool MASK>
__device__ __forceinline__ void fa_exp16(float (&e)[16], const f32x16 &sc, float c2, float K,
                                         int lim) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t pk = pack2(sc[2 * j], sc[2 * j + 1]);
        e[2 * j] = __builtin_amdgcn_exp2f(fmaf(__uint_as_float(pk << 16), c2, -K));
        e[2 * j + 1] = __builtin_amdgcn_exp2f(fmaf(__uint_as_float(pk & 0xffff0000u), c2, -K));
    }
    if (MASK) {
#pragma unroll
        for (int i = 0; i < 16; i++) e[i] = fa_keep(i, lim) ? e[i] : 0.0f;
    }
}

// the K operand address of S^T step ks
__device__ __forceinline__ const char *fa_kaddr(const char *Kp, int kbase, int ks) {
    return Kp + kbase + ks * 32;
}
// the V^T operand address of P.V MFMA jj (step jj/8, d-tile jj%8)
__device__ __forceinline__ const char *fa_vaddr(const char *Vp, int vbase, int jj) {
    return Vp + (vbase ^ ((jj >> 3) << 5)) + (jj & 7) * 32 * VB * 2;
}

// S^T of the 32-key K block at byte offset Kn of fa_lds for this lane's
// query (element i <-> key 16(i/8) + 8h + i%8 of the block), operands
// read 4 ahead; no other work.
__device__ __forceinline__ f32x16 fa_s(const FaCtx &c, int Kn, const bf16x8 (&q)[D / 16]) {
    const int kbase = fa_kbase();
    const char *Kp = fa_lds + Kn;
    f32x16 sc;
#pragma unroll
    for (int i = 0; i < 16; i++) sc[i] = 0.0f;
    u16x8 kq[3];
#pragma unroll
    for (int i = 0; i < 3; i++) kq[i] = lds16(fa_kaddr(Kp, kbase, i));
#pragma unroll
    for (int ks = 0; ks < D / 16; ks++) {
        const bf16x8 k = __builtin_bit_cast(bf16x8, kq[ks % 3]);
        if (ks + 3 < D / 16) kq[ks % 3] = lds16(fa_kaddr(Kp, kbase, ks + 3));
        sc = mfma32(k, q[ks], sc);
    }
    fa_groups16<3, 0>();
    fa_split(c.nkeys);
    return sc;
}

// pass-1 step j: S(j+1) from the K block at Kn (when NEXT), interleaved
// with folding S(j) = sc (keys from kj) into the row's sum. The terms are
// taken against the row's current reference point M, with no max over the
// step: a sum taken against any M < max A is the sum against the max times
// e^{max A - M}, and pass 2's exponent M c2 + log2(s) is the same either
// way. M starts at -inf, so the first step's sum is +inf and takes the
// slow path, which sets M to the running max as before; it is raised
// again only if the sum reaches 2^100 (scores ~100 / c2 above M),
// so the terms never overflow and none underflows that would not against
// the true max.
template <bool NEXT, bool MASK>
__device__ __forceinline__ void fa_p1_step(const FaCtx &c, int Kn, int kj,
                                           const bf16x8 (&q)[D / 16], f32x16 &sc, FaRow &w) {
    const int lim = w.qpos - kj - 8 * (fa_lane() >> 5);
    f32x16 nx;
    float e[16];
    float ps = 0.0f;
    const float Kc = w.M * c.c2;
    if (NEXT) {
        const int kbase = fa_kbase();
        const char *Kp = fa_lds + Kn;
#pragma unroll
        for (int i = 0; i < 16; i++) nx[i] = 0.0f;
        u16x8 kq[4];
#pragma unroll
        for (int i = 0; i < 4; i++) kq[i] = lds16(fa_kaddr(Kp, kbase, i));
        uint32_t pk = 0;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < D / 16; ks++) {
            const bf16x8 k = __builtin_bit_cast(bf16x8, kq[ks % 4]);
            if (ks + 4 < D / 16) kq[ks % 4] = lds16(fa_kaddr(Kp, kbase, ks + 4));
            nx = mfma32(k, q[ks], nx);
            if ((ks & 1) == 0) pk = pack2(sc[ks], sc[ks + 1]);
            const float r = __uint_as_float((ks & 1) ? (pk & 0xffff0000u) : (pk << 16));
            float ev = __builtin_amdgcn_exp2f(fmaf(r, c.c2, -Kc));
            if (MASK) ev = fa_keep(ks, lim) ? ev : 0.0f;
            ps += ev;
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        fa_exp16<MASK>(e, sc, c.c2, Kc, lim);
#pragma unroll
        for (int i = 0; i < 16; i++) ps += e[i];
    }
    const float ls = w.lsum + sum32(ps);
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(ls < 0x1p100f)) != 0, 0)) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) mx = fmaxf(mx, !MASK || fa_keep(i, lim) ? sc[i] : -INFINITY);
        const float mn = fmaxf(w.M, rnd_hw(max32(mx)));
        fa_exp16<MASK>(e, sc, c.c2, mn * c.c2, lim);
        ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) ps += e[i];
        w.lsum = w.lsum * __builtin_amdgcn_exp2f((w.M - mn) * c.c2) + sum32(ps);
        w.M = mn;
    } else {
        w.lsum = ls;
    }
    if (NEXT) sc = nx;
    fa_split(c.nkeys);
}

// pass-2 step j: S(j) from the K block at Kn; then (when PV) the MFMAs of
// P(j-1).V(j-1) from the V block at Vp, interleaved with forming P(j)
// (keys from kj). pp holds P(j-1) on entry and P(j) on
// return, as the B operands of the two P.V steps (keys 8h..8h+7 and
// 16 + 8h..).
template <bool PV, bool MASK>
__device__ __forceinline__ void fa_p2_step(const FaCtx &c, int Kn, int Vp, int kj,
                                           const bf16x8 (&q)[D / 16], const FaRow &w,
                                           bf16x8 (&pp)[2], f32x16 (&o)[D / 32]) {
    const f32x16 sc = fa_s(c, Kn, q);
    const int lim = w.qpos - kj - 8 * (fa_lane() >> 5);
    uint32_t pw[8];
    if (PV) {
        const int vbase = fa_vbase();
        const char *Vb = fa_lds + Vp;
        u16x8 vq[2];
#pragma unroll
        for (int i = 0; i < 2; i++) vq[i] = lds16(fa_vaddr(Vb, vbase, i));
        uint32_t pk = 0;
        float ep = 0.0f;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jj = 0; jj < 2 * (D / 32); jj++) {
            const bf16x8 va = __builtin_bit_cast(bf16x8, vq[jj % 2]);
            if (jj + 2 < 2 * (D / 32)) vq[jj % 2] = lds16(fa_vaddr(Vb, vbase, jj + 2));
            o[jj & 7] = mfma32(va, pp[jj >> 3], o[jj & 7]);
            if ((jj & 1) == 0) pk = pack2(sc[jj], sc[jj + 1]);
            const float r = __uint_as_float((jj & 1) ? (pk & 0xffff0000u) : (pk << 16));
            float ev = __builtin_amdgcn_exp2f(fmaf(r, c.c2, -w.K2));
            if (MASK) ev = fa_keep(jj, lim) ? ev : 0.0f;
            if (jj & 1) pw[jj >> 1] = pack2(ep, ev);
            else ep = ev;
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        float e[16];
        fa_exp16<MASK>(e, sc, c.c2, w.K2, lim);
#pragma unroll
        for (int i = 0; i < 8; i++) pw[i] = pack2(e[2 * i], e[2 * i + 1]);
    }
    // keep P(j) in this block (else it is sunk past the next step's S)
    asm volatile("" : "+v"(pw[0]), "+v"(pw[1]), "+v"(pw[2]), "+v"(pw[3]), "+v"(pw[4]),
                 "+v"(pw[5]), "+v"(pw[6]), "+v"(pw[7]));
#pragma unroll
    for (int st = 0; st < 2; st++) {
        const uint32_t w4[4] = {pw[4 * st], pw[4 * st + 1], pw[4 * st + 2], pw[4 * st + 3]};
        pp[st] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u16x8 *>(w4));
    }
    fa_split(c.nkeys);
}

// the last P.V (no S after it)
__device__ __forceinline__ void fa_pv_last(const FaCtx &c, int Vp, const bf16x8 (&pp)[2],
                                           f32x16 (&o)[D / 32]) {
    const int vbase = fa_vbase();
    const char *Vb = fa_lds + Vp;
#pragma unroll
    for (int jj = 0; jj < 2 * (D / 32); jj++) {
        const bf16x8 va = __builtin_bit_cast(bf16x8, lds16(fa_vaddr(Vb, vbase, jj)));
        o[jj & 7] = mfma32(va, pp[jj >> 3], o[jj & 7]);
    }
}

// wait for this wavefront's copies, then the barrier that publishes them
__device__ __forceinline__ void fa_publish() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

__global__ __launch_bounds__(64 * NW) void k_attn_fa(
    FaSeqs sq, const int32_t *__restrict__ dmeta, const uint16_t *__restrict__ qn_w,
    const uint16_t *__restrict__ rope,
    const uint16_t *__restrict__ qg, KvRef kv, int nh, int nkv, float scale,
    uint16_t *__restrict__ y, const uint16_t *__restrict__ sig_bf, uint16_t *__restrict__ tr_attno) {
    const int n = sq.n;
    const int32_t *cu = dmeta ? dmeta : sq.cu;
    const int32_t *pos0 = dmeta ? dmeta + n + 1 : sq.pos0;
    const int32_t *toff = dmeta ? dmeta + 2 * n + 1 : sq.toff;
    const int32_t *hdv = dmeta ? dmeta + 3 * n + 2 : sq.hd;
    const int ntiles = toff[n];
    const int g = ntiles - 1 - (int)(blockIdx.x / nkv);
    const int kvh = blockIdx.x % nkv;
    // workgroup-uniform (loaded values are not provably so: readfirstlane
    // keeps them in SGPRs)
    const int s = __builtin_amdgcn_readfirstlane(seq_of(toff, n, g));
    const int tb = __builtin_amdgcn_readfirstlane(cu[s] + (g - toff[s]) * TQ);  // first token
    const int nt = __builtin_amdgcn_readfirstlane(min(TQ, cu[s + 1] - tb));
    const int qpos0 = __builtin_amdgcn_readfirstlane(pos0[s] + (tb - cu[s]));  // its position

    FaCtx c;
    c.nkeys = qpos0 + nt;
    c.tid = threadIdx.x;
    c.lane = c.tid & 63;
    c.h = c.lane >> 5;
    c.l32 = c.lane & 31;
    c.wave = __builtin_amdgcn_readfirstlane(c.tid >> 6);
    c.kv = kv;
    c.hd = __builtin_amdgcn_readfirstlane(hdv[s]);
    c.kvh = kvh;
    c.nkv = nkv;
    c.nkt = (c.nkeys + KT - 1) / KT;
    c.nblk = (c.nkeys + VB - 1) / VB;
    c.lds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)fa_lds);
    c.c2 = scale * 1.44269504088896341f;
    const int nkt = c.nkt;
    // byte offsets of tile u's buffers in fa_lds
    auto kbuf = [&](int u) { return (u & 1) * KBUF; };
    auto vbuf = [&](int u, int half) { return 2 * KBUF + ((2 * u + half) % 5) * VHALF; };

    // tile u = 0 .. 2nkt-1 of the key stream: pass u / nkt, key tile u %
    // nkt. An identity (flat) table puts the sequence's blocks of this kv head
    // at a fixed stride: one resource per cache covers them all and a tile
    // only moves a scalar offset. A paged table builds each block's
    // resources from its block id, read a tile ahead.
    const bool flat = kv.btab == nullptr;
    const int blk_bytes = nkv * KVB * D * 2;
    i32x4 kflat = {0, 0, 0, 0}, vflat = {0, 0, 0, 0};
    if (flat) {
        const size_t b0 = (size_t)c.hd * kv.bstride * nkv + kvh;   // block 0 of this kv head
        kflat = dma_rsrc(kv.k + b0 * KVB * D,
                         (uint32_t)((c.nblk - 1) * blk_bytes + (c.nkeys - KVB * (c.nblk - 1)) * D * 2));
        vflat = dma_rsrc(kv.v + b0 * D * KVB, (uint32_t)((c.nblk - 1) * blk_bytes + D * KVB * 2));
    }
    // A tile's copy is in 8 parts: part p is K rows 8p..8p+7 and V^T
    // groups 4p..4p+3, from cache block 2 kt + p / 4. Wavefronts 0..3 (one
    // per SIMD) issue parts w and w + 4, wavefronts 4..7 none: a wavefront
    // issuing copies stalls while the address unit takes them, and with
    // every wavefront copying both wavefronts of a SIMD stalled at each
    // tile start; with one copier per SIMD the other keeps issuing MFMAs
    // (T=8192: 0.96 -> 0.92 ms). idn[half]: the block ids of the next tile
    // to copy, read a tile ahead (the loads complete under the copies).
    const bool copier = c.wave < 4;
    int idn[2] = {0, 0};
    auto copy_tile = [&](int u, int kt, bool withv) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int part = c.wave + 4 * half;
            i32x4 kr = kflat, vr = vflat;
            int off = (2 * kt + half) * blk_bytes;
            if (!flat) {
                const int id = __builtin_amdgcn_readfirstlane(idn[half]);
                kr = fa_krsrc(c, kt, half, id);
                vr = fa_vrsrc(c, kt, half, id);
                off = 0;
            }
            fa_dma_k(c.lds + kbuf(u), kr, off, part);
            if (withv) fa_dma_v(c.lds + vbuf(u, 0), c.lds + vbuf(u, 1), vr, off, part);
        }
    };
    auto next_ids = [&](int kt) {
        if (!flat) {
            idn[0] = fa_block_id(c, fa_block(c, kt, 0));
            idn[1] = fa_block_id(c, fa_block(c, kt, 1));
        }
    };
    if (copier) {
        next_ids(0);
        copy_tile(0, 0, false);
        next_ids(1 % nkt);
    }

    // query row of this lane: token 4w + l32/8, head l32%8 of the kv head
    const int tk = c.wave * 4 + c.l32 / GRP, head = kvh * GRP + c.l32 % GRP;
    // The q row, formed here from the layer's input as k_attn_prep forms k
    // (c/attn.h:175-236 via c/layer.h:300-312): (1+w) RMSNorm with the
    // ascending sum of squares, then NeoX RoPE on dims 0..63 at the token's
    // position, each product rounded as the reference rounds it. The lane
    // holds dims 16 ks + 8 h .. +7, and lane l ^ 32 the other 8 of each 16;
    // each lane takes its partner's chunks by exchange and runs the whole
    // ascending sum over the 32 8-dim chunks itself. A RoPE pair (d, d + 32)
    // lies in chunks ks and ks + 2 of the same lane.
    bf16x8 q[D / 16];
    {
        constexpr int R = 32;                  // rotary pairs (64 rotated dims)
        const int tq = min(tk, nt - 1);
        const uint16_t *xr = qg + ((size_t)(tb + tq) * nh + head) * 2 * D + c.h * 8;
        float ss = 0.0f;
        {
            u16x8 xv[D / 16];
#pragma unroll
            for (int ks = 0; ks < D / 16; ks++) xv[ks] = *reinterpret_cast<const u16x8 *>(xr + ks * 16);
            // the other half's chunks (independent exchanges, all in flight
            // together); then both halves run the whole chain, in order
            u16x8 px[D / 16];
#pragma unroll
            for (int ks = 0; ks < D / 16; ks++) {
                const uint4 u = __builtin_bit_cast(uint4, xv[ks]);
                px[ks] = __builtin_bit_cast(u16x8, make_uint4(__shfl_xor(u.x, 32), __shfl_xor(u.y, 32),
                                                              __shfl_xor(u.z, 32), __shfl_xor(u.w, 32)));
            }
#pragma unroll
            for (int ks = 0; ks < D / 16; ks++) {
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const u16x8 xc = hh == c.h ? xv[ks] : px[ks];   // chunk (ks, hh)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float f = bf2f(xc[e]);
                        ss = fmaf(f, f, ss);   // f * f exact: bf16 squared
                    }
                }
            }
        }
        // the row is read again below, a chunk at a time (an L2 hit), so
        // that the 64 registers of the first read are not live beside q
        asm volatile("" ::: "memory");
        const float rr = 1.0f / sqrtf(ss / (float)D + 1e-6f);
        // normed value of dim e of the lane's chunk ks
        auto nrm = [&](const u16x8 &xk, int e, const u16x8 &wv) {
            return rndf((bf2f(xk[e]) * rr) * (1.0f + bf2f(wv[e])));
        };
        auto ldx = [&](int ks) { return *reinterpret_cast<const u16x8 *>(xr + ks * 16); };
        const uint16_t *cs = rope + (size_t)(qpos0 + tq) * (2 * R);
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const u16x8 w0 = *reinterpret_cast<const u16x8 *>(qn_w + ks * 16 + c.h * 8);
            const u16x8 w1 = *reinterpret_cast<const u16x8 *>(qn_w + (ks + 2) * 16 + c.h * 8);
            const int i0 = ks * 16 + c.h * 8;          // pair index of the chunk's first dim
            const u16x8 cv = *reinterpret_cast<const u16x8 *>(cs + i0);
            const u16x8 sv = *reinterpret_cast<const u16x8 *>(cs + R + i0);
            const u16x8 x0 = ldx(ks), x1 = ldx(ks + 2);
            u16x8 lo, hi;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float a = nrm(x0, e, w0), b = nrm(x1, e, w1);
                const float cc = bf2f(cv[e]), sn = bf2f(sv[e]);
                lo[e] = f2bf(rndf(a * cc) + rndf(-b * sn));     // dim d < 32
                hi[e] = f2bf(rndf(b * cc) + rndf(a * sn));      // dim d + 32
            }
            q[ks] = __builtin_bit_cast(bf16x8, lo);
            q[ks + 2] = __builtin_bit_cast(bf16x8, hi);
        }
#pragma unroll
        for (int ks = 4; ks < D / 16; ks++) {
            const u16x8 wv = *reinterpret_cast<const u16x8 *>(qn_w + ks * 16 + c.h * 8);
            const u16x8 xk = ldx(ks);
            u16x8 out;
#pragma unroll
            for (int e = 0; e < 8; e++) out[e] = f2bf(nrm(xk, e, wv));
            q[ks] = __builtin_bit_cast(bf16x8, out);
        }
    }
    FaRow w{qpos0 + tk, -INFINITY, 0.0f, 0.0f};

    // Tile u = 0 .. 2nkt-1 of the key stream: pass u / nkt, key tile
    // u % nkt. begin_tile(u) publishes tile u and starts the copy of u+1.
    auto begin_tile = [&](int u) {
        fa_publish();
        if (u + 1 < 2 * nkt && copier) {
            copy_tile(u + 1, (u + 1) % nkt, u + 1 >= nkt);
            next_ids((u + 2) % nkt);
        }
        // the last tile's V keys past nkeys: zero (P is 0 there, but
        // 0 * NaN from unwritten cache memory would not be)
        if (u == 2 * nkt - 1 && c.nkeys % VB != 0) {
            const int kbase = (nkt - 1) * KT;
            for (int e = c.tid; e < KT * D; e += 64 * NW) {
                const int bb = e / (D * VB), rem = e % (D * VB), row = rem / VB, kk = rem % VB;
                if (kbase + bb * VB + kk >= c.nkeys) {
                    uint16_t *Vn = reinterpret_cast<uint16_t *>(fa_lds + vbuf(u, bb));
                    const int cc = (kk >> 3) ^ ((row >> 2) & 3);
                    Vn[row * VB + cc * 8 + (kk & 7)] = 0;
                }
            }
            __syncthreads();
        }
    };
    constexpr int HALF = KHALF;
    // a step with keys from kj needs the causal mask when it reaches past
    // this wavefront's first query
    const int qminw = qpos0 + 4 * c.wave;
#define FA_P1(NEXT, Kn, kj)                                                    \
    do {                                                                       \
        const int kj_ = (kj);                                                  \
        if (kj_ + 31 > qminw) fa_p1_step<NEXT, true>(c, Kn, kj_, q, sc, w);    \
        else fa_p1_step<NEXT, false>(c, Kn, kj_, q, sc, w);                    \
    } while (0)

    // pass 1 (steps j = 0 .. 2nkt-1; step j folds S(j) while S(j+1) is
    // formed)
    begin_tile(0);
    f32x16 sc = fa_s(c, kbuf(0), q);
    FA_P1(true, kbuf(0) + HALF, 0);
    for (int u = 1; u < nkt; u++) {
        begin_tile(u);
        FA_P1(true, kbuf(u), (u - 1) * KT + 32);
        FA_P1(true, kbuf(u) + HALF, u * KT);
    }
    begin_tile(nkt);                     // pass 2's key tile 0 (and its V)
    FA_P1(false, 0, (nkt - 1) * KT + 32);
    w.K2 = w.M * c.c2 + __builtin_amdgcn_logf(w.lsum);     // v_log_f32: log2

    // pass 2 (step j = 2kt + half of key tile kt, in stream tile nkt + kt)
    f32x16 o[D / 32];
#pragma unroll
    for (int mt = 0; mt < D / 32; mt++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[mt][i] = 0.0f;
    bf16x8 pp[2];
    // Key tiles below nmf need no mask for any query of the workgroup; the
    // rest (one or two) are masked. Two loops rather than a branch per
    // step: a branch around the O^T updates makes the register allocator
    // spill. Key tile 0 is always run masked.
    const int nmf = (qpos0 + 1) / KT;
    fa_p2_step<false, true>(c, kbuf(nkt), 0, 0, q, w, pp, o);
    fa_p2_step<true, true>(c, kbuf(nkt) + HALF, vbuf(nkt, 0), 32, q, w, pp, o);
    int u = nkt + 1;
    for (; u < nkt + nmf; u++) {
        const int kt = u - nkt;
        begin_tile(u);
        fa_p2_step<true, false>(c, kbuf(u), vbuf(u - 1, 1), kt * KT, q, w, pp, o);
        fa_p2_step<true, false>(c, kbuf(u) + HALF, vbuf(u, 0), kt * KT + 32, q, w, pp, o);
    }
    for (; u < 2 * nkt; u++) {
        const int kt = u - nkt;
        begin_tile(u);
        fa_p2_step<true, true>(c, kbuf(u), vbuf(u - 1, 1), kt * KT, q, w, pp, o);
        fa_p2_step<true, true>(c, kbuf(u) + HALF, vbuf(u, 0), kt * KT + 32, q, w, pp, o);
    }
    fa_pv_last(c, vbuf(2 * nkt - 1, 1), pp, o);

#undef FA_P1
    // epilogue: o = rnd(O); y = rnd(o * rnd(sigmoid(gate)))
    if (tk < nt) {
        const size_t row = (size_t)(tb + tk) * nh + head;
        const uint16_t *gr = qg + row * 2 * D + D;
        uint16_t *yr = y + row * D;
#pragma unroll
        for (int mt = 0; mt < D / 32; mt++) {
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const int d0 = mt * 32 + 8 * q4 + 4 * c.h;
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
        // (trace) rnd(o) before the gate, in a loop of its own: a
        // conditional store inside the loop above would make the compiler
        // drain the memory counter at every join
        if (tr_attno) {
#pragma unroll
            for (int mt = 0; mt < D / 32; mt++) {
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const int d0 = mt * 32 + 8 * q4 + 4 * c.h;
                    u16x4 oc;
#pragma unroll
                    for (int i = 0; i < 4; i++) oc[i] = f2bf(rndf(o[mt][4 * q4 + i]));
                    *reinterpret_cast<u16x4 *>(tr_attno + row * D + d0) = oc;
                }
            }
        }
    }
}

}  // namespace

namespace apus {

int attn_prefill_kv(const ApusHipAttnLayer *L, size_t B, const int32_t *cu, const int32_t *pos0,
                    const int32_t *rows, const uint16_t *qg, const uint16_t *k,
                    const uint16_t *v, const KvRef &kv, uint16_t *y) {
    if (int r = attn_check_layer(L)) return r;
    if (B == 0) return kOk;
    // q/k norm + RoPE + cache append (shared with decode); the metadata
    // also checks the offsets and the cache capacity
    AttnSeqs as;
    const int32_t *adm = nullptr;
    size_t mt = 0;
    if (int r = attn_meta(B, cu, pos0, rows, (size_t)kv.bstride, L->nkv, 0, &as, &adm, &mt))
        return r;
    const size_t Ttot = (size_t)cu[B];
    if (Ttot == 0) return kOk;
    size_t max_pos = 0;
    std::vector<int32_t> meta(4 * B + 2);
    int32_t *mcu = meta.data(), *mpos = mcu + B + 1, *mtoff = mpos + B, *mhd = mtoff + B + 1;
    mtoff[0] = 0;
    for (size_t s = 0; s < B; s++) {
        const int32_t ns = cu[s + 1] - cu[s];
        max_pos = std::max(max_pos, (size_t)pos0[s] + (size_t)ns);
        mtoff[s + 1] = mtoff[s] + (ns + TQ - 1) / TQ;
        mhd[s] = rows ? rows[s] : (int32_t)s;
    }
    memcpy(mcu, cu, (B + 1) * 4);
    memcpy(mpos, pos0, B * 4);
    const size_t ntiles = (size_t)mtoff[B];
    FaSeqs fs;
    fs.n = (int32_t)B;
    const int32_t *fdm = nullptr;
    if (B <= (size_t)kFaInline) {
        memcpy(fs.cu, cu, (B + 1) * 4);
        memcpy(fs.pos0, pos0, B * 4);
        memcpy(fs.toff, mtoff, (B + 1) * 4);
        memcpy(fs.hd, mhd, B * 4);
    } else {
        fdm = (const int32_t *)upload_async(meta.data(), meta.size() * 4);
        if (!fdm) return kErrHip;
    }
    // the q rows are formed by the flash kernel itself; prep norms, ropes
    // and appends the k rows (and, for a traced call, also writes the q rows
    // the trace records; with one kv head a prep block's k rows would span
    // more tokens than its metadata holds, so it keeps the q rows too)
    const bool qrows = attn_trace() != nullptr || L->nkv < 2;
    uint16_t *qn = nullptr;
    if (qrows) {
        qn = (uint16_t *)scratch(kScratchAttnQ, Ttot * L->nh * D * 2);
        if (!qn) return kErrHip;
    }
    if (int r = attn_prep(L, as, adm, Ttot, max_pos, attn_max_vblocks(B, cu, pos0), qg, k, v,
                          kv, qn, qrows))
        return r;
    const uint16_t *rope = rope_table(L->rot, L->theta, max_pos);
    if (!rope) return kErrHip;
    const float scale = (float)(1.0 / sqrt((double)L->d));
    const ActTables *tabs = act_tables();
    if (!tabs) return kErrHip;
    APUS_TIMED("k_attn_fa",
               k_attn_fa<<<(unsigned)(ntiles * L->nkv), 64 * NW, 0, stream()>>>(
                   fs, fdm, L->qn_w, rope, qg, kv, (int)L->nh, (int)L->nkv, scale, y, tabs->sig_bf,
                   attn_trace() ? attn_trace()->attno : nullptr));
    APUS_LAUNCHED("k_attn_fa");
    return kOk;
}

}  // namespace apus

extern "C" {

int apus_hip_attn_prefill(const ApusHipAttnLayer *L, size_t B, const int32_t *cu,
                          const int32_t *pos0, const uint16_t *qg, const uint16_t *k,
                          const uint16_t *v, uint16_t *kcache, uint16_t *vcache,
                          size_t max_seq, uint16_t *y) {
    APUS_READY();
    if (max_seq % VB != 0) return set_error(kErrArgument, "max_seq must be a multiple of %d", VB);
    return attn_prefill_kv(L, B, cu, pos0, nullptr, qg, k, v, kv_flat(kcache, vcache, max_seq),
                           y);
}

int apus_hip_attn_prefill_paged(const ApusHipAttnLayer *L, size_t B, const int32_t *rows,
                                const int32_t *cu, const int32_t *pos0, const uint16_t *qg,
                                const uint16_t *k, const uint16_t *v, const ApusHipKvCache *kv,
                                uint16_t *y) {
    APUS_READY();
    KvRef r;
    if (int e = kv_paged_ref(kv, B, rows, cu, pos0, &r)) return e;
    return attn_prefill_kv(L, B, cu, pos0, rows, qg, k, v, r, y);
}

}  // extern "C"
