// attn_mixer.hip -- batched, device-resident gated-GQA mixer for gfx950:
// the op sequence of c/layer.h:300-322 (decode) for B sequences of 1..4
// new tokens each (more than one is the MTP verify shape, c/mtp.h:36-75).
//
// The KV cache is addressed in blocks of 32 positions through a block
// table (attn_mixer.h): the flat layout of apus_hip_attn_decode is the
// identity table, a paged cache (apus_hip_kv_pool_*) passes its own.
//
// Decode kernels (split-K over the context; the 8 q heads of a kv head and
// up to 4 new tokens form the MFMA rows, so K and V are read once per
// group). The splits are balanced ("stream-K"): the (sequence, kv head)
// pairs' key ranges, each padded to a multiple of 64, are laid end to end
// and cut into equal runs of T keys, one per wavefront, so every wavefront
// streams the same number of keys however ragged the contexts are; a run
// that crosses a pair boundary is processed as two segments. Segment
// (pair p, wavefront w) keeps its partial results in slot p + w (unique:
// consecutive segments raise p or w or both).
//   k_attn_prep     q/k (1+w) RMSNorm, RoPE, K append; V append (other
//                   blocks of the same launch)
//   k_attn_scores   A = rnd(rnd(q.k)*scale) on MFMA 16x16x32 bf16 into a
//                   bf16 score buffer, per-segment (max, sum exp)
//   k_attn_pv       P = rnd(exp(A-m)/s) with the pair's global (m, s) --
//                   the reference's normalised bf16 probabilities
//                   (c/attn.h:354-360) -- times V on MFMA, fp32 partials
//   k_attn_combine  sum of the partials in key order, rnd, sigmoid gate
// Scores and the P.V sum accumulate in a different order than the
// reference's sequential loops (a tolerance class); everything else
// follows the reference op for op.
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

constexpr int D = 256, ROT = 64, GRP = 8;     // head dim, rotary dims, q heads per kv head
constexpr int kRows = 32;                     // rows: GRP heads x up to 4 tokens
constexpr float kEps = 1e-6f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr float kL2E = 1.44269504088896341f;
// two fp32 values as bf16 codes (hardware round-to-nearest-even), lo first
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));

// 16-byte loads from global memory through pointers whose address space
// the compiler cannot infer (built from scalar registers, or selected
// between kernel-argument and device copies): as flat loads they would
// also count on the LDS counter, so every LDS wait of the stream would
// wait for the loads in flight
typedef const __attribute__((address_space(1))) u16x8 *gu16x8p;
__device__ __forceinline__ u16x8 gld16(const uint16_t *p) { return *(gu16x8p)p; }
__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t *p) {
    return __builtin_bit_cast(bf16x8, gld16(p));
}

__host__ __device__ inline int seq_of(const int32_t *off, int n, int x) {
    int lo = 0, hi = n - 1;          // largest s with off[s] <= x
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= x) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Metadata views: by value (AttnSeqs) or, for large batches, a device
// array cu[B+1] | pos0[B] | ccap[B+1] | hd[B].
struct Meta {
    const int32_t *cu, *pos0, *ccap, *hd;
};
__device__ __forceinline__ Meta meta_of(const AttnSeqs &sq, const int32_t *dmeta) {
    if (!dmeta) return Meta{sq.cu, sq.pos0, sq.ccap, sq.hd};
    const int n = sq.n;
    return Meta{dmeta, dmeta + n + 1, dmeta + 2 * n + 1, dmeta + 3 * n + 2};
}

// The prep blocks of k_attn_prep: one block of 256 threads per rpb <= 64 rows, a row being one
// (token, slot) with slots 0..nh-1 the q heads and nh..nh+nkv-1 the kv
// heads. Rows are staged in LDS as bf16 with 16-byte loads; lane r of the
// first wavefront takes row r's ascending sum of squares (c/attn.h:177-182,
// the reference's order, so rs is bit-exact); then each thread takes one
// 16-byte piece (8 dims) of a row at a time: (1+w) RMSNorm with one
// rounding, the partial NeoX RoPE with the host-made cos/sin codes
// (c/attn.h:244-266, the partner dims +-32 read from the staged row), and
// a 16-byte store of q to qn or of k to the K cache. V is appended by
// the launch's other blocks (vappend_block).
constexpr int PRB = 32;                  // rows per k_attn_prep block
constexpr int PRS = D + 8;               // LDS row pitch (bf16): rows on distinct banks
constexpr int PTK = PRB / 2 + 2;             // tokens a prep block's rows can span (nslot >= 2)
// the prep block's LDS: rows, cos / sin codes, rs, cache offsets, tokens
struct PrepLds {
    uint16_t xs[PRB * PRS];
    uint16_t rcs[PRB * ROT];                 // cos / sin codes
    float rs[PRB];
    size_t rdst[PRB];                        // k rows: element offset of the cache row
    int tpos[PTK], thd[PTK];                 // the tokens' positions and block-table rows
};
constexpr int kVappLds = 32 * PRS * 2;       // the V append block's staged rows
constexpr int kPrepKernLds = sizeof(PrepLds) > kVappLds ? sizeof(PrepLds) : kVappLds;

__device__ __forceinline__ void prep_block(
    int bid, PrepLds &L, const Meta &mt, const AttnSeqs &sq, const uint16_t *__restrict__ qg,
    const uint16_t *__restrict__ kin, const uint16_t *__restrict__ qn_w,
    const uint16_t *__restrict__ kn_w, const uint16_t *__restrict__ rope, const KvRef &kv,
    uint16_t *__restrict__ qn, int nh, int nkv, int nrows, int rpb, uint16_t *__restrict__ tr_kf,
    int qrows) {
    const int32_t *cu = mt.cu, *pos0 = mt.pos0;
    // rows are (token, q head or kv head), or with qrows == 0 (a prefill,
    // whose flash kernel forms its q rows itself) (token, kv head) only
    const int nslot = qrows ? nh + nkv : nkv, s0 = qrows ? 0 : nh;
    const int r0 = bid * rpb, nr = min(rpb, nrows - r0);
    const int tid = threadIdx.x;
    uint16_t *xs = L.xs, *rcs = L.rcs;
    float *rs = L.rs;
    size_t *rdst = L.rdst;
    int *tpos = L.tpos, *thd = L.thd;
    // The block's tokens' metadata first (a lookup chain of a few dependent
    // loads, with nothing else in flight yet), then every row and cos/sin
    // load of the block unconditionally (rows clamped into the block), so
    // no wait drains the stream.
    const int tt0 = r0 / nslot, ntk = (r0 + nr - 1) / nslot - tt0 + 1;
    if (tid < ntk) {
        const int tt = tt0 + tid, s = seq_of(cu, sq.n, tt);
        tpos[tid] = pos0[s] + (tt - cu[s]);
        thd[tid] = mt.hd[s];
    }
    u16x8 xv8[PRB * (D / 8) / 256], cv2[PRB * (ROT / 8) / 256];
#pragma unroll
    for (int k = 0; k < PRB * (D / 8) / 256; k++) {
        const int e = tid + 256 * k, r = min(e / (D / 8), nr - 1), pc = e % (D / 8);
        const int row = r0 + r, tt = row / nslot, slot = s0 + row % nslot;
        const uint16_t *x = slot < nh ? qg + ((size_t)tt * nh + slot) * 2 * D
                                      : kin + ((size_t)tt * nkv + (slot - nh)) * D;
        xv8[k] = *reinterpret_cast<const u16x8 *>(x + pc * 8);
    }
    __syncthreads();                          // the tokens' metadata
#pragma unroll
    for (int k = 0; k < PRB * (ROT / 8) / 256; k++) {
        const int e = tid + 256 * k, r = min(e / (ROT / 8), nr - 1), pc = e % (ROT / 8);
        cv2[k] = *reinterpret_cast<const u16x8 *>(rope + (size_t)tpos[(r0 + r) / nslot - tt0] * ROT + pc * 8);
    }
    if (tid < nr) {                           // k rows' cache offsets, one lane per row
        const int slot = s0 + (r0 + tid) % nslot, ti = (r0 + tid) / nslot - tt0;
        if (slot >= nh) {
            const int pos = tpos[ti];
            rdst[tid] = ((kv_block_id(kv, thd[ti], pos / KVB) * nkv + (slot - nh)) * KVB +
                         pos % KVB) * D;
        }
    }
#pragma unroll
    for (int k = 0; k < PRB * (D / 8) / 256; k++) {
        const int e = tid + 256 * k, r = e / (D / 8), pc = e % (D / 8);
        if (r < nr) *reinterpret_cast<u16x8 *>(xs + r * PRS + pc * 8) = xv8[k];
    }
#pragma unroll
    for (int k = 0; k < PRB * (ROT / 8) / 256; k++) {
        const int e = tid + 256 * k, r = e / (ROT / 8), pc = e % (ROT / 8);
        if (r < nr) *reinterpret_cast<u16x8 *>(rcs + r * ROT + pc * 8) = cv2[k];
    }
    __syncthreads();
    if (tid < nr) {                           // ascending, as the reference sums
        const u16x8 *xr = reinterpret_cast<const u16x8 *>(xs + tid * PRS);
        float ss = 0.0f;
#pragma unroll 4
        for (int j = 0; j < D / 8; j++) {
            const u16x8 v = xr[j];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float f = bf2f(v[i]);
                ss = fmaf(f, f, ss);   // f * f exact: bf16 squared
            }
        }
        rs[tid] = 1.0f / sqrtf(ss / (float)D + kEps);
    }
    __syncthreads();
    constexpr int R = ROT / 2;
    const int p = tid & 31;                   // this thread's piece: dims 8p..8p+7
    const int pp = p ^ (R / 8);               // partner piece (dims +-32) of a rotary pair
    // the (1+w) weights of the piece and of its partner, for q and for k
    const u16x8 wq = *reinterpret_cast<const u16x8 *>(qn_w + p * 8);
    const u16x8 wk = *reinterpret_cast<const u16x8 *>(kn_w + p * 8);
    const u16x8 wqp = *reinterpret_cast<const u16x8 *>(qn_w + pp * 8);
    const u16x8 wkp = *reinterpret_cast<const u16x8 *>(kn_w + pp * 8);
    const int i0 = (p & (R / 8 - 1)) * 8;     // pair index of dim 0 of a rotary piece
    for (int it = 0; it < (nr + 7) / 8; it++) {
        const int r = it * 8 + (tid >> 5);
        if (r >= nr) break;
        const int row = r0 + r, tt = row / nslot, slot = s0 + row % nslot;
        const bool isq = slot < nh;
        const u16x8 wv = isq ? wq : wk;
        const float rr = rs[r];
        const u16x8 xv = *reinterpret_cast<const u16x8 *>(xs + r * PRS + p * 8);
        float n[8];
#pragma unroll
        for (int i = 0; i < 8; i++) n[i] = rndf((bf2f(xv[i]) * rr) * (1.0f + bf2f(wv[i])));
        u16x8 out;
        if (p < ROT / 8) {
            const u16x8 xp = *reinterpret_cast<const u16x8 *>(xs + r * PRS + pp * 8);
            const u16x8 wpv = isq ? wqp : wkp;
            const uint16_t *cs = rcs + r * ROT;
            const u16x8 cv = *reinterpret_cast<const u16x8 *>(cs + i0);
            const u16x8 sv = *reinterpret_cast<const u16x8 *>(cs + R + i0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float np = rndf((bf2f(xp[i]) * rr) * (1.0f + bf2f(wpv[i])));
                const float c = bf2f(cv[i]), sn = bf2f(sv[i]);
                out[i] = p < R / 8 ? f2bf(rndf(n[i] * c) + rndf(-np * sn))
                                   : f2bf(rndf(n[i] * c) + rndf(np * sn));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) out[i] = f2bf(n[i]);
        }
        // (no loads in this loop: a load's wait would also wait for the
        // stores of the iterations before it)
        uint16_t *dst = isq ? qn + ((size_t)tt * nh + slot) * D : kv.k + rdst[r];
        *reinterpret_cast<u16x8 *>(dst + p * 8) = out;
        if (!isq && tr_kf)                    // (trace) the appended k row
            *reinterpret_cast<u16x8 *>(tr_kf + ((size_t)tt * nkv + (slot - nh)) * D + p * 8) = out;
    }
}

// The V append blocks: the new tokens' v rows (raw, c/layer.h:315-316) into the
// transposed V blocks [kv head][d][32]. One block per
// (sequence, kv head, 32-position block the new tokens touch): the rows are
// staged in LDS, then thread d writes its 32 keys -- one 64-byte run, so
// the block is written as contiguous 16 KiB (a block only partly covered
// by new tokens keeps its other keys: element stores for those).
__device__ __forceinline__ void vappend_block(int bid, uint16_t *vt, const Meta &mt,
                                              const uint16_t *__restrict__ vin, const KvRef &kv,
                                              int nkv, int maxnb) {
    const int s = bid / (nkv * maxnb), rem = bid % (nkv * maxnb);
    const int kvh = rem / maxnb, bi = rem % maxnb;
    const int t0 = mt.cu[s], ns = mt.cu[s + 1] - t0, p0 = mt.pos0[s];
    if (ns <= 0) return;
    const int b = p0 / 32 + bi;
    if (b > (p0 + ns - 1) / 32) return;
    const int klo = max(p0, b * 32) - b * 32, khi = min(p0 + ns, b * 32 + 32) - b * 32;
    const int tid = threadIdx.x;
    u16x8 v4[32 * (D / 8) / 256];               // every load in flight at once
#pragma unroll
    for (int j = 0; j < 32 * (D / 8) / 256; j++) {
        const int e = tid + 256 * j, k = e / (D / 8), pc = e % (D / 8);
        if (k >= klo && k < khi) {
            const int t = t0 + (b * 32 + k - p0);
            v4[j] = *reinterpret_cast<const u16x8 *>(vin + ((size_t)t * nkv + kvh) * D + pc * 8);
        }
    }
#pragma unroll
    for (int j = 0; j < 32 * (D / 8) / 256; j++) {
        const int e = tid + 256 * j, k = e / (D / 8), pc = e % (D / 8);
        if (k >= klo && k < khi) *reinterpret_cast<u16x8 *>(vt + k * PRS + pc * 8) = v4[j];
    }
    __syncthreads();
    uint16_t *blk = kv.v + (kv_block_id(kv, mt.hd[s], b) * nkv + kvh) * D * KVB;
    const int d = tid;
    if (klo == 0 && khi == 32) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            u16x8 v;
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = vt[(q * 8 + i) * PRS + d];
            *reinterpret_cast<u16x8 *>(blk + d * 32 + q * 8) = v;
        }
    } else {
        for (int k = klo; k < khi; k++) blk[d * 32 + k] = vt[k * PRS + d];
    }
}

// One launch for both: blocks [0, nprep) are prep blocks of rpb rows,
// the rest V append blocks (B * nkv * maxnb of them). Neither reads what
// the other writes (the K and V caches, qn), so they need no order.
__global__ __launch_bounds__(256) void k_attn_prep(
    AttnSeqs sq, const int32_t *__restrict__ dmeta, const uint16_t *__restrict__ qg,
    const uint16_t *__restrict__ kin, const uint16_t *__restrict__ vin,
    const uint16_t *__restrict__ qn_w, const uint16_t *__restrict__ kn_w,
    const uint16_t *__restrict__ rope, KvRef kv, uint16_t *__restrict__ qn, int nh, int nkv,
    int nrows, int rpb, int nprep, int maxnb, uint16_t *__restrict__ tr_kf, int qrows) {
    __shared__ __attribute__((aligned(16))) char lds[kPrepKernLds];
    const Meta mt = meta_of(sq, dmeta);
    if ((int)blockIdx.x < nprep)
        prep_block((int)blockIdx.x, *reinterpret_cast<PrepLds *>(lds), mt, sq, qg, kin, qn_w,
                   kn_w, rope, kv, qn, nh, nkv, nrows, rpb, tr_kf, qrows);
    else
        vappend_block((int)blockIdx.x - nprep, reinterpret_cast<uint16_t *>(lds), mt, vin, kv,
                      nkv, maxnb);
}

// Row n of the 32 MFMA rows is (token n / GRP, q head n % GRP of the kv
// head); rows past the sequence's tokens are padding.
//
// A segment: keys [k0, k1) of the pair (sequence s, kv head kvh), its
// partial results in slot p + w (p = s*nkv + kvh, w the wavefront's run).
struct Seg {
    int s, kvh, slot, tq, pos0, k0, k1, cap;
    size_t abase;                  // the pair's scores: As + abase (a_index)
};

// A pair's bf16 scores (kRows rows x cap keys) in 1 KiB pieces of 16 rows
// x 32 keys, [row block][32-key chunk][row][key], so that the P.V operand
// loads (16 rows x 32 keys per instruction) read whole lines
__device__ __forceinline__ size_t a_index(int row, int key, int cap) {
    return ((size_t)((row >> 4) * (cap >> 5) + (key >> 5)) * 16 + (row & 15)) * 32 + (key & 31);
}

// a wave-uniform value held in a scalar register (the identity on the
// host, where the split plan is checked)
__host__ __device__ inline int uni(int x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_readfirstlane(x);
#else
    return x;
#endif
}

// The segment of run w (keys x1 > x of the padded pair space) starting at
// x; *xn is where the next one starts. False for a segment that holds only
// padding keys (nothing to compute or store). Host and device: the split
// plan is also walked on the host (apus_hip_attn_split_check).
__host__ __device__ inline bool seg_at(const Meta &mt, int n, int nkv, int w, int x, int x1,
                                       Seg &g, int *xn) {
    const int s = seq_of(mt.ccap, n, x / nkv);
    const int base = nkv * mt.ccap[s], cap = mt.ccap[s + 1] - mt.ccap[s];
    const int local = x - base, kvh = local / cap, k0 = local % cap;
    const int xe = min(x1, base + (kvh + 1) * cap);
    g.s = s;
    g.kvh = kvh;
    g.slot = s * nkv + kvh + w;
    g.tq = mt.cu[s + 1] - mt.cu[s];
    g.pos0 = mt.pos0[s];
    g.k0 = k0;
    g.k1 = min(k0 + (xe - x), g.pos0 + g.tq);
    g.cap = uni(cap);
    g.abase = (size_t)kRows * (size_t)uni(base + kvh * cap);
    *xn = xe;
    return g.k0 < g.k1;
}

// The runs of T keys a pair's real keys fall in: w0 .. w1 (inclusive).
__host__ __device__ inline void pair_runs(const Meta &mt, int nkv, int s, int kvh, int T,
                                          int *w0, int *w1) {
    const int cap = mt.ccap[s + 1] - mt.ccap[s];
    const int ps = nkv * mt.ccap[s] + kvh * cap;
    const int ctx = mt.pos0[s] + mt.cu[s + 1] - mt.cu[s];
    *w0 = ps / T;
    *w1 = (ps + ctx - 1) / T;
}


// The 64-key groups run `run` (keys [run*T, min(run*T + T, total)) of the
// padded pair space) publishes through the score ring: the writer's count,
// formed before it stores anything. The streaming wavefront walks the same
// segments and steps each one's keys by 64 (scores_seg).
__host__ __device__ inline int run_groups(const Meta &mt, int n, int nkv, int run, int T,
                                          int total) {
    int x = run * T, ng = 0;
    const int x1 = min(x + T, total);
    while (x < x1) {
        Seg g;
        int xn;
        if (seg_at(mt, n, nkv, run, x, x1, g, &xn)) ng += (g.k1 - g.k0 + 63) / 64;
        x = xn;
    }
    return ng;
}

// ---- k_attn_scores: W streaming wavefronts + 1 writer per workgroup ------
// Each streaming wavefront owns one run of T1 keys (one or more segments).
// MFMA 16x16x32 bf16 (A: lane l holds row l%16, k (l/16)*8..+8; B: col
// l%16, same k; D: rows (l/16)*4+i, col l%16). S^T[key][row] = K Q^T: the
// four lanes of a key row read 64 contiguous bytes of it per instruction.
// NRB row blocks of 16 (NRB = 2 when a sequence has more than 2 tokens).
//
// The streaming wavefronts issue no global stores. The vector memory
// counter is shared by loads and stores and retires in order, and a store
// issued into a saturated read stream is acknowledged microseconds late, so
// any later wait on a K load would stall behind it (measured: a 3% store mix
// costs ~20% of the stream, whether or not the stores reach HBM). Instead
// each 64-key group's scores go into a per-wavefront LDS ring of kScRing
// slots with a header saying where they belong, a "ready" count in LDS
// publishes them, and the workgroup's last wavefront copies published
// slots to global memory and returns them with a "done" count. A
// wavefront's DS instructions execute in issue order, so a count written
// after its data is never seen before that data.
constexpr int kScRing = 3;
template <int NRB> struct ScoresShape {
    static constexpr int W = NRB == 1 ? 11 : 7;   // streaming wavefronts (+1 writer)
    static constexpr int SLOT = 2 * NRB * 64;     // uint4 per slot: 16*NRB rows x 64 keys
};
template <int NRB> constexpr int scores_waves_per_block() { return ScoresShape<NRB>::W; }

// where a ring slot's scores go: the pair's rows at As + abase (a_index), keys
// kq0 .. min(kq0 + 64, k1), rows of tokens < tq
struct RingHdr {
    uint32_t alo, ahi;
    int cap, kq0, k1, tq;
};

// relaxed workgroup-scope atomics: no cached values, and (unlike volatile)
// no wait on the vector memory counter
__device__ __forceinline__ int lds_count_load(int *p) {
    return __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}
__device__ __forceinline__ void lds_count_store(int *p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// a bounded wait of k_attn_scores expired: tell the workgroup's other
// waves (LDS flag) and the host (the device fault word, read by
// apus_hip_synchronize); vector atomics from one lane
__device__ __forceinline__ void scores_abort(int *abortp, uint32_t *__restrict__ fault) {
    if ((threadIdx.x & 63) == 0) {
        lds_count_store(abortp, 1);
        __hip_atomic_fetch_or(fault, kFaultScoresWait, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// a wave-uniform pointer held in scalar registers
__device__ __forceinline__ const uint16_t *uniform_ptr(const uint16_t *p) {
    const uint64_t a = (uint64_t)p;
    return (const uint16_t *)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(a >> 32))
                               << 32) |
                              (uint32_t)__builtin_amdgcn_readfirstlane((int)a));
}

// K rows of cache block b of segment g (kv head g.kvh); hd its sequence's
// block-table row (read once per segment: a per-group read of it would be
// a vector load whose wait drains the K stream)
__device__ __forceinline__ const uint16_t *kblock(const KvRef &kv, int hd, const Seg &g, int nkv,
                                                  int b) {
    return uniform_ptr(kv.k + (kv_block_id_u(kv, hd, b) * nkv + g.kvh) * KVB * D);
}

// The streaming wavefront's part for one segment whose sequence has NR
// row blocks of queries; grp counts the wavefront's ring groups across its
// segments.
template <int NR, int SLOT>
__device__ __forceinline__ void scores_seg(const Meta &mt, const Seg &c,
                                           const uint16_t *__restrict__ qn, const KvRef &kv,
                                           int nh, int nkv, float scale,
                                           float2 *__restrict__ stats, uint4 *ringw,
                                           RingHdr *hdrw, int *readyw, int *donew, int &grp,
                                           uint4 *stg, int *abortp, uint32_t spin,
                                           uint32_t *__restrict__ fault) {
    const int32_t *cu = mt.cu;
    const int l = threadIdx.x & 63, c16 = l & 15, q4 = l >> 4;

    bf16x8 qf[NR][D / 32];
    int lim[NR];
    bool vrow[NR];
#pragma unroll
    for (int rb = 0; rb < NR; rb++) {
        const int n = rb * 16 + c16, t = n / GRP, g = n % GRP;
        vrow[rb] = t < c.tq;
        lim[rb] = c.pos0 + t;
        const uint16_t *qrow =
            qn + ((size_t)(cu[c.s] + (vrow[rb] ? t : 0)) * nh + c.kvh * GRP + g) * D;
#pragma unroll
        for (int ds = 0; ds < D / 32; ds++) {
            const bf16x8 v = ld_bf16x8(qrow + ds * 32 + q4 * 8);
            qf[rb][ds] = vrow[rb] ? v : bf16x8{};
        }
    }
    float mrun[NR], lrun[NR];
#pragma unroll
    for (int rb = 0; rb < NR; rb++) { mrun[rb] = -INFINITY; lrun[rb] = 0.0f; }

    // Keys are processed in groups of 64 as four MFMA blocks j = 0..3. MFMA
    // row m of block j is key g0 + (m/4)*16 + 4*j + m%4, so the lane whose
    // output rows are m = 4*q4 .. 4*q4+3 ends a group holding the 16
    // consecutive scores g0 + 16*q4 .. +15 of its row: 32 bytes per lane and
    // 128 contiguous bytes per row. K rows past the segment end are clamped
    // to its last row, never zeroed (touching a loaded value on issue would
    // wait for it); their scores are never stored or counted. A group's 64
    // keys lie in two cache blocks (g0 is a multiple of 64); their bases are
    // looked up one group ahead (scalar loads).
    // K rows are read whole: load instruction i reads MFMA rows 2i and
    // 2i+1 of the block (512 contiguous bytes each, lanes 0-31 and 32-63)
    // with the streaming (non-temporal) policy, and the rows pass through
    // this wavefront's LDS tile (row pitch 528 bytes) into the operand
    // layout (lane (q4, c16): row c16, bytes 64 ds + 16 q4). Operand-shaped
    // loads (64 bytes of each of 16 rows per instruction) held the stream
    // at the vector L1's miss rate, and the streaming policy with them
    // lost each line's second half.
    const int blast = (c.k1 - 1) >> 5;
    auto load_k = [&](int g0, int j, int bA, const uint16_t *pA, const uint16_t *pB,
                      u16x8 (&f)[D / 32]) {
#pragma unroll
        for (int i = 0; i < D / 32; i++) {
            const int rr = 2 * i + (l >> 5);
            const int key = min(g0 + (rr >> 2) * 16 + 4 * j + (rr & 3), c.k1 - 1);
            const uint16_t *kr = ((key >> 5) == bA ? pA : pB) + (size_t)(key & 31) * D + (l & 31) * 8;
            f[i] = __builtin_nontemporal_load((gu16x8p)kr);
        }
        // keep the loads here: the scheduler would otherwise sink them to
        // their first use and leave nothing in flight
        __builtin_amdgcn_sched_barrier(0);
    };
    auto stage = [&](const u16x8 (&f)[D / 32]) {
#pragma unroll
        for (int i = 0; i < D / 32; i++)
            stg[(2 * i + (l >> 5)) * 33 + (l & 31)] = __builtin_bit_cast(uint4, f[i]);
    };
    auto unstage = [&](bf16x8 (&k)[D / 32]) {
#pragma unroll
        for (int ds = 0; ds < D / 32; ds++) k[ds] = __builtin_bit_cast(bf16x8, stg[c16 * 33 + ds * 4 + q4]);
    };
    // the first key past which some row's scores are masked
    int kmask = c.k1;
#pragma unroll
    for (int rb = 0; rb < NR; rb++)
        if (vrow[rb]) kmask = min(kmask, lim[rb] + 1);
    kmask = __builtin_amdgcn_readfirstlane(min(kmask, c.pos0 + 1));
    // Double buffering: while one 16-key block is multiplied the next one's
    // 8 loads are in flight (the loads are unconditional: the prefetch past
    // the segment's end re-reads its last row), so the stream never drains
    // between groups.
    // block bases of groups g0 (pA, pB), g0 + 64 (qA, qB); the lookups for
    // g0 + 128 are issued after the group's LDS count read, so their
    // scalar-load latency is never part of an LDS wait
    const int hd = __builtin_amdgcn_readfirstlane(mt.hd[c.s]);
    int bA = min(c.k0 >> 5, blast);
    const uint16_t *pA = kblock(kv, hd, c, nkv, bA), *pB = kblock(kv, hd, c, nkv, min(bA + 1, blast));
    int nA = min((c.k0 + 64) >> 5, blast);
    const uint16_t *qA = kblock(kv, hd, c, nkv, nA), *qB = kblock(kv, hd, c, nkv, min(nA + 1, blast));
    u16x8 kL[D / 32];                       // the next block's rows, as loaded
    bf16x8 kM[D / 32];                      // the current block's operands
    load_k(c.k0, 0, bA, pA, pB, kL);
    for (int g0 = c.k0; g0 < c.k1; g0 += 64, grp++) {
        // the writer must have drained this group's ring slot (read early;
        // it is normally long done)
        const int dn = lds_count_load(donew);
        const int mA = min((g0 + 128) >> 5, blast);
        const uint16_t *rA = kblock(kv, hd, c, nkv, mA), *rB = kblock(kv, hd, c, nkv, min(mA + 1, blast));
        uint32_t sc[NR][8];                  // bf16 score codes, two per word
        auto mma = [&](int j, const bf16x8 *kf) {
            f32x4 acc[NR];
#pragma unroll
            for (int rb = 0; rb < NR; rb++) acc[rb] = f32x4{};
#pragma unroll
            for (int ds = 0; ds < D / 32; ds++)
#pragma unroll
                for (int rb = 0; rb < NR; rb++)
                    acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ds], qf[rb][ds], acc[rb], 0, 0, 0);
            // A = rnd(rnd(q.k) * scale) = rnd(q.k * scale): scale = 1/sqrt(256)
            // is a power of two (hardware RNE, two scores per instruction)
#pragma unroll
            for (int rb = 0; rb < NR; rb++)
#pragma unroll
                for (int e = 0; e < 4; e += 2)
                    sc[rb][2 * j + e / 2] = pack2(acc[rb][e] * scale, acc[rb][e + 1] * scale);
        };
        stage(kL);
        load_k(g0, 1, bA, pA, pB, kL);
        unstage(kM);
        mma(0, kM);
        stage(kL);
        load_k(g0, 2, bA, pA, pB, kL);
        unstage(kM);
        mma(1, kM);
        stage(kL);
        load_k(g0, 3, bA, pA, pB, kL);
        unstage(kM);
        mma(2, kM);
        stage(kL);
        load_k(g0 + 64, 0, nA, qA, qB, kL);
        unstage(kM);
        mma(3, kM);
        bA = nA;
        pA = qA;
        pB = qB;
        nA = mA;
        qA = rA;
        qB = rB;

        // publish the group's scores to the writer through the ring. The
        // wait is bounded: past `spin` polls (or once another wavefront of
        // the workgroup gave up) the call is marked failed in the device
        // fault word and the wavefront runs on without waiting, so every
        // wave still exits
        if (grp >= kScRing && dn <= grp - kScRing) {
            uint32_t polls = 0;
            while (lds_count_load(donew) <= grp - kScRing) {
                if (lds_count_load(abortp) || ++polls > spin) {
                    scores_abort(abortp, fault);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        compiler_fence();
        const int rs = grp % kScRing;
        uint4 *sl = ringw + rs * SLOT;
#pragma unroll
        for (int rb = 0; rb < NR; rb++) {          // row rb*16 + c16, keys 16*q4..+15
            uint4 *r = sl + (rb * 16 + c16) * 8 + 2 * q4;
            r[0] = make_uint4(sc[rb][0], sc[rb][1], sc[rb][2], sc[rb][3]);
            r[1] = make_uint4(sc[rb][4], sc[rb][5], sc[rb][6], sc[rb][7]);
        }
        if (l == 0)
            hdrw[rs] = RingHdr{(uint32_t)c.abase, (uint32_t)(c.abase >> 32), c.cap, g0, c.k1, c.tq};
        compiler_fence();
        if (l == 0) lds_count_store(readyw, grp + 1);

        const int kq = g0 + 16 * q4;           // this lane's 16 keys
#pragma unroll
        for (int rb = 0; rb < NR; rb++) {
            if (!vrow[rb]) continue;
            float a[16];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                a[2 * e] = __uint_as_float(sc[rb][e] << 16);
                a[2 * e + 1] = __uint_as_float(sc[rb][e] & 0xffff0000u);
            }
            if (g0 + 64 > kmask) {             // (wave-uniform) keys past a query or the segment
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int kk = kq + e;
                    if (!(kk <= lim[rb] && kk < c.k1)) a[e] = -INFINITY;
                }
            }
            float bmax = a[0];
#pragma unroll
            for (int e = 1; e < 16; e++) bmax = fmaxf(bmax, a[e]);
            if (bmax > -INFINITY) {
                // running (max, sum of e^{A - m}) with the hardware exp2
                const float mn = fmaxf(mrun[rb], bmax), kn = mn * kL2E;
                float add = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) add += __builtin_amdgcn_exp2f(fmaf(a[e], kL2E, -kn));
                lrun[rb] = lrun[rb] * __builtin_amdgcn_exp2f((mrun[rb] - mn) * kL2E) + add;
                mrun[rb] = mn;
            }
        }
    }
    // the four lanes l%16 + {0,16,32,48} hold the key quarters of one row
#pragma unroll
    for (int rb = 0; rb < NR; rb++) {
        float m = mrun[rb], ls = lrun[rb];
#pragma unroll
        for (int off = 16; off < 64; off <<= 1) {
            const float mo = __shfl_xor(m, off), lo = __shfl_xor(ls, off);
            const float mm = fmaxf(m, mo);
            ls = mm > -INFINITY ? ls * exp_fast(m - mm) + lo * exp_fast(mo - mm) : 0.0f;
            m = mm;
        }
        if (q4 == 0 && vrow[rb]) stats[(size_t)c.slot * kRows + rb * 16 + c16] = make_float2(m, ls);
    }
}

template <int NRB>
__global__ __launch_bounds__(64 * (ScoresShape<NRB>::W + 1)) void k_attn_scores(
    AttnSeqs sq, const int32_t *__restrict__ dmeta, const uint16_t *__restrict__ qn, KvRef kv,
    int nh, int nkv, float scale, uint16_t *__restrict__ As, float2 *__restrict__ stats,
    int nruns, uint32_t spin, uint32_t *__restrict__ fault) {
    constexpr int W = ScoresShape<NRB>::W, SLOT = ScoresShape<NRB>::SLOT;
    __shared__ uint4 ring[W][kScRing][SLOT];
    __shared__ uint4 kstage[W][16 * 33];            // per wavefront: one 16-key K block
    __shared__ RingHdr hdr[W][kScRing];
    __shared__ int ready[W], done[W], abort_flag;
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
    if (threadIdx.x < W) {
        ready[threadIdx.x] = 0;
        done[threadIdx.x] = 0;
    }
    if (threadIdx.x == 0) abort_flag = 0;
    __syncthreads();
    const Meta mt = meta_of(sq, dmeta);
    const int n = sq.n, T = sq.T1, total = nkv * mt.ccap[n];

    if (wave == W) {
        // ---- writer: copy published slots of the W runs to global memory.
        // The group counts are computed before any store is issued: a load
        // after a store would wait for the store's acknowledgement.
        int nxt[W], ng[W];
#pragma unroll
        for (int w = 0; w < W; w++) {
            nxt[w] = 0;
            const int run = blockIdx.x * W + w;
            ng[w] = run < nruns ? run_groups(mt, n, nkv, run, T, total) : 0;
        }
        // the writer's polls over its life, bounded like the streaming
        // wavefronts' waits (a normal launch makes a few thousand at most;
        // a run of more groups than the ring holds always needs two)
        uint32_t polls = 0;
        for (;;) {
            bool left = false, moved = false;
#pragma unroll
            for (int w = 0; w < W; w++) {
                if (nxt[w] >= ng[w]) continue;
                left = true;
                const int rd = lds_count_load(&ready[w]);
                if (rd <= nxt[w]) continue;
                compiler_fence();
                // slot layout [row][64 keys]: lane l stores 16 bytes (8 keys)
                // of row 8*i + l/8, two 64-byte runs a row. The streaming
                // policy: with the default one the dirty score lines were
                // written back from L2 while P.V streamed V (config 4: P.V
                // 222 -> 204 us, scores 206 -> 214 us)
                for (int g = nxt[w]; g < rd; g++) {
                    const uint4 *sl = ring[w][g % kScRing];
                    const RingHdr h = hdr[w][g % kScRing];
                    uint16_t *Ab = As + (((size_t)h.ahi << 32) | h.alo);
                    const int kq = h.kq0 + 8 * (l & 7);
#pragma unroll
                    for (int i = 0; i < 2 * NRB; i++) {
                        const int row = 8 * i + (l >> 3);
                        if (row / GRP < h.tq && kq < h.k1)
                            __builtin_nontemporal_store(
                                __builtin_bit_cast(u16x8, sl[i * 64 + l]),
                                reinterpret_cast<u16x8 *>(Ab + a_index(row, kq, h.cap)));
                    }
                }
                compiler_fence();
                nxt[w] = rd;
                if (l == 0) lds_count_store(&done[w], rd);
                moved = true;
            }
            if (!left) break;
            if (lds_count_load(&abort_flag) || ++polls > spin) {
                scores_abort(&abort_flag, fault);
                break;
            }
            if (!moved) __builtin_amdgcn_s_sleep(2);
        }
        return;
    }

    // ---- streaming wavefront: its run's segments in order
    const int run = blockIdx.x * W + wave;
    if (run >= nruns) return;
    int x = run * T, grp = 0;
    const int x1 = min(x + T, total);
    while (x < x1) {
        Seg g;
        int xn;
        if (seg_at(mt, n, nkv, run, x, x1, g, &xn)) {
            // a sequence with at most 2 tokens fills one row block
            if (NRB == 2 && g.tq <= 2)
                scores_seg<1, SLOT>(mt, g, qn, kv, nh, nkv, scale, stats, ring[wave][0],
                                    hdr[wave], &ready[wave], &done[wave], grp, kstage[wave],
                                    &abort_flag, spin, fault);
            else
                scores_seg<NRB, SLOT>(mt, g, qn, kv, nh, nkv, scale, stats, ring[wave][0],
                                      hdr[wave], &ready[wave], &done[wave], grp, kstage[wave],
                                      &abort_flag, spin, fault);
        }
        x = xn;
    }
}

// ---- k_attn_pv: one run of T2 keys per item ------------------------------
// O^T[d][row] = sum_key V^T[d][key] P^T[key][row] on MFMA 16x16x32: the
// transposed V blocks are the A operand (4 lanes read 64 contiguous bytes
// of one d row), the probabilities the B operand. DH = 2 wavefronts share a
// run, each owning half of the d rows: the accumulators and the next
// step's V operands then fit three wavefronts per SIMD for one row block
// and two for two.
// P.V over one segment for a sequence with NR row blocks of queries; this
// wavefront owns d blocks hb*NB .. +NB
template <int NR, int NB>
__device__ __forceinline__ void pv_seg(const Meta &mt, const Seg &c, int hb, const AttnSeqs &sq,
                                       const KvRef &kv, int nkv, const uint16_t *__restrict__ As,
                                       const float2 *__restrict__ stats, float *__restrict__ Op) {
    const int l = threadIdx.x, c16 = l & 15, q4 = l >> 4;

    // global (max, sum) of each row over the pair's score segments
    int w0, w1;
    pair_runs(mt, nkv, c.s, c.kvh, sq.T1, &w0, &w1);
    const int p = c.s * nkv + c.kvh;
    float m[NR], rsum[NR];
    bool vrow[NR];
    int lim[NR];
#pragma unroll
    for (int rb = 0; rb < NR; rb++) {
        const int n = rb * 16 + c16, t = n / GRP;
        vrow[rb] = t < c.tq;
        lim[rb] = c.pos0 + t;
        float mm = -INFINITY, ss = 0.0f;
        if (vrow[rb]) {
            // eight segments' statistics in flight at a time (a long pair
            // has dozens; one dependent load each would serialise their
            // latencies)
            for (int w = w0; w <= w1; w += 8) {
                float2 st[8];
#pragma unroll
                for (int i = 0; i < 8; i++)
                    st[i] = w + i <= w1 ? stats[(size_t)(p + w + i) * kRows + n]
                                        : make_float2(-INFINITY, 0.0f);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (st[i].x == -INFINITY) continue;
                    const float mn = fmaxf(mm, st[i].x);
                    ss = ss * exp_fast(mm - mn) + st[i].y * exp_fast(st[i].x - mn);
                    mm = mn;
                }
            }
        }
        // P = rnd(e^{A - m} / s) formed as rnd(exp2(A log2(e) - K)), K =
        // m log2(e) + log2(s): the division folded into the exponent (a
        // relative difference of a few 1e-7 from the quotient, the
        // tolerance class of the hardware exp2)
        m[rb] = mm;
        rsum[rb] = mm * kL2E + __builtin_amdgcn_logf(ss);
    }
    const uint16_t *Ab = As + c.abase;
    f32x4 acc[NR][NB];
#pragma unroll
    for (int rb = 0; rb < NR; rb++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[rb][b] = f32x4{};

    // V^T and score fragments of the next 32-key step are loaded while the
    // current step is multiplied. Loads never touch their value on issue
    // (that would wait for them): addresses are clamped into the segment's
    // valid 8-key groups and the out-of-range keys are masked at use. A
    // step's 32 keys are one cache block (its base a scalar lookup).
    const int kclamp = ((c.k1 - 1) / 8) * 8;   // last aligned group holding a valid key
    const int kmask = min(c.k1, c.pos0 + 1);   // the first key masked for some row
    const int hd = __builtin_amdgcn_readfirstlane(mt.hd[c.s]);   // (read once, into a scalar)
    // V block of the step at kb (clamped lanes stay in kb's block: kclamp
    // lies in [kb, kb + 24] whenever kb + 8*q4 passes it)
    auto vblock = [&](int kb) {
        return uniform_ptr(kv.v + (kv_block_id_u(kv, hd, min(kb, c.k1 - 1) >> 5) * nkv + c.kvh) *
                                      D * KVB);
    };
    u16x8 vf[NB], af[NR];
    auto load_step = [&](int kb, const uint16_t *Vb, u16x8 *fv, u16x8 *fa) {
        const int kq = min(kb + q4 * 8, kclamp);
#pragma unroll
        for (int b = 0; b < NB; b++)
            fv[b] = __builtin_nontemporal_load((gu16x8p)(Vb + ((hb * NB + b) * 16 + c16) * KVB + (kq & 31)));
#pragma unroll
        for (int rb = 0; rb < NR; rb++)
            fa[rb] = gld16(Ab + a_index(rb * 16 + c16, kq, c.cap));
    };
    load_step(c.k0, vblock(c.k0), vf, af);
    for (int kb = c.k0; kb < c.k1; kb += 32) {
        // the next step's operands, unconditionally (past the segment's end
        // the clamped addresses re-read its last step): a branch around
        // the loads would make the compiler wait for them at its join
        u16x8 vn[NB], an[NR];
        load_step(kb + 32, vblock(kb + 32), vn, an);
        const int kq = kb + q4 * 8;            // this lane's 8 keys
        bf16x8 pf[NR];
#pragma unroll
        for (int rb = 0; rb < NR; rb++) {
            // (rows of absent tokens are left unmasked: never written out)
            f32x8 e8;
#pragma unroll
            for (int e = 0; e < 8; e++)
                e8[e] = __builtin_amdgcn_exp2f(fmaf(bf2f(af[rb][e]), kL2E, -rsum[rb]));
            if (kb + 32 > kmask) {             // (wave-uniform) keys past a query or the segment
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (!(kq + e <= lim[rb] && kq + e < c.k1)) e8[e] = 0.0f;
            }
            pf[rb] = __builtin_convertvector(e8, bf16x8);     // hardware RNE
        }
        const bool partial = kq + 8 > c.k1;    // keys past the end: zero V too
#pragma unroll
        for (int b = 0; b < NB; b++) {
            u16x8 v8 = vf[b];
            if (partial)
                for (int e = 0; e < 8; e++)
                    if (kq + e >= c.k1) v8[e] = 0;
            const bf16x8 va = __builtin_bit_cast(bf16x8, v8);
#pragma unroll
            for (int rb = 0; rb < NR; rb++)
                acc[rb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[rb], acc[rb][b], 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) vf[b] = vn[b];
#pragma unroll
        for (int rb = 0; rb < NR; rb++) af[rb] = an[rb];
    }
#pragma unroll
    for (int rb = 0; rb < NR; rb++) {
        if (!vrow[rb]) continue;
        float *orow = Op + ((size_t)c.slot * kRows + rb * 16 + c16) * D;
#pragma unroll
        for (int b = 0; b < NB; b++)
            *reinterpret_cast<float4 *>(orow + (hb * NB + b) * 16 + q4 * 4) =
                make_float4(acc[rb][b][0], acc[rb][b][1], acc[rb][b][2], acc[rb][b][3]);
    }
}

template <int NRB, int DH>
__global__ __launch_bounds__(64) void k_attn_pv(
    AttnSeqs sq, const int32_t *__restrict__ dmeta, KvRef kv, int nkv,
    const uint16_t *__restrict__ As, const float2 *__restrict__ stats, float *__restrict__ Op) {
    const Meta mt = meta_of(sq, dmeta);
    constexpr int NB = D / 16 / DH;            // 16-row d blocks of this wavefront
    const int hb = DH == 1 ? 0 : (int)(blockIdx.x % DH);
    const int run = (int)(blockIdx.x / DH), n = sq.n, T = sq.T2;
    int x = run * T;
    const int x1 = min(x + T, nkv * mt.ccap[n]);
    while (x < x1) {
        Seg g;
        int xn;
        if (seg_at(mt, n, nkv, run, x, x1, g, &xn)) {
            // a sequence with at most 2 tokens fills one row block
            if (NRB == 2 && g.tq <= 2)
                pv_seg<1, NB>(mt, g, hb, sq, kv, nkv, As, stats, Op);
            else
                pv_seg<NRB, NB>(mt, g, hb, sq, kv, nkv, As, stats, Op);
        }
        x = xn;
    }
}

// ---- k_attn_combine: one block per (token, kv head, 4 of its q heads) --
// A thread owns 4 consecutive d of one (token, q head) row: its gate codes
// are loaded first, then up to 16 of the pair's run partials at once
// (float4 each), summed in run order from 0.0f; rnd, times
// rnd(sigmoid(gate)). One block per (token, q head) with a thread per d
// needed three rounds of resident waves on config 4, each a chain of
// dependent loads.
__global__ __launch_bounds__(256) void k_attn_combine(
    AttnSeqs sq, const int32_t *__restrict__ dmeta, const float *__restrict__ Op,
    const uint16_t *__restrict__ qg, int nh, int nkv, uint16_t *__restrict__ y,
    const uint16_t *__restrict__ sig_bf, uint16_t *__restrict__ tr_attno) {
    const Meta mt = meta_of(sq, dmeta);
    const int half = blockIdx.x & 1, tk = blockIdx.x >> 1;
    const int tt = tk / nkv, kvh = tk % nkv;
    const int s = seq_of(mt.cu, sq.n, tt), t = tt - mt.cu[s];
    const int g = half * (GRP / 2) + (threadIdx.x >> 6), h = kvh * GRP + g, n = t * GRP + g;
    const int d = (threadIdx.x & 63) * 4;
    const size_t row = (size_t)tt * nh + h;
    const uint2 gc = *reinterpret_cast<const uint2 *>(qg + row * 2 * D + D + d);
    int w0, w1;
    pair_runs(mt, nkv, s, kvh, sq.T2, &w0, &w1);
    const int nw = w1 - w0;
    const float *P0 = Op + ((size_t)(s * nkv + kvh + w0) * kRows + n) * D + d;
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int w = 0; w <= nw; w += 16) {
        f32x4 v[16];
#pragma unroll
        for (int i = 0; i < 16; i++)
            v[i] = *reinterpret_cast<const f32x4 *>(P0 + (size_t)min(w + i, nw) * kRows * D);
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (w + i <= nw) sum += v[i];
    }
    const uint16_t code[4] = {(uint16_t)gc.x, (uint16_t)(gc.x >> 16), (uint16_t)gc.y,
                              (uint16_t)(gc.y >> 16)};
    uint16_t yo[4], ao[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float o = rndf(sum[e]);
        ao[e] = f2bf(o);
        yo[e] = f2bf(o * bf2f(sig_bf[code[e]]));       // rnd(sigmoid(gate))
    }
    *reinterpret_cast<uint2 *>(y + row * D + d) =
        make_uint2(yo[0] | (uint32_t)yo[1] << 16, yo[2] | (uint32_t)yo[3] << 16);
    if (tr_attno)                                        // (trace)
        *reinterpret_cast<uint2 *>(tr_attno + row * D + d) =
            make_uint2(ao[0] | (uint32_t)ao[1] << 16, ao[2] | (uint32_t)ao[3] << 16);
}

// (trace) mgate = rnd(sigmoid(gate)) for every (token, head, d)
__global__ void k_trace_mgate(const uint16_t *__restrict__ qg, size_t n, int nh,
                              const uint16_t *__restrict__ sig_bf, uint16_t *__restrict__ mg) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n) return;
    const size_t row = e / D, dd = e % D;     // row = token * nh + head
    mg[e] = sig_bf[qg[row * 2 * D + D + dd]];
    (void)nh;
}

// ---- cache layout conversion (one sequence: block-table row h) ---------
// reference layout [ntok][nkv][D] <-> the cache blocks of row h
__global__ void k_cache_pack(const uint16_t *__restrict__ kref, const uint16_t *__restrict__ vref,
                             size_t ntok, int nkv, KvRef kv, int h) {
    size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= ntok * nkv * D) return;
    size_t p = e / (nkv * D), r = e % (nkv * D);
    int hk = (int)(r / D), dd = (int)(r % D);
    const size_t id = kv_block_id(kv, h, (int)(p / KVB)) * nkv + hk;
    kv.k[(id * KVB + p % KVB) * D + dd] = kref[e];
    kv.v[(id * D + dd) * KVB + p % KVB] = vref[e];
}

__global__ void k_cache_unpack(KvRef kv, int h, size_t ntok, int nkv,
                               uint16_t *__restrict__ kref, uint16_t *__restrict__ vref) {
    size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= ntok * nkv * D) return;
    size_t p = e / (nkv * D), r = e % (nkv * D);
    int hk = (int)(r / D), dd = (int)(r % D);
    const size_t id = kv_block_id(kv, h, (int)(p / KVB)) * nkv + hk;
    kref[e] = kv.k[(id * KVB + p % KVB) * D + dd];
    vref[e] = kv.v[(id * D + dd) * KVB + p % KVB];
}

}  // namespace

namespace apus {

int attn_check_layer(const ApusHipAttnLayer *L) {
    if (!L) return set_error(kErrArgument, "NULL layer");
    if (L->d != (size_t)D || L->rot != (size_t)ROT || L->nkv == 0 ||
        L->nh != (size_t)GRP * L->nkv)
        return set_error(kErrUnsupported,
                         "attention mixer supports d=256, rot=64, nh=8*nkv (got nh=%zu "
                         "nkv=%zu d=%zu rot=%zu)", L->nh, L->nkv, L->d, L->rot);
    return kOk;
}

KvRef kv_flat(uint16_t *kcache, uint16_t *vcache, size_t max_seq) {
    return KvRef{kcache, vcache, nullptr, (int32_t)(max_seq / KVB)};
}

static size_t ceil64(size_t x) { return (x + 63) / 64 * 64; }

// decode: balanced runs of T keys per wavefront over `total` padded keys,
// each kernel's grid one round of resident wavefronts (scores: W streaming
// wavefronts per CU; P.V: two wavefronts per run, each owning half of d,
// at three wavefronts per SIMD for one row block, two for two)
static void attn_split_sizes(size_t total, size_t max_tok, size_t cus, int32_t *T1, int32_t *T2) {
    const size_t w1 = (max_tok <= 2 ? scores_waves_per_block<1>() : scores_waves_per_block<2>()) * cus;
    const size_t w2 = (max_tok <= 2 ? 3 : 2) * 4 * cus / 2;
    *T1 = (int32_t)std::max<size_t>(64, ceil64((total + w1 - 1) / w1));
    *T2 = (int32_t)std::max<size_t>(64, ceil64((total + w2 - 1) / w2));
}

int attn_meta(size_t B, const int32_t *cu, const int32_t *pos0, const int32_t *rows,
              size_t bstride, size_t nkv, int max_new, AttnSeqs *sq, const int32_t **dmeta,
              size_t *max_tok) {
    if (!cu || !pos0 || cu[0] != 0) return set_error(kErrArgument, "bad offsets");
    std::vector<int32_t> ccap(B + 1, 0);
    size_t mt = 0;
    for (size_t s = 0; s < B; s++) {
        const int32_t tq = cu[s + 1] - cu[s];
        if (tq < 0) return set_error(kErrArgument, "token offsets must ascend");
        if (max_new > 0 && (tq < 1 || tq > max_new))
            return set_error(kErrUnsupported, "decode takes 1..%d new tokens per sequence (got %d)",
                             max_new, tq);
        if (pos0[s] < 0 || (size_t)pos0[s] + (size_t)tq > bstride * KVB)
            return set_error(kErrArgument, "sequence %zu overflows the cache (%d+%d > %zu)", s,
                             pos0[s], tq, bstride * KVB);
        if (rows && rows[s] < 0) return set_error(kErrArgument, "negative block-table row");
        const size_t cap = ceil64((size_t)pos0[s] + (size_t)tq);
        if (nkv * ((size_t)ccap[s] + cap) > (size_t)0x7ff00000)
            return set_error(kErrUnsupported, "too many cached keys in one call");
        ccap[s + 1] = ccap[s] + (int32_t)cap;
        if ((size_t)tq > mt) mt = (size_t)tq;
    }
    *max_tok = mt;
    attn_split_sizes(nkv * (size_t)ccap[B], mt, (size_t)cu_count(), &sq->T1, &sq->T2);
    sq->n = (int32_t)B;
    *dmeta = nullptr;
    if (B <= (size_t)kAttnInlineSeqs) {
        memcpy(sq->cu, cu, (B + 1) * 4);
        memcpy(sq->pos0, pos0, B * 4);
        memcpy(sq->ccap, ccap.data(), (B + 1) * 4);
        for (size_t s = 0; s < B; s++) sq->hd[s] = rows ? rows[s] : (int32_t)s;
    } else {
        std::vector<int32_t> m(4 * B + 2);
        memcpy(m.data(), cu, (B + 1) * 4);
        memcpy(m.data() + B + 1, pos0, B * 4);
        memcpy(m.data() + 2 * B + 1, ccap.data(), (B + 1) * 4);
        for (size_t s = 0; s < B; s++) m[3 * B + 2 + s] = rows ? rows[s] : (int32_t)s;
        *dmeta = (const int32_t *)upload_async(m.data(), m.size() * 4);
        if (!*dmeta) return kErrHip;
    }
    return kOk;
}

int attn_prep(const ApusHipAttnLayer *L, const AttnSeqs &sq, const int32_t *dmeta,
              size_t Ttot, size_t max_pos, int maxnb, const uint16_t *qg, const uint16_t *k,
              const uint16_t *v, const KvRef &kv, uint16_t *qn, bool qrows) {
    const uint16_t *rope = rope_table(L->rot, L->theta, max_pos);
    if (!rope) return kErrHip;
    const size_t nrows = Ttot * (qrows ? L->nh + L->nkv : L->nkv);
    // few rows (decode): small blocks, so they spread over the chip
    const int rpb = nrows < (size_t)8 * PRB * cu_count() ? 8 : PRB;
    const unsigned nprep = cdiv(nrows, rpb), nvapp = (unsigned)(sq.n * L->nkv * maxnb);
    APUS_TIMED("k_attn_prep",
               k_attn_prep<<<nprep + nvapp, 256, 0, stream()>>>(
        sq, dmeta, qg, k, v, L->qn_w, L->kn_w, rope, kv, qn, (int)L->nh, (int)L->nkv,
        (int)nrows, rpb, (int)nprep, maxnb, attn_trace() ? attn_trace()->kf : nullptr,
        qrows ? 1 : 0));
    if (int r = launch_check("k_attn_prep")) return r;
    if (const ApusHipAttnTrace *tr = attn_trace()) {
        if (tr->qf && qrows)
            APUS_HIP_TRY(hipMemcpyAsync(tr->qf, qn, Ttot * L->nh * D * 2, hipMemcpyDeviceToDevice,
                                        stream()));
        if (tr->mgate) {
            const ActTables *tabs = act_tables();
            if (!tabs) return kErrHip;
            const size_t n = Ttot * L->nh * D;
            k_trace_mgate<<<cdiv(n, 256), 256, 0, stream()>>>(qg, n, (int)L->nh, tabs->sig_bf,
                                                               tr->mgate);
            if (int r = launch_check("k_trace_mgate")) return r;
        }
    }
    return kOk;
}

// the most 32-position cache blocks one sequence's new tokens touch
int attn_max_vblocks(size_t B, const int32_t *cu, const int32_t *pos0) {
    int m = 1;
    for (size_t s = 0; s < B; s++) {
        const int ns = cu[s + 1] - cu[s];
        if (ns > 0) m = std::max(m, (pos0[s] + ns - 1) / KVB - pos0[s] / KVB + 1);
    }
    return m;
}

int attn_decode_kv(const ApusHipAttnLayer *L, size_t B, const int32_t *cu, const int32_t *pos0,
                   const int32_t *rows, const uint16_t *qg, const uint16_t *k,
                   const uint16_t *v, const KvRef &kv, uint16_t *y) {
    if (int r = attn_check_layer(L)) return r;
    if (B == 0) return kOk;
    AttnSeqs sq;
    const int32_t *dmeta = nullptr;
    size_t mt = 0;
    if (int r = attn_meta(B, cu, pos0, rows, (size_t)kv.bstride, L->nkv, kRows / GRP, &sq, &dmeta,
                          &mt))
        return r;
    const size_t Ttot = (size_t)cu[B], nkv = L->nkv;
    size_t max_pos = 0, keys = 0;
    for (size_t s = 0; s < B; s++) {
        max_pos = std::max(max_pos, (size_t)pos0[s] + (size_t)(cu[s + 1] - cu[s]));
        keys += ceil64((size_t)pos0[s] + (size_t)(cu[s + 1] - cu[s]));
    }
    const size_t total = nkv * keys;
    const size_t nruns1 = (total + sq.T1 - 1) / sq.T1, nruns2 = (total + sq.T2 - 1) / sq.T2;
    uint16_t *qn = (uint16_t *)scratch(kScratchAttnQ, Ttot * L->nh * D * 2);
    uint16_t *As = (uint16_t *)scratch(kScratchAttnA, total * kRows * 2);
    float2 *st = (float2 *)scratch(kScratchAttnStat, (nruns1 + B * nkv) * kRows * 8);
    float *Op = (float *)scratch(kScratchAttnPart, (nruns2 + B * nkv) * kRows * D * 4);
    if (!qn || !As || !st || !Op) return kErrHip;
    if (int r = attn_prep(L, sq, dmeta, Ttot, max_pos, attn_max_vblocks(B, cu, pos0), qg, k, v,
                          kv, qn))
        return r;
    const float scale = (float)(1.0 / sqrt((double)L->d));
    const ActTables *tabs = act_tables();
    if (!tabs) return kErrHip;
    // one 16-row block covers up to 2 new tokens per sequence (8 heads each)
    if (mt <= 2) {
        APUS_TIMED("k_attn_scores",
                   k_attn_scores<1><<<cdiv(nruns1, scores_waves_per_block<1>()),
                                      64 * (scores_waves_per_block<1>() + 1), 0, stream()>>>(
                       sq, dmeta, qn, kv, (int)L->nh, (int)nkv, scale, As, st, (int)nruns1,
                       spin_limit(), fault_word()));
        APUS_LAUNCHED("k_attn_scores");
        APUS_TIMED("k_attn_pv",
                   k_attn_pv<1, 2><<<(unsigned)(2 * nruns2), 64, 0, stream()>>>(
                       sq, dmeta, kv, (int)nkv, As, st, Op));
        APUS_LAUNCHED("k_attn_pv");
    } else {
        APUS_TIMED("k_attn_scores",
                   k_attn_scores<2><<<cdiv(nruns1, scores_waves_per_block<2>()),
                                      64 * (scores_waves_per_block<2>() + 1), 0, stream()>>>(
                       sq, dmeta, qn, kv, (int)L->nh, (int)nkv, scale, As, st, (int)nruns1,
                       spin_limit(), fault_word()));
        APUS_LAUNCHED("k_attn_scores");
        APUS_TIMED("k_attn_pv",
                   k_attn_pv<2, 2><<<(unsigned)(2 * nruns2), 64, 0, stream()>>>(
                       sq, dmeta, kv, (int)nkv, As, st, Op));
        APUS_LAUNCHED("k_attn_pv");
    }
    APUS_TIMED("k_attn_combine",
               k_attn_combine<<<(unsigned)(Ttot * nkv * 2), 256, 0, stream()>>>(
                   sq, dmeta, Op, qg, (int)L->nh, (int)nkv, y, tabs->sig_bf,
                   attn_trace() ? attn_trace()->attno : nullptr));
    APUS_LAUNCHED("k_attn_combine");
    return kOk;
}

int kv_paged_ref(const ApusHipKvCache *c, size_t B, const int32_t *rows, const int32_t *cu,
                 const int32_t *pos0, KvRef *r) {
    if (!c || !c->k || !c->v || !c->block_table || c->max_blocks == 0 ||
        c->max_blocks > 0x7fffffff || c->max_rows == 0 || c->max_rows > 0x7fffffff)
        return set_error(kErrArgument, "bad paged KV cache descriptor");
    if (!rows) return set_error(kErrArgument, "NULL block-table rows");
    if (B && (!cu || !pos0)) return set_error(kErrArgument, "NULL offsets");
    for (size_t s = 0; s < B; s++) {
        if (rows[s] < 0 || (size_t)rows[s] >= c->max_rows)
            return set_error(kErrArgument, "block-table row %d of sequence %zu is outside the "
                             "table's %zu rows", rows[s], s, c->max_rows);
        if (!c->row_blocks) continue;
        // positions 0 .. pos0 + new - 1 must lie in blocks the row holds
        const int64_t end = (int64_t)pos0[s] + (int64_t)(cu[s + 1] - cu[s]);
        const int32_t held = c->row_blocks[rows[s]];
        if (held < 0)
            return set_error(kErrArgument, "block-table row %d of sequence %zu is not open",
                             rows[s], s);
        if (end > (int64_t)held * KVB)
            return set_error(kErrArgument, "sequence %zu reaches position %lld but row %d has "
                             "reserved %d positions", s, (long long)end, rows[s], held * KVB);
    }
    *r = KvRef{c->k, c->v, c->block_table, (int32_t)c->max_blocks};
    return kOk;
}

}  // namespace apus

extern "C" {

int apus_hip_attn_decode(const ApusHipAttnLayer *L, size_t B, const int32_t *cu,
                         const int32_t *pos0, const uint16_t *qg, const uint16_t *k,
                         const uint16_t *v, uint16_t *kcache, uint16_t *vcache,
                         size_t max_seq, uint16_t *y) {
    APUS_READY();
    if (max_seq % KVB != 0) return set_error(kErrArgument, "max_seq must be a multiple of %d", KVB);
    return attn_decode_kv(L, B, cu, pos0, nullptr, qg, k, v, kv_flat(kcache, vcache, max_seq), y);
}

int apus_hip_attn_decode_paged(const ApusHipAttnLayer *L, size_t B, const int32_t *rows,
                               const int32_t *cu, const int32_t *pos0, const uint16_t *qg,
                               const uint16_t *k, const uint16_t *v, const ApusHipKvCache *kv,
                               uint16_t *y) {
    APUS_READY();
    KvRef r;
    if (int e = kv_paged_ref(kv, B, rows, cu, pos0, &r)) return e;
    return attn_decode_kv(L, B, cu, pos0, rows, qg, k, v, r, y);
}

// Host walk of the decode split plan for a batch (no device needed): the
// scores kernel's two enumerations of each run's 64-key groups, the
// writer's (run_groups) and the streaming wavefront's (its segments' keys
// stepped by 64), must agree or the ring's producer / consumer waits would
// not meet; every real key of every (sequence, kv head) pair must fall in
// exactly one segment; segment slots must be distinct and inside the
// statistics buffer; and the runs P.V folds for a pair (pair_runs) must be
// exactly the runs holding one of its segments. out[12]: runs, runs whose
// two counts differ, writer groups, streaming groups, keys missed or
// covered twice, slot collisions or overflows, pair_runs mismatches, T1,
// and (the same for P.V's runs of T2) runs, keys missed or covered twice,
// slot problems, pair_runs mismatches.
int apus_hip_attn_split_check(size_t B, const int32_t *cu, const int32_t *pos0, size_t nkv,
                              size_t cus, int64_t *out) {
    if (!cu || !pos0 || !out || B == 0 || nkv == 0 || cus == 0 || cu[0] != 0)
        return set_error(kErrArgument, "bad split-check arguments");
    std::vector<int32_t> ccap(B + 1, 0), hd(B);
    size_t mt = 0;
    for (size_t s = 0; s < B; s++) {
        const int32_t tq = cu[s + 1] - cu[s];
        if (tq < 1 || tq > kRows / GRP || pos0[s] < 0)
            return set_error(kErrArgument, "sequence %zu: 1..4 new tokens after pos0 >= 0", s);
        ccap[s + 1] = ccap[s] + (int32_t)ceil64((size_t)pos0[s] + tq);
        mt = std::max<size_t>(mt, (size_t)tq);
        hd[s] = (int32_t)s;
    }
    const size_t total = nkv * (size_t)ccap[B];
    if (total > (size_t)0x7ff00000) return set_error(kErrArgument, "too many keys");
    int32_t T[2];
    attn_split_sizes(total, mt, cus, &T[0], &T[1]);
    const Meta m{cu, pos0, ccap.data(), hd.data()};
    const int n = (int)B;
    for (int i = 0; i < 12; i++) out[i] = 0;
    out[7] = T[0];
    for (int k = 0; k < 2; k++) {
        const int Tk = T[k];
        const size_t nruns = (total + Tk - 1) / Tk;
        int64_t *o = k == 0 ? out : out + 8;       // runs, keys, slots, pair_runs
        std::vector<uint8_t> cover(total, 0), slot_used(nruns + B * nkv, 0);
        std::vector<std::vector<int>> pair_seg_runs(B * nkv);
        o[0] = (int64_t)nruns;
        for (size_t run = 0; run < nruns; run++) {
            int x = (int)(run * Tk), sg = 0;
            const int x1 = (int)std::min<size_t>((size_t)x + Tk, total);
            while (x < x1) {
                Seg g;
                int xn;
                if (seg_at(m, n, (int)nkv, (int)run, x, x1, g, &xn)) {
                    for (int g0 = g.k0; g0 < g.k1; g0 += 64) sg++;   // scores_seg's loop
                    const size_t base = (size_t)g.abase / kRows;       // the pair's first key
                    for (int key = g.k0; key < g.k1; key++) cover[base + key]++;
                    if ((size_t)g.slot >= slot_used.size() || slot_used[g.slot]++)
                        o[k == 0 ? 5 : 2]++;
                    pair_seg_runs[(size_t)g.s * nkv + g.kvh].push_back((int)run);
                }
                x = xn;
            }
            if (k == 0) {
                const int wg = run_groups(m, n, (int)nkv, (int)run, Tk, (int)total);
                out[2] += wg;
                out[3] += sg;
                if (wg != sg) out[1]++;
            }
        }
        int64_t bad_keys = 0, bad_pairs = 0;
        for (size_t s = 0; s < B; s++)
            for (size_t h = 0; h < nkv; h++) {
                const int cap = ccap[s + 1] - ccap[s], ctx = pos0[s] + cu[s + 1] - cu[s];
                const size_t base = nkv * (size_t)ccap[s] + h * cap;
                for (int key = 0; key < cap; key++)
                    if (cover[base + key] != (key < ctx ? 1 : 0)) bad_keys++;
                int w0, w1;
                pair_runs(m, (int)nkv, (int)s, (int)h, Tk, &w0, &w1);
                const auto &r = pair_seg_runs[s * nkv + h];
                bool ok = (int)r.size() == w1 - w0 + 1;
                for (size_t i = 0; ok && i < r.size(); i++) ok = r[i] == w0 + (int)i;
                if (!ok) bad_pairs++;
            }
        if (k == 0) {
            out[4] = bad_keys;
            out[6] = bad_pairs;
        } else {
            out[9] = bad_keys;
            out[11] = bad_pairs;
        }
    }
    return kOk;
}

static int cache_xfer(bool pack, const uint16_t *kc_ref, const uint16_t *vc_ref, uint16_t *ko,
                      uint16_t *vo, size_t ntok, size_t nkv, size_t d, const KvRef &kv, int h) {
    if (d != (size_t)D) return set_error(kErrUnsupported, "cache pack supports d=256");
    if (ntok > (size_t)kv.bstride * KVB) return set_error(kErrArgument, "ntok exceeds the cache");
    if (ntok == 0) return kOk;
    if (pack) {
        k_cache_pack<<<cdiv(ntok * nkv * D, 256), 256, 0, stream()>>>(kc_ref, vc_ref, ntok,
                                                                       (int)nkv, kv, h);
        APUS_LAUNCHED("k_cache_pack");
    } else {
        k_cache_unpack<<<cdiv(ntok * nkv * D, 256), 256, 0, stream()>>>(kv, h, ntok, (int)nkv,
                                                                         ko, vo);
        APUS_LAUNCHED("k_cache_unpack");
    }
    return kOk;
}

int apus_hip_attn_cache_pack(const uint16_t *kc_ref, const uint16_t *vc_ref, size_t ntok,
                             size_t nkv, size_t d, uint16_t *kcache, uint16_t *vcache,
                             size_t max_seq) {
    APUS_READY();
    if (max_seq % KVB) return set_error(kErrArgument, "max_seq must be a multiple of %d", KVB);
    return cache_xfer(true, kc_ref, vc_ref, nullptr, nullptr, ntok, nkv, d,
                      kv_flat(kcache, vcache, max_seq), 0);
}

int apus_hip_attn_cache_unpack(const uint16_t *kcache, const uint16_t *vcache, size_t ntok,
                               size_t nkv, size_t d, size_t max_seq, uint16_t *kc_ref,
                               uint16_t *vc_ref) {
    APUS_READY();
    if (max_seq % KVB) return set_error(kErrArgument, "max_seq must be a multiple of %d", KVB);
    return cache_xfer(false, nullptr, nullptr, kc_ref, vc_ref, ntok, nkv, d,
                      kv_flat(const_cast<uint16_t *>(kcache), const_cast<uint16_t *>(vcache),
                              max_seq), 0);
}

int apus_hip_attn_cache_pack_paged(const uint16_t *kc_ref, const uint16_t *vc_ref, size_t ntok,
                                   size_t nkv, size_t d, const ApusHipKvCache *kv, int32_t row) {
    APUS_READY();
    KvRef r;
    const int32_t cu1[2] = {0, (int32_t)std::min<size_t>(ntok, 0x7fffffff)}, p0[1] = {0};
    if (int e = kv_paged_ref(kv, 1, &row, cu1, p0, &r)) return e;
    return cache_xfer(true, kc_ref, vc_ref, nullptr, nullptr, ntok, nkv, d, r, row);
}

int apus_hip_attn_cache_unpack_paged(const ApusHipKvCache *kv, int32_t row, size_t ntok,
                                     size_t nkv, size_t d, uint16_t *kc_ref, uint16_t *vc_ref) {
    APUS_READY();
    KvRef r;
    const int32_t cu1[2] = {0, (int32_t)std::min<size_t>(ntok, 0x7fffffff)}, p0[1] = {0};
    if (int e = kv_paged_ref(kv, 1, &row, cu1, p0, &r)) return e;
    return cache_xfer(false, nullptr, nullptr, kc_ref, vc_ref, ntok, nkv, d, r, row);
}

}  // extern "C"
