// proj.hip -- the bf16 projections on either side of the attention path
// (c/bf16.h:178-231: y[m][o] = rnd(sum_k w[o][k] x[m][k]), w [O][K],
// x [M][K], y [M][O], bf16 codes in and out, fp32 accumulation), the
// reference's apus_bf16_gemv_hot / apus_bf16_gemm_hot and the
// ApusBackendHooks bf16_gemv / bf16_gemm slots (c/backend_metal.h:68-75).
//
// Two kernels:
//   k_gemm_seq   one lane per output, the k sum in the reference's order
//                (ascending, one rounding per multiply and per add: the
//                scalar anchor c/bf16.h:285-293, which the reference's
//                threaded and Metal paths reproduce bitwise). Bitwise
//                against the reference (products below fp32's normal range
//                aside: see k_gemm_seq). The weight row is read 16 bytes
//                at a time, 16 to 32 pieces ahead of the add chain; the x row
//                is staged in LDS once per wavefront.
//   k_gemm_tile  the 32x32x16 bf16 MFMA with fp32 accumulation, for every
//                row count: a workgroup computes a (BO outputs x BM rows)
//                tile, its operands copied global -> LDS by buffer_load ...
//                lds in stages of 32 k through a 4-deep ring; each
//                wavefront reads the next k16 step's fragments while the
//                current step's MFMAs issue. Tile shapes are chosen per call
//                shape (decode batches: small tiles, many workgroups;
//                prefill: 256 x 256). It sums in its own order: the
//                tolerance class of the attention kernels (|c - r| <=
//                2e-3 (|r| + esc), esc = sum_k |w x|).
// Host-pointer drop-ins keep device copies of the weights keyed by their
// host address, as the reference's Metal backend keys weights by stable
// pointers (c/backend_metal.h:42-48).
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <type_traits>
#include <unordered_map>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"
#include "proj.h"

using namespace apus;

namespace {

typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One output per lane: outputs blockIdx.x*64 + lane of row blockIdx.y.
// VEC: K is a multiple of 8 and the rows are 16-byte aligned. XF: the x
// row is staged in LDS as fp32 (widened once per wavefront instead of once
// per output; K up to 16384), so a k costs the weight's widening and one
// fused multiply-add. The product of two bf16 values (8-bit significands)
// is exact in fp32 whenever it lies in fp32's normal range, so the fused
// form rounds exactly where the reference's multiply-then-add does: once,
// at the add. Only a product below 2^-126 in magnitude (a subnormal,
// which the reference rounds before adding) can differ, and then only if
// the running sum is itself that small. (25.4 -> 21.0 us for 12352 x 2048.)
template <bool VEC, bool XF = false>
__global__ __launch_bounds__(64) void k_gemm_seq(const uint16_t *__restrict__ w,
                                                 const uint16_t *__restrict__ x,
                                                 uint16_t *__restrict__ y, int O, int K) {
    const int o = blockIdx.x * 64 + threadIdx.x;
    const int m = blockIdx.y;
    const uint16_t *xr = x + (size_t)m * K;
    const uint16_t *wr = w + (size_t)min(o, O - 1) * K;
    float acc = 0.0f;
    if (VEC) {
        // the x row in LDS (dynamic, K codes): its reads wait on the LDS
        // counter, so the vector-memory waits count weight loads only
        extern __shared__ __attribute__((aligned(16))) u16x8 xs_lds[];
        const int n8 = K / 8;
        if (XF) {
            float4 *xf = reinterpret_cast<float4 *>(xs_lds);
            for (int i = threadIdx.x; i < n8; i += 64) {
                const u16x8 v = reinterpret_cast<const u16x8 *>(xr)[i];
                xf[2 * i] = make_float4(bf2f(v[0]), bf2f(v[1]), bf2f(v[2]), bf2f(v[3]));
                xf[2 * i + 1] = make_float4(bf2f(v[4]), bf2f(v[5]), bf2f(v[6]), bf2f(v[7]));
            }
        } else {
            for (int i = threadIdx.x; i < n8; i += 64)
                xs_lds[i] = reinterpret_cast<const u16x8 *>(xr)[i];
        }
        __syncthreads();
        // k values 8i .. 8i+7 of x as floats
        auto xk = [&](int i, float (&f)[8]) {
            if (XF) {
                const float4 *xf = reinterpret_cast<const float4 *>(xs_lds);
                const float4 a = xf[2 * i], b = xf[2 * i + 1];
                f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
                f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
            } else {
                const u16x8 v = xs_lds[i];
#pragma unroll
                for (int j = 0; j < 8; j++) f[j] = bf2f(v[j]);
            }
        };
        const u16x8 *w8 = reinterpret_cast<const u16x8 *>(wr);
        constexpr int R = 16;          // pieces per round; two register sets
        // rounds alternate between the sets: while one set is summed the
        // next round's loads are in flight into the other. Prefetch indices
        // are clamped to the row (no branch around a load), so each wait
        // counts only the loads issued after the set it needs.
        u16x8 qa[R], qb[R];
#pragma unroll
        for (int i = 0; i < R; i++) qa[i] = w8[min(i, n8 - 1)];
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        int p = 0;
        for (; p + 2 * R <= n8; p += 2 * R) {
#pragma unroll
            for (int i = 0; i < R; i++) qb[i] = w8[min(p + R + i, n8 - 1)];
            // keep the prefetches here (the compiler would sink each load
            // to its first use and wait on it there)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < R; i++) {
                float xv[8];
                xk(p + i, xv);
#pragma unroll
                for (int j = 0; j < 8; j++) acc = fmaf(bf2f(qa[i][j]), xv[j], acc);
            }
#pragma unroll
            for (int i = 0; i < R; i++) qa[i] = w8[min(p + 2 * R + i, n8 - 1)];
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < R; i++) {
                float xv[8];
                xk(p + R + i, xv);
#pragma unroll
                for (int j = 0; j < 8; j++) acc = fmaf(bf2f(qb[i][j]), xv[j], acc);
            }
        }
        for (int i = 0; p + i < n8; i++) {
            const u16x8 wv = w8[p + i];
            float xv[8];
            xk(p + i, xv);
#pragma unroll
            for (int j = 0; j < 8; j++) acc = fmaf(bf2f(wv[j]), xv[j], acc);
        }
    } else {
        for (int k = 0; k < K; k++) acc = acc + bf2f(wr[k]) * bf2f(xr[k]);
    }
    if (o < O) y[(size_t)m * O + o] = f2bf(acc);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
int check_dims(size_t M, size_t O, size_t K) {
    if (M > 0x7fffffffu || O > 0x7fffffffu || K > 0x7fffffffu)
        return set_error(kErrUnsupported, "gemm dims past 2^31");
    return kOk;
}

// byte offset of 16-byte chunk c (0..3) of row r in a stage's 64-byte rows:
// chunks are XOR-swizzled by (r / 4) % 4, so the 32 rows one MFMA operand
// read touches spread over the LDS banks
__device__ __forceinline__ int tile_slot(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }

constexpr int kTileStages = 4;            // LDS ring depth (stages of 32 k)

// Workgroup -> (output tile, row tile). Workgroups are dealt round-robin
// to the 8 XCDs (id % 8), each XCD running its ids in order. The tiles are
// grouped into blocks of GO output tiles x GM row tiles (GO GM = 32, GM =
// 8 for 8 or more row tiles); block g goes to XCD g % 8 as its (g / 8)-th group of
// 32 ids. The 32 workgroups an XCD runs together then share GO weight
// tiles and GM x tiles, which stay in that XCD's L2 while they walk K in
// step (prefill: 12 distinct 256-row operand tiles per XCD instead of 18
// with whole row-tile columns per XCD).
__host__ __device__ inline void tile_groups(int nbo, int nbm, int &go, int &gm, int &ngo,
                                            int &ngm) {
    gm = nbm < 8 ? nbm : 8;
    go = 32 / gm;
    ngo = (nbo + go - 1) / go;
    ngm = (nbm + gm - 1) / gm;
}
// Fewer than 8 row tiles (decode batches): output tile ob's row tiles all
// go to XCD ob % 8 instead (ids ((ob / 8) nbm + mb) 8 + ob % 8), which
// measured faster there (w_out at 325 rows: 27 vs 29 us).
__host__ __device__ inline int tile_grid(int nbo, int nbm) {
    if (nbm < 8) return (nbo + 7) / 8 * 8 * nbm;
    int go, gm, ngo, ngm;
    tile_groups(nbo, nbm, go, gm, ngo, ngm);
    return (ngo * ngm + 7) / 8 * 8 * 32;
}
__host__ __device__ inline void tile_of(int id, int nbo, int nbm, int &ob, int &mb) {
    if (nbm < 8) {
        const int band = id / (8 * nbm), rem = id % (8 * nbm);
        mb = rem / 8;
        ob = band * 8 + rem % 8;
        return;
    }
    int go, gm, ngo, ngm;
    tile_groups(nbo, nbm, go, gm, ngo, ngm);
    const int x = id % 8, slot = id / 8;
    const int g = (slot / 32) * 8 + x, p = slot % 32;
    const int gi = g / ngm, gj = g % ngm;          // group (output, row)
    ob = gi * go + p % go;
    mb = gj * gm + p / go;
    if (gi >= ngo) ob = nbo;                       // past the last group
}

__device__ __forceinline__ int seg_of(const GemmSegs &g, int o) {
    int i = 0;
#pragma unroll
    for (int j = 1; j < kMaxSegs; j++)
        if (j < g.n && o >= g.row0[j]) i = j;
    return i;
}

// bf16 stores of a wavefront's TO x TMM accumulator tiles (D[o][m]): tile
// (t, u) holds outputs ob0 + 32 t .. and rows mb0 + 32 u + lane % 32; lane
// -> o = 8 (i / 4) + 4 (lane / 32) + i % 4 of register i. Each 32-output
// tile lies in one segment.
template <int TO, int TMM>
__device__ __forceinline__ void store_tiles(const GemmSegs &sg, const f32x16 (&acc)[TO][TMM],
                                            int ob0, int mb0, int O, int M, int lane) {
#pragma unroll
    for (int t = 0; t < TO; t++) {
        const int ot = ob0 + t * 32;
        if (ot >= O) continue;
        const int si = seg_of(sg, ot);
        uint16_t *yb = sg.y[si] - sg.row0[si];
        const int ld = sg.ldy[si];
        const bool vec = ((ld | sg.row0[si]) & 3) == 0 && ((uintptr_t)sg.y[si] & 7) == 0;
#pragma unroll
        for (int u = 0; u < TMM; u++) {
            const int m = mb0 + u * 32 + (lane & 31);
            if (m >= M) continue;
            const f32x16 &a = acc[t][u];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int o = ot + 8 * q + 4 * (lane >> 5);
                if (vec) {
                    if (o < O)
                        *reinterpret_cast<uint2 *>(yb + (size_t)m * ld + o) =
                            make_uint2(pk2(a[4 * q], a[4 * q + 1]), pk2(a[4 * q + 2], a[4 * q + 3]));
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (o + i < O) yb[(size_t)m * ld + o + i] = f2bf(a[4 * q + i]);
                }
            }
        }
    }
}

// y[m][o] = rnd(sum_k w[o][k] x[m][k]) on the 32x32x16 bf16 MFMA. The
// workgroup has WO x WM wavefronts; wavefront (wo, wm) = (wave / WM,
// wave % WM) -- so the WM wavefronts sharing output columns sit on
// different SIMDs -- computes TO x TMM MFMA tiles: outputs
// o0 + 32 (TO wo + t) .., rows m0 + 32 (TMM wm + u) ... The product is
// formed transposed (D[o][m]: A = w rows, B = x rows) so that a lane holds
// 4 consecutive outputs of one row and stores them as 8 bytes.
// Stages: each stage's w rows (BO x 64 B) and x rows (BM x 64 B) are copied
// global -> LDS in 1 KiB pieces (16 rows each; lane L fills byte 16 L of
// the piece: row L / 4, chunk (L % 4) ^ ((row / 4) % 4)); rows past O or M
// lie past their buffer's end and read zero. Stage s is issued ST - 1
// stages ahead, unconditionally (past the last stage the copy re-reads
// it), so every wait is a constant count; one barrier per stage. MFMAs of
// tiles wholly past O or M are skipped (wave-uniform).
// Workgroup order: the row tiles of an output tile are dealt to one XCD
// (block ids congruent mod 8), so they share its w rows in that XCD's L2.
// Split K (part != nullptr): block b works on k stages of split b / nb
// (nb: the blocks of one split) and stores its fp32 partial tile to
// part[split][m][o]; k_gemm_reduce then sums the splits in order.
template <int WO, int WM, int TO, int TMM, int ST>
__global__ __launch_bounds__(64 * WO * WM) void k_gemm_tile(GemmSegs sg,
                                                       const uint16_t *__restrict__ x, int M,
                                                       int K, float *__restrict__ part, int nsplit) {
    const int O = sg.row0[sg.n];
    constexpr int NW = WO * WM, BO = 32 * TO * WO, BM = 32 * TMM * WM;
    constexpr int PB = BO * 64, SB = (BO + BM) * 64;
    constexpr int NPIECE = (BO + BM) / 16;
    static_assert(NPIECE % NW == 0, "copy pieces must split evenly over the wavefronts");
    constexpr int PPW = NPIECE / NW;
    __shared__ __attribute__((aligned(16))) char sm[ST * SB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wo = wave / WM, wm = wave % WM;
    const int nbo = (O + BO - 1) / BO, nbm = (M + BM - 1) / BM;
    const int nb = tile_grid(nbo, nbm);
    const int id = blockIdx.x % nb, ks = blockIdx.x / nb;
    int ob, mb;
    tile_of(id, nbo, nbm, ob, mb);
    if (ob >= nbo || mb >= nbm) return;         // (the grid rounds up to whole groups)
    const int o0 = ob * BO, m0 = mb * BM;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)sm);
    // this wave's copy pieces: the buffer of each (x, or its weight
    // segment; wave-uniform) and each lane's byte offset in it
    i32x4 rs[PPW];
    int voff[PPW];
    uint32_t loff[PPW];
#pragma unroll
    for (int i = 0; i < PPW; i++) {
        const int p = wave * PPW + i;
        const bool pw = p < BO / 16;
        const int pr = pw ? p : p - BO / 16;
        const int r = pr * 16 + lane / 4;
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        if (pw) {
            const int si = __builtin_amdgcn_readfirstlane(seg_of(sg, o0 + pr * 16));
            const int rows = sg.row0[si + 1] - sg.row0[si], gr = o0 + r - sg.row0[si];
            rs[i] = dma_rsrc(sg.w[si], (uint32_t)((size_t)rows * K * 2));
            voff[i] = gr < rows ? (gr * K + c * 8) * 2 : 0x7fffffff;
        } else {
            rs[i] = dma_rsrc(x, (uint32_t)((size_t)M * K * 2));
            voff[i] = m0 + r < M ? ((m0 + r) * K + c * 8) * 2 : 0x7fffffff;
        }
        loff[i] = pw ? pr * 1024 : PB + pr * 1024;
    }
    // this block's k stages: [kt0, kt0 + nk)
    const int nkall = K / 32;
    const int kt0 = ks * nkall / nsplit, nk = (ks + 1) * nkall / nsplit - kt0;
    auto issue = [&](int st) {
        const int kb = (kt0 + min(st, nk - 1)) * 64;
        const uint32_t base = lds0 + (st % ST) * SB;
#pragma unroll
        for (int i = 0; i < PPW; i++) dma16(rs[i], voff[i], kb, base + loff[i]);
    };
    f32x16 acc[TO][TMM];
#pragma unroll
    for (int t = 0; t < TO; t++)
#pragma unroll
        for (int u = 0; u < TMM; u++) acc[t][u] = f32x16{};
    auto rd = [&](int kt, int s, bf16x8 (&af)[TO], bf16x8 (&bf)[TMM]) {
        const char *Wl = sm + (kt % ST) * SB;
        const char *Xl = Wl + PB;
        const int c = s * 2 + (lane >> 5);
#pragma unroll
        for (int t = 0; t < TO; t++)
            af[t] = *reinterpret_cast<const bf16x8 *>(Wl + tile_slot(wo * TO * 32 + t * 32 + (lane & 31), c));
#pragma unroll
        for (int u = 0; u < TMM; u++)
            bf[u] = *reinterpret_cast<const bf16x8 *>(Xl + tile_slot(wm * TMM * 32 + u * 32 + (lane & 31), c));
    };
    const int tv = min(TO, max(0, (O - (o0 + wo * TO * 32) + 31) / 32));
    const int uv = min(TMM, max(0, (M - (m0 + wm * TMM * 32) + 31) / 32));
    // MFMAs of tiles past O or M are skipped; a wavefront whose tiles are
    // all inside runs the loop without the per-MFMA tests (as uniform
    // branches they split the loop into a block per MFMA and cost ~10 %)
    auto loop = [&](auto edge) {
        auto mma = [&](const bf16x8 (&af)[TO], const bf16x8 (&bf)[TMM]) {
#pragma unroll
            for (int t = 0; t < TO; t++)
#pragma unroll
                for (int u = 0; u < TMM; u++)
                    if (!decltype(edge)::value || (t < tv && u < uv))
                        acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[t], bf[u], acc[t][u], 0, 0, 0);
        };
#pragma unroll
        for (int s = 0; s < ST - 1; s++) issue(s);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PPW * (ST - 2)) : "memory");
        __syncthreads();
        issue(ST - 1);
        bf16x8 fa0[TO], fb0[TMM], fa1[TO], fb1[TMM];
        rd(0, 0, fa0, fb0);
        // the scheduling barriers keep each phase's LDS reads ahead of the
        // MFMAs that do not need them (left free, the scheduler sank them
        // to their first use)
        for (int kt = 0; kt < nk; kt++) {
            rd(kt, 1, fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
            mma(fa0, fb0);
            __builtin_amdgcn_sched_barrier(0);
            // stage kt+1 landed (this wave's copies), then visible to all;
            // every wave is past its reads of stage kt, whose slot the next
            // issue fills
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PPW * (ST - 2)) : "memory");
            __syncthreads();
            issue(kt + ST);
            rd(kt + 1, 0, fa0, fb0);
            __builtin_amdgcn_sched_barrier(0);
            mma(fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (tv == TO && uv == TMM)
        loop(std::false_type{});
    else
        loop(std::true_type{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // D[o][m]: lane -> m = lane % 32, o = 8 (i / 4) + 4 (lane / 32) + i % 4;
    // each 32-output tile lies in one segment
    if (part) {                                 // fp32 partials, [split][m][O]
        float *pb = part + (size_t)ks * M * O;
#pragma unroll
        for (int t = 0; t < TO; t++) {
            const int ot = o0 + wo * TO * 32 + t * 32;
            if (ot >= O) continue;
#pragma unroll
            for (int u = 0; u < TMM; u++) {
                const int m = m0 + wm * TMM * 32 + u * 32 + (lane & 31);
                if (m >= M) continue;
                const f32x16 &a = acc[t][u];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int o = ot + 8 * q + 4 * (lane >> 5);
                    if (o < O)
                        *reinterpret_cast<float4 *>(pb + (size_t)m * O + o) =
                            make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
                }
            }
        }
        return;
    }
    store_tiles<TO, TMM>(sg, acc, o0 + wo * TO * 32, m0 + wm * TMM * 32, O, M, lane);
}

// Decode-sized row counts: one BO x BM tile per workgroup (BO = 32 TO
// outputs, BM = 32 TMM rows), its NW wavefronts each over a contiguous
// 1/NW share of the k stages. Each wavefront copies its own stages into a
// private R-deep LDS ring (the same 1 KiB pieces and swizzle as
// k_gemm_tile) and waits only for its own copies: no barrier in the k loop,
// where the shared-ring kernel's per-stage barrier left a decode tile's
// two wavefronts waiting on each other for every 32 k. The NW partial
// tiles are then summed through LDS in a fixed tree (NW = 4: (p0 + p2) +
// (p1 + p3), p_w the partial of share w), and wavefront 0 stores the
// tile. An element's sum order depends on K and NW only.
// y = rnd(sum over the splits of part, in split order), scattered to the
// segments; a thread owns 4 consecutive outputs of one row (O % 4 == 0)
__global__ __launch_bounds__(256) void k_gemm_reduce(GemmSegs sg, const float *__restrict__ part,
                                                     int M, int nsplit) {
    const int O = sg.row0[sg.n], O4 = O / 4;
    const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (size_t)M * O4) return;
    const int m = (int)(e / O4), o = (int)(e % O4) * 4;
    float4 sm = *reinterpret_cast<const float4 *>(part + (size_t)m * O + o);
    for (int s = 1; s < nsplit; s++) {
        const float4 v = *reinterpret_cast<const float4 *>(part + ((size_t)s * M + m) * O + o);
        sm.x += v.x; sm.y += v.y; sm.z += v.z; sm.w += v.w;
    }
    const int si = seg_of(sg, o);
    uint16_t *yr = sg.y[si] + (size_t)m * sg.ldy[si] + (o - sg.row0[si]);
    yr[0] = f2bf(sm.x);
    yr[1] = f2bf(sm.y);
    yr[2] = f2bf(sm.z);
    yr[3] = f2bf(sm.w);
}

template <int WO, int WM, int TO, int TMM, int ST = kTileStages>
int launch_tile(const GemmSegs &sg, const uint16_t *x, int M, int K, const char *name,
                int nsplit) {
    constexpr int BO = 32 * TO * WO, BM = 32 * TMM * WM;
    const int O = sg.row0[sg.n];
    const int nbo = (O + BO - 1) / BO, nbm = (M + BM - 1) / BM;
    const unsigned grid = (unsigned)tile_grid(nbo, nbm);
    float *part = nullptr;
    if (nsplit > 1) {
        part = (float *)scratch(kScratchWork3, (size_t)nsplit * M * O * 4);
        if (!part) return kErrHip;
    }
    APUS_TIMED(name, k_gemm_tile<WO, WM, TO, TMM, ST><<<grid * nsplit, 64 * WO * WM, 0, stream()>>>(
                         sg, x, M, K, part, nsplit));
    if (int r = launch_check(name)) return r;
    if (nsplit > 1) {
        APUS_TIMED("k_gemm_reduce", k_gemm_reduce<<<cdiv((size_t)M * O / 4, 256), 256, 0,
                                                    stream()>>>(sg, part, M, nsplit));
        return launch_check("k_gemm_reduce");
    }
    return kOk;
}

}  // namespace

namespace apus {

// Tile shape per call shape (measured on MI355X for the model's projection
// shapes, K = 2048 / 4096): decode batches want many small workgroups
// (the weights stream once; x is re-read from L2), prefill the 256 x 256
// tile (operand traffic M O K (1/BO + 1/BM) through L2).
int gemm_tile_split(const GemmSegs &sg, const uint16_t *x, size_t M, size_t K, const char *nm,
                    int cfg, int nsplit) {
    const int m = (int)M, k = (int)K;
    const size_t O = (size_t)sg.row0[sg.n];
    if (nsplit > 1 && O % 4) nsplit = 1;
    nsplit = std::max(1, std::min(nsplit, (int)(K / 32)));
    if (cfg < 0)
        cfg = M > 512 ? 3 : (M > 64 && O > 10000) ? 2 : (M > 64 && O > 4096) ? 1 : 0;
    // Within a configuration the row tile follows M (measured on the
    // model's shapes: the slowest workgroup sets the time, so a row tile
    // that is mostly past M wastes its CU): M <= 128 with long outputs
    // runs 128 x 128 tiles on 8 wavefronts (39 -> 31 us at M = 128), M <=
    // 384 128 x 192 (the in-projection at M = 325: 42 -> 39 us), and
    // decode rows past 64 with short outputs 128 x 64 (the out-projection
    // at M = 325: 21 -> 19 us).
    switch (cfg) {
    case 3: return launch_tile<2, 4, 4, 2>(sg, x, m, k, nm, nsplit);      // 256 x 256
    case 2:
        if (m <= 128) return launch_tile<2, 4, 2, 1>(sg, x, m, k, nm, nsplit);   // 128 x 128
        if (m <= 384) return launch_tile<2, 2, 2, 3>(sg, x, m, k, nm, nsplit);   // 128 x 192
        return launch_tile<2, 2, 2, 4>(sg, x, m, k, nm, nsplit);                 // 128 x 256
    case 1: return launch_tile<4, 1, 1, 4>(sg, x, m, k, nm, nsplit);      // 128 x 128
    default:
        if (m > 64) return launch_tile<2, 2, 2, 1>(sg, x, m, k, nm, nsplit);     // 128 x 64
        return launch_tile<2, 1, 1, 2>(sg, x, m, k, nm, nsplit);                 // 64 x 64
    }
}

// Decode-sized row counts with a long K (the output projections, K =
// 4096) split K in two: twice the workgroups for the few output tiles
// (w_out at 325 rows: 27 -> 21 us). The split depends on M and K only, so
// a product's summation order is the same whichever launch (segmented or
// not) computes it.
int gemm_tile(const GemmSegs &sg, const uint16_t *x, size_t M, size_t K, const char *nm) {
    return gemm_tile_split(sg, x, M, K, nm, -1, (M <= 512 && K >= 4096) ? 2 : 1);
}

// checks shared by the MFMA entry points: K a multiple of 32 (stages),
// 16-byte aligned operands (16-byte copies), byte offsets under 2 GiB
int gemm_tile_check(const uint16_t *x, size_t M, size_t O, size_t K) {
    if (int r = check_dims(M, O, K)) return r;
    if (!x) return set_error(kErrArgument, "NULL operand");
    if (K == 0 || K % 32 != 0 || (uintptr_t)x % 16 != 0)
        return set_error(kErrUnsupported, "MFMA gemm needs K a multiple of 32 and 16-byte "
                         "aligned operands (K=%zu)", K);
    if (O * K * 2 >= 0x7fff0000u || M * K * 2 >= 0x7fff0000u)
        return set_error(kErrUnsupported, "MFMA gemm operands must stay under 2 GiB");
    return kOk;
}

int launch_seq(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t M, size_t O,
               size_t K) {
    if (int r = check_dims(M, O, K)) return r;
    if (M == 0 || O == 0) return kOk;
    if (M > 65535) return set_error(kErrUnsupported, "sequential gemm takes up to 65535 rows");
    const bool vec = K % 8 == 0 && ((uintptr_t)w | (uintptr_t)x) % 16 == 0;
    const dim3 grid(cdiv(O, 64), (unsigned)M);
    if (vec) {
        if (K * 2 > 64 * 1024) return set_error(kErrUnsupported, "sequential gemm takes K up to 32768");
        if (K * 4 <= 64 * 1024)
            APUS_TIMED("k_gemm_seq",
                       k_gemm_seq<true, true><<<grid, 64, K * 4, stream()>>>(w, x, y, (int)O, (int)K));
        else
            APUS_TIMED("k_gemm_seq",
                       k_gemm_seq<true><<<grid, 64, K * 2, stream()>>>(w, x, y, (int)O, (int)K));
    } else {
        APUS_TIMED("k_gemm_seq", k_gemm_seq<false><<<grid, 64, 0, stream()>>>(w, x, y, (int)O, (int)K));
    }
    return launch_check("k_gemm_seq");
}

// Device copies of host weights, keyed by host address (and size).
struct WeightCopy {
    void *dev = nullptr;
    size_t bytes = 0;
    int device = -1;
};
std::unordered_map<const void *, WeightCopy> g_weights;

const uint16_t *weight_copy(const uint16_t *w, size_t bytes) {
    WeightCopy &e = g_weights[w];
    const int dev = current_device();
    if (e.dev && (e.bytes != bytes || e.device != dev)) {
        if (e.device == dev) (void)hipFree(e.dev);
        e = WeightCopy{};
    }
    if (!e.dev) {
        if (hipMalloc(&e.dev, bytes) != hipSuccess) {
            e = WeightCopy{};
            set_error(kErrHip, "weight copy: hipMalloc of %zu bytes failed", bytes);
            return nullptr;
        }
        if (hipMemcpyAsync(e.dev, w, bytes, hipMemcpyHostToDevice, stream()) != hipSuccess) {
            set_error(kErrHip, "weight copy: upload of %zu bytes failed", bytes);
            return nullptr;
        }
        e.bytes = bytes;
        e.device = dev;
    }
    return (const uint16_t *)e.dev;
}

int host_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t M, size_t O, size_t K) {
    APUS_READY();
    if (int r = check_dims(M, O, K)) return r;
    if (M == 0 || O == 0) return kOk;
    if (!w || !x || !y) return set_error(kErrArgument, "NULL operand");
    const uint16_t *dw = weight_copy(w, O * K * 2);
    if (!dw && O * K) return kErrHip;
    APUS_STAGE(dx, uint16_t, kScratchIn, x, M * K * 2);
    uint16_t *dy = (uint16_t *)scratch(kScratchOut, M * O * 2);
    if (!dy) return kErrHip;
    if (int r = launch_seq(dw, dx, dy, M, O, K)) return r;
    return stage_out(y, dy, M * O * 2);
}

}  // namespace apus

extern "C" {

int apus_hip_bf16_gemv(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t O, size_t K) {
    return host_gemm(w, x, y, 1, O, K);
}

int apus_hip_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t M, size_t O,
                       size_t K) {
    return host_gemm(w, x, y, M, O, K);
}

int apus_hip_bf16_weights_release(void) {
    APUS_READY();
    APUS_HIP_TRY(hipStreamSynchronize(stream()));
    const int dev = current_device();
    for (auto &kv : g_weights)
        if (kv.second.dev && kv.second.device == dev) (void)hipFree(kv.second.dev);
    g_weights.clear();
    return kOk;
}

int apus_hip_bf16_gemm_dev(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t M,
                           size_t O, size_t K) {
    APUS_READY();
    return launch_seq(w, x, y, M, O, K);
}

int apus_hip_bf16_gemm_mfma_dev(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t M,
                                size_t O, size_t K) {
    APUS_READY();
    if (M == 0 || O == 0) return check_dims(M, O, K);
    if (!w || !y) return set_error(kErrArgument, "NULL operand");
    if (int r = gemm_tile_check(x, M, O, K)) return r;
    if ((uintptr_t)w % 16 != 0)
        return set_error(kErrUnsupported, "MFMA gemm needs 16-byte aligned operands");
    GemmSegs sg{};
    sg.n = 1;
    sg.row0[1] = (int)O;
    sg.w[0] = w;
    sg.y[0] = y;
    sg.ldy[0] = (int)O;
    return gemm_tile(sg, x, M, K, "k_gemm_tile");
}

}  // extern "C"
