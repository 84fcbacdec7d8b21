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
//                against the reference. The weight row is read 16 bytes
//                at a time, 16 to 32 pieces ahead of the add chain; the x row
//                is staged in LDS once per wavefront.
//   k_gemm_mfma  the 16x16x32 bf16 MFMA with fp32 accumulation for
//                decode batches (up to kMfmaRows rows): one workgroup per
//                (64 outputs, 64 rows), its 4 wavefronts splitting K, so
//                each weight piece is loaded once per row tile. Larger
//                batches (prefill) go to rocBLAS's bf16 GEMM (fp32
//                compute), a plain library GEMM. Both sum in their own order:
//                the tolerance class of the attention kernels (|c - r| <=
//                2e-3 (|r| + esc), esc = sum_k |w x|).
// Host-pointer drop-ins keep device copies of the weights keyed by their
// host address, as the reference's Metal backend keys weights by stable
// pointers (c/backend_metal.h:42-48).
#include <stdint.h>
#include <string.h>

#include <unordered_map>

#include <rocblas/rocblas.h>

#include "../../include/apus_hip.h"
#include "apus_dev.h"
#include "apus_host.h"

using namespace apus;

namespace {

typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One output per lane: outputs blockIdx.x*64 + lane of row blockIdx.y.
// VEC: K is a multiple of 8 and the rows are 16-byte aligned.
template <bool VEC>
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
        for (int i = threadIdx.x; i < n8; i += 64)
            xs_lds[i] = reinterpret_cast<const u16x8 *>(xr)[i];
        __syncthreads();
        const u16x8 *w8 = reinterpret_cast<const u16x8 *>(wr);
        const u16x8 *x8 = xs_lds;
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
                const u16x8 xv = x8[p + i];
#pragma unroll
                for (int j = 0; j < 8; j++) acc = acc + bf2f(qa[i][j]) * bf2f(xv[j]);
            }
#pragma unroll
            for (int i = 0; i < R; i++) qa[i] = w8[min(p + 2 * R + i, n8 - 1)];
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < R; i++) {
                const u16x8 xv = x8[p + R + i];
#pragma unroll
                for (int j = 0; j < 8; j++) acc = acc + bf2f(qb[i][j]) * bf2f(xv[j]);
            }
        }
        for (int i = 0; p + i < n8; i++) {
            const u16x8 wv = w8[p + i], xv = x8[p + i];
#pragma unroll
            for (int j = 0; j < 8; j++) acc = acc + bf2f(wv[j]) * bf2f(xv[j]);
        }
    } else {
        for (int k = 0; k < K; k++) acc = acc + bf2f(wr[k]) * bf2f(xr[k]);
    }
    if (o < O) y[(size_t)m * O + o] = f2bf(acc);
}

// One workgroup per (64 outputs, up to 64 rows); its 4 wavefronts split K
// (32-wide k step st goes to wavefront st % 4), each with all 4 x 4
// 16x16 output blocks, the next step's operands in flight, and add their
// partial sums through LDS. Operands come through buffer loads whose rows
// past M or O sit out of the buffer's range and read as zero, so every
// load and MFMA is unconditional (no branch joins for the compiler to
// drain the memory counter at). Needs K % 32 == 0.
constexpr int MT = 64, OT = 64, MB = MT / 16, OB = OT / 16, NWV = 4;
constexpr int kOutOfRange = 0x40000000;   // a byte offset past every operand

__global__ __launch_bounds__(256) void k_gemm_mfma(const uint16_t *__restrict__ w,
                                                   const uint16_t *__restrict__ x,
                                                   uint16_t *__restrict__ y, int M, int O, int K) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g8 = (lane >> 4) * 8, kq = (lane >> 4) * 4;
    const int o0 = blockIdx.x * OT, m0 = blockIdx.y * MT;
    const auto wr = buf_rsrc(w, (uint32_t)((size_t)O * K * 2));
    const auto xr = buf_rsrc(x, (uint32_t)((size_t)M * K * 2));
    int woff[OB], xoff[MB];
#pragma unroll
    for (int c = 0; c < OB; c++) {
        const int o = o0 + c * 16 + r16;
        woff[c] = o < O ? (o * K + g8) * 2 : kOutOfRange;
    }
#pragma unroll
    for (int b = 0; b < MB; b++) {
        const int m = m0 + b * 16 + r16;
        xoff[b] = m < M ? (m * K + g8) * 2 : kOutOfRange;
    }
    f32x4 acc[MB][OB];
#pragma unroll
    for (int b = 0; b < MB; b++)
#pragma unroll
        for (int c = 0; c < OB; c++) acc[b][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nsteps = K / 32;
    bf16x8 bw[OB], ax[MB];
    // step st's operands; steps past K are clamped to the last (loaded,
    // not used)
    auto load = [&](int st) {
        const int kb = min(st, nsteps - 1) * 64;
#pragma unroll
        for (int c = 0; c < OB; c++)
            bw[c] = __builtin_bit_cast(bf16x8, llvm_raw_ptr_buffer_load_v4f32(wr, woff[c] + kb, 0, 0));
#pragma unroll
        for (int b = 0; b < MB; b++)
            ax[b] = __builtin_bit_cast(bf16x8, llvm_raw_ptr_buffer_load_v4f32(xr, xoff[b] + kb, 0, 0));
    };
    load(wave);
    for (int st = wave; st < nsteps; st += NWV) {
        bf16x8 bc[OB], ac[MB];
#pragma unroll
        for (int c = 0; c < OB; c++) bc[c] = bw[c];
#pragma unroll
        for (int b = 0; b < MB; b++) ac[b] = ax[b];
        load(st + NWV);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < MB; b++)
#pragma unroll
            for (int c = 0; c < OB; c++)
                acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac[b], bc[c], acc[b][c], 0, 0, 0);
    }
    // the partial sums of the 4 wavefronts through LDS, added in wavefront
    // order; wavefront v then finishes row block v
    __shared__ f32x4 part[NWV][MB][OB][64];
#pragma unroll
    for (int b = 0; b < MB; b++)
#pragma unroll
        for (int c = 0; c < OB; c++) part[wave][b][c][lane] = acc[b][c];
    __syncthreads();
    const int b = wave;
#pragma unroll
    for (int c = 0; c < OB; c++) {
        f32x4 s = part[0][b][c][lane];
#pragma unroll
        for (int v = 1; v < NWV; v++) s += part[v][b][c][lane];
        // D[row kq + i][column r16]: row m0 + 16b + kq + i, output o0 + 16c + r16
        const int o = o0 + c * 16 + r16;
        if (o < O) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + b * 16 + kq + i;
                if (m < M) y[(size_t)m * O + o] = f2bf(s[i]);
            }
        }
    }
}

int check_dims(size_t M, size_t O, size_t K) {
    if (M > 0x7fffffffu || O > 0x7fffffffu || K > 0x7fffffffu)
        return set_error(kErrUnsupported, "gemm dims past 2^31");
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

// rocBLAS for prefill-sized row counts: y (column-major O x M, ldc O) =
// w^T (w is column-major K x O) . x (column-major K x M), bf16 in and
// out, fp32 compute. One handle per device, on the library's stream.
constexpr size_t kMfmaRows = 256;
std::unordered_map<int, rocblas_handle> g_blas;

int blas_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y, size_t M, size_t O, size_t K) {
    const int dev = current_device();
    rocblas_handle &h = g_blas[dev];
    if (!h && rocblas_create_handle(&h) != rocblas_status_success) {
        h = nullptr;
        return set_error(kErrHip, "rocblas_create_handle failed");
    }
    if (rocblas_set_stream(h, stream()) != rocblas_status_success)
        return set_error(kErrHip, "rocblas_set_stream failed");
    const float one = 1.0f, zero = 0.0f;
    const rocblas_status st = rocblas_gemm_ex(
        h, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)O, (rocblas_int)M,
        (rocblas_int)K, &one, w, rocblas_datatype_bf16_r, (rocblas_int)K, x,
        rocblas_datatype_bf16_r, (rocblas_int)K, &zero, y, rocblas_datatype_bf16_r,
        (rocblas_int)O, y, rocblas_datatype_bf16_r, (rocblas_int)O, rocblas_datatype_f32_r,
        rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success)
        return set_error(kErrHip, "rocblas_gemm_ex failed (%d)", (int)st);
    return kOk;
}

}  // namespace

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
    if (int r = check_dims(M, O, K)) return r;
    if (M == 0 || O == 0) return kOk;
    // the hand kernel: decode-sized M, K % 32 == 0, 16-byte aligned rows,
    // operands under 1 GiB; everything else (prefill) through rocBLAS
    if (M > kMfmaRows || K % 32 != 0 || ((uintptr_t)w | (uintptr_t)x) % 16 != 0 ||
        O * K * 2 >= (size_t)kOutOfRange || M * K * 2 >= (size_t)kOutOfRange) {
        int r = kOk;
        APUS_TIMED("rocblas_gemm_bf16", r = blas_gemm(w, x, y, M, O, K));
        return r;
    }
    const dim3 grid(cdiv(O, OT), cdiv(M, MT));
    APUS_TIMED("k_gemm_mfma",
               k_gemm_mfma<<<grid, 256, 0, stream()>>>(w, x, y, (int)M, (int)O, (int)K));
    return launch_check("k_gemm_mfma");
}

}  // extern "C"
