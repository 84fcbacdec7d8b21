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
//                at a time, four pieces ahead of the add chain; the x row
//                is uniform across the wavefront (scalar loads).
//   k_gemm_mfma  the 16x16x32 bf16 MFMA with fp32 accumulation for many
//                rows (prefill, large decode batches): one workgroup per
//                (64 outputs, 64 rows); wavefront w owns outputs
//                16w..16w+15 and every row block, so each weight piece is
//                loaded once per row tile. The MFMA sums in its own order:
//                the tolerance class of the attention kernels (|c - r| <=
//                2e-3 (|r| + esc), esc = sum_k |w x|).
// Host-pointer drop-ins keep device copies of the weights keyed by their
// host address, as the reference's Metal backend keys weights by stable
// pointers (c/backend_metal.h:42-48).
#include <stdint.h>
#include <string.h>

#include <unordered_map>

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
        const u16x8 *w8 = reinterpret_cast<const u16x8 *>(wr);
        const u16x8 *x8 = reinterpret_cast<const u16x8 *>(xr);
        const int n8 = K / 8;
        constexpr int AHEAD = 4;
        u16x8 wq[AHEAD];
#pragma unroll
        for (int i = 0; i < AHEAD; i++) wq[i] = i < n8 ? w8[i] : u16x8{0, 0, 0, 0, 0, 0, 0, 0};
        for (int p = 0; p < n8; p += AHEAD) {
#pragma unroll
            for (int i = 0; i < AHEAD; i++) {
                if (p + i < n8) {
                    const u16x8 wv = wq[i];
                    if (p + i + AHEAD < n8) wq[i] = w8[p + i + AHEAD];
                    const u16x8 xv = x8[p + i];
#pragma unroll
                    for (int j = 0; j < 8; j++) acc = acc + bf2f(wv[j]) * bf2f(xv[j]);
                }
            }
        }
    } else {
        for (int k = 0; k < K; k++) acc = acc + bf2f(wr[k]) * bf2f(xr[k]);
    }
    if (o < O) y[(size_t)m * O + o] = f2bf(acc);
}

// 16 consecutive codes of row r at k (zeros past the row or past K)
__device__ __forceinline__ bf16x8 ld_op(const uint16_t *base, int r, int nrows, int K, int k) {
    u16x8 v = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if (r < nrows && k < K) v = *reinterpret_cast<const u16x8 *>(base + (size_t)r * K + k);
    return __builtin_bit_cast(bf16x8, v);
}

constexpr int MT = 64, OT = 64, MB = MT / 16;

__global__ __launch_bounds__(256) void k_gemm_mfma(const uint16_t *__restrict__ w,
                                                   const uint16_t *__restrict__ x,
                                                   uint16_t *__restrict__ y, int M, int O, int K) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g8 = (lane >> 4) * 8, kq = (lane >> 4) * 4;
    const int o = blockIdx.x * OT + wave * 16 + r16;     // this lane's weight row
    const int m0 = blockIdx.y * MT;
    f32x4 acc[MB];
#pragma unroll
    for (int b = 0; b < MB; b++) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    // one k step ahead
    bf16x8 bw = ld_op(w, o, O, K, g8), ax[MB];
#pragma unroll
    for (int b = 0; b < MB; b++) ax[b] = ld_op(x, m0 + b * 16 + r16, M, K, g8);
    for (int k = 0; k < K; k += 32) {
        const bf16x8 bc = bw;
        bf16x8 ac[MB];
#pragma unroll
        for (int b = 0; b < MB; b++) ac[b] = ax[b];
        bw = ld_op(w, o, O, K, k + 32 + g8);
#pragma unroll
        for (int b = 0; b < MB; b++) ax[b] = ld_op(x, m0 + b * 16 + r16, M, K, k + 32 + g8);
#pragma unroll
        for (int b = 0; b < MB; b++)
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac[b], bc, acc[b], 0, 0, 0);
    }
    // D[row kq + i][column r16] of row block b: row m0 + 16b + kq + i, output o
    if (o < O) {
#pragma unroll
        for (int b = 0; b < MB; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + b * 16 + kq + i;
                if (m < M) y[(size_t)m * O + o] = f2bf(acc[b][i]);
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
        APUS_TIMED("k_gemm_seq", k_gemm_seq<true><<<grid, 64, 0, stream()>>>(w, x, y, (int)O, (int)K));
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
    if (K % 8 != 0 || ((uintptr_t)w | (uintptr_t)x) % 16 != 0)
        return set_error(kErrUnsupported, "MFMA gemm needs K %% 8 == 0 and 16-byte aligned rows");
    const dim3 grid(cdiv(O, OT), cdiv(M, MT));
    APUS_TIMED("k_gemm_mfma",
               k_gemm_mfma<<<grid, 256, 0, stream()>>>(w, x, y, (int)M, (int)O, (int)K));
    return launch_check("k_gemm_mfma");
}

}  // extern "C"
