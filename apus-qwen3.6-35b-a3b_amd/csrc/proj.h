// proj.h -- the MFMA GEMM of proj.hip for the other translation units
// (the layer entry points of layer.hip).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace apus {

// The output rows of one GEMM may come from up to four weight matrices
// with their own outputs (the reference's in_proj_qkv / _z / _b / _a,
// c/layer.h:250-253, or wq / wk / wv, c/layer.h:300-302, computed as one
// launch over the same x): output row o in [row0[i], row0[i+1]) is row
// o - row0[i] of w[i] and lands in y[i][m * ldy[i] + o - row0[i]].
// Boundaries are multiples of 32, so a 16-row copy piece and a 32-row MFMA
// tile each lie in one segment.
constexpr int kMaxSegs = 4;
struct GemmSegs {
    int n;
    int row0[kMaxSegs + 1];
    const uint16_t *w[kMaxSegs];
    uint16_t *y[kMaxSegs];
    int ldy[kMaxSegs];
};

// y = x w^T over the segments of sg (row0[n] output rows in all) for M rows
// of x [M][K]; name: the timing / error name of the launch. Call
// gemm_tile_check first.
int gemm_tile(const GemmSegs &sg, const uint16_t *x, size_t M, size_t K, const char *name);
// the same with an explicit tile configuration (cfg 0: 64x64, or 128x64
// past 64 rows; 1: 128x128; 2: 128x128 up to 128 rows, 128x192 up to 384,
// else 128x256; 3: 256x256; -1: by shape) and nsplit k splits (fp32
// partials in library scratch, summed in split order by k_gemm_reduce)
int gemm_tile_split(const GemmSegs &sg, const uint16_t *x, size_t M, size_t K, const char *name,
                    int cfg, int nsplit);
// K a multiple of 32, x 16-byte aligned, operands under 2 GiB (weights:
// the caller checks their alignment)
int gemm_tile_check(const uint16_t *x, size_t M, size_t O, size_t K);

}  // namespace apus
