// FP32 MFMA GEMM shared by the batched decode and the chunked prefill:
//   Y[m, n] = sum_k X[m, k] * W[n, k]   (+ fused epilogue)
// X: activations, row-major (M, K); W: weights, row-major (N, K) in fp32 or
// INT4 groups (quant.c's packing, dequantized bit-exactly while staging).
#pragma once

#include "common.h"

namespace snhip {

enum GemmEpi {
    GEPI_STORE = 0,   // Y = acc
    GEPI_WEDGE = 1,   // Y = acc (1 + a/2 / (1 + |acc|))
    GEPI_RESID = 2,   // Y = acc + (b_gain s + sfb + Y)
    GEPI_ADD = 3,     // Y = Y + acc
    GEPI_RELU2 = 4,   // Y = max(acc, 0)^2
    // Competitive gate and state update of the decode step on the U product
    // (rows in the qrow_u / qrow_g order, N = 2 * channels): for channel i,
    // Y[m, i] = u and s[m, i] <- p s + (1 - p) u. See gemm_fuses_compete.
    GEPI_COMPETE = 5,
};

struct GemmArgs {
    // X rows. If shift_T > 0, row m reads X[m - 1] except when m % shift_T == 0,
    // where it reads X0[m / shift_T] (the previous time step within each
    // sequence, the carried state at t = 0).
    const float* X; long ldx;
    const float* X0; long ldx0; int shift_T;
    // weights
    const float* w;           // fp32 (N, K) row-major, or nullptr
    const uint8_t* q;         // int4 (N, K/2)
    const float* sc;          // int4 scales (N, K/block)
    int block;                // int4 group size (32 or 64), 0 for fp32
    int M, N, K;
    float* Y; long ldy;
    // epilogue
    int epi;
    float a_tanh, b_gain;
    const float* s; long lds;     // GEPI_RESID: Y = acc + (b_gain * s + sfb + Y)
    const float* sfb; long ldf;
    // GEPI_COMPETE: per-channel delta, the state in s / lds, p clamp
    const float* delta; int clamp; float p_floor;
};

// Device scratch of the GEMMs: split-K partials and the per-tile arrival
// counters of the skinny path (zero between launches; each launch leaves
// them zero).
struct GemmWork {
    float* part = nullptr;
    size_t part_floats = 0;
    unsigned* cnt = nullptr;
    int ncnt = 0;
};

// Products with at most 64 rows of X take the tiny-tile path (16 x 16 tiles,
// no exchange between workgroups) when N <= 8192 and K is a multiple of 64
// up to 3072, else the skinny path (64 x 64 tiles, split K with an in-kernel
// reduction) when `w` has counters, else the general kernel.
bool gemm_skinny(const GemmArgs& g, const GemmWork& w);
// Whether launch_gemm can apply GEPI_COMPETE to `g` (tiny-tile or skinny path).
bool gemm_fuses_compete(const GemmArgs& g, const GemmWork& w);

// Enqueue Y = X W^T with the epilogue. `work` is scratch for split-K partials
// (may be nullptr; then no split is used) of `work_floats` floats.
snhip_status launch_gemm(const GemmArgs& g, float* work, size_t work_floats, hipStream_t st);
// Same, with the skinny path available when `w` has counters.
snhip_status launch_gemm(const GemmArgs& g, const GemmWork& w, hipStream_t st);
// Two independent products in one launch when both take the skinny path with
// the same weight format; otherwise two launches.
snhip_status launch_gemm2(const GemmArgs& a, const GemmArgs& b, const GemmWork& w, hipStream_t st);

}  // namespace snhip
