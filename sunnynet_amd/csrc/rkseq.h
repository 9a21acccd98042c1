// Order-faithful RWKV-7 step kernels (rkseq.hip): every rounding step of the
// reference's C runtime (sunnynet/runtime/rwkv7.c:89-360) in its order, so a
// step on identical inputs gives the reference's bits.
#pragma once

#include "common.h"

namespace snhip {

// Product epilogues, applied to the finished sum y of an output.
enum RkqEpi {
    RKQ_STORE = 0,     // Y = y
    RKQ_ADD = 1,       // Y = Y + y            (residual, rwkv7.c:297, 317)
    RKQ_RELU2 = 2,     // t = y > 0 ? y : 0; Y = t * t   (rwkv7.c:309-313)
    RKQ_TANH = 3,      // Y = tanhf(y)         (rwkv7.c:235)
    RKQ_SIGMOID = 4,   // Y = 1 / (1 + expf(-y)) (rwkv7.c:256)
};

// One product Y[b] = W X[b] for the batch's rows b: W (M, Kd) row-major, fp32
// (w) or INT4 codes + scales in quant.c's packing (q, sc). Each output is the
// reference's chain acc = fmaf(X[b][k], W[j][k], acc) over k = 0 .. Kd-1 from
// acc = 0 (outputs j >= M & ~7 take acc = acc + X W, two roundings, as the
// reference's scalar column tail does). Kd is a multiple of 4 (fp32) or of the
// group size (INT4); X rows 16-byte aligned.
struct RkqJob {
    const float* X;
    int ldx;
    const float* w;
    const uint8_t* q;
    const float* sc;
    int M, Kd;
    float* Y;
    int ldy;
    int epi;
};
constexpr int kRkqMaxJobs = 8;

// Jobs share the weight format: block 0 = fp32 rows, 32 or 64 = INT4 group,
// -1 = tiled fp32 (float4 (t * Kd / 4 + kb) * 64 + l = inputs 4 kb .. 4 kb + 3
// of row 64 t + l, then a zeroed pad; launch_rkq_block4 makes them).
snhip_status launch_rkq_mm(const RkqJob* jobs, int n, int B, int block, hipStream_t st);
// floats of the tiled fp32 form of an M x Kd matrix, pad included
size_t rkq_tiled_floats(int M, int Kd);
// out (rkq_tiled_floats) = the tiled fp32 form of an M x Kd matrix given as
// fp32 rows w (block 0) or INT4 codes q and scales sc (block 32 or 64), each
// value the one the products multiply by.
snhip_status launch_rkq_block4(const float* w, const uint8_t* q, const float* sc, int block, int M, int Kd,
                               float* out, hipStream_t st);
// The same with the INT4 workgroup shape given: nc consumer waves of s chains
// of 4 sequences (nc in {1, 2, 4}, s in {1, 2}, not 4 x 2), or s = 16: one
// 16x16x1 chain of 16 sequences per consumer; 0 = chosen by B and the grid.
snhip_status launch_rkq_mm_cfg(const RkqJob* jobs, int n, int B, int block, int nc, int s,
                               hipStream_t st);

// Row LayerNorm (rwkv7.c:127-140: sequential sums, two passes) over D <= 4096,
// then one of the step's uses of it.
enum RkqLnMode {
    RKQ_LN_EMBED = 0,  // x[b] = LN(E[tok[b]])             (rwkv7.c:351-352)
    RKQ_LN_MIX1 = 1,   // xn = LN(x[b]); the six token-shift mixes; shift_0 = xn (:213-227)
    RKQ_LN_MIX2 = 2,   // xn2 = LN(x[b]); xk2 = xn2 + cmk_lerp (shift_1 - xn2); shift_1 = xn2
    RKQ_LN_PLAIN = 3,  // y[b] = LN(x[b])                  (output norm, :358)
};
struct RkqLnArgs {
    int mode, D, vocab;
    float eps;
    const int32_t* tok;      // EMBED
    const float* embed;      // EMBED
    const float* x;          // row b at x + b * D (EMBED writes it)
    const float *g, *c;      // gain, bias
    const float* lerp;       // MIX1: (6, D); MIX2: (D)
    float* shift;            // MIX1: shift_0 row of sequence b at shift + b * shift_bstride; MIX2: shift_1
    size_t shift_bstride;
    float* out;              // EMBED: x; MIX1: X6 (B, 6, D); MIX2: xk2 (B, D); PLAIN: y (B, D)
};
snhip_status launch_rkq_ln(const RkqLnArgs& a, int B, hipStream_t st);

// Per (head, sequence): decay, value residual, in-context rate, normalized
// kk, the 64 x 64 state update and read-out with the reference's eight
// stride-8 partial sums, group norm, bonus and gate (rwkv7.c:143-189, 228-299).
struct RkqHeadArgs {
    const float *r, *k, *v, *dw, *da, *dv, *g;   // (B, D) each; dv unused in layer 0
    float* vfirst;                                // (B, D)
    const float *w0, *a0, *v0, *kk_w, *ka_w, *rk_w, *lnx_w, *lnx_b;
    float* S;            // layer base; sequence b at S + b * s_bstride, head h at + h * 64 * 64
    size_t s_bstride;
    float* y;            // (B, D)
    int D, NH, first;
    float* dbg;          // if set: sequence 0's k, v, a, ww at dbg + 2D, 3D, 4D, 6D (rwkv7.c:308-319)
    // The LoRA up-projections w2, a2, g2, v2 computed here from their INT4
    // codes (up_blk 32 or 64, ranks up_k <= 128; v2 not in layer 0) instead
    // of read from dw, da, g, dv (up_blk 0): inputs lw, la, lg, lv of
    // sequence b at up_x[m] + b * up_ldx; the gate also goes to g (the dump
    // reads it there).
    const uint8_t* up_q[4];
    const float* up_sc[4];
    const float* up_x[4];
    int up_k[4];
    int up_blk, up_ldx;
    float* g_out;
};
snhip_status launch_rkq_heads(const RkqHeadArgs& a, int B, hipStream_t st);

}  // namespace snhip
