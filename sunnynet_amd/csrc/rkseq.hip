// Order-faithful RWKV-7 step kernels (rkseq.h).
//
// The reference's C runtime (sunnynet/runtime/rwkv7.c) rounds in a fixed
// order: every matrix product is a sequential fmaf chain over the inputs,
// LayerNorm and group-norm statistics are sequential sums, the head state
// dots use eight stride-8 partial sums folded as ((0+4)+(1+5))+((2+6)+(3+7)),
// and expf / tanhf are glibc's. The kernels here repeat exactly that:
//
// * Products run on the matrix cores with v_mfma_f32_4x4x1_16b_f32. With one
//   product per output per instruction, each instruction is acc + x w with a
//   single rounding (checked on gfx950: equal to fmaf on every output, and a
//   chain of them in k order equal to the sequential fmaf chain), so issuing
//   them in k order gives the reference's chain. A wave owns 64 output rows
//   (lane l supplies row out0 + l as the B operand and holds that column of
//   every 4 x 4 block) and S groups of 4 sequences (the A operands); INT4
//   weights are dequantized in registers as fma(q, s, -8 s), which equals
//   quant.c's (q - 8) s.
// * LayerNorm: one wave per row, the row in LDS, one lane running each
//   sequential sum while the others prepare the squared deviations.
// * Heads: one wave per (head, sequence), lane i owning state row i.
// * expf / tanhf: refmath.h (glibc's algorithms).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <type_traits>

#include "lanesum.h"
#include "refmath.h"
#include "rkseq.h"
#include "snhip_rwkv7.h"

namespace snhip {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

constexpr float kR2 = 0.6065306597126334f;   // 1/sqrt(e), rwkv7.c:38
constexpr float kEpsGroup = 6.4e-4f;          // rwkv7.c:39
constexpr int kHS = 64;
constexpr int kLnMax = 4096;

__device__ __forceinline__ float hsum8(const float* v) {
    const float c0 = v[0] + v[4], c1 = v[1] + v[5], c2 = v[2] + v[6], c3 = v[3] + v[7];
    return (c0 + c1) + (c2 + c3);
}

// ------------------------------------------------------------------ rows
// Sequential fp32 sum of n4 float4 in LDS (element order), by one lane.
// Rows whose length is a multiple of 64 run through a window of 16 float4:
// slot i is added, then refilled with the same slot of the next block, so
// the reads stay one block (64 dependent adds) ahead with no register copies
// and only the chain of dependent adds is exposed.
__device__ __forceinline__ float seq_sum(const float4* v, int n4) {
    float s = 0.0f;
    if (n4 % 16 == 0) {
        float4 w[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = v[i];
        for (int base = 0; base < n4; base += 16) {
            const int nb = min(base + 16, n4 - 16);   // the next block (the last block again at the end)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s = s + w[i].x; s = s + w[i].y; s = s + w[i].z; s = s + w[i].w;
                w[i] = v[nb + i];
            }
        }
        return s;
    }
    for (int i = 0; i < n4; ++i) {
        const float4 b = v[i];
        s = s + b.x; s = s + b.y; s = s + b.z; s = s + b.w;
    }
    return s;
}

// Row LayerNorm of rows up to kLnMax, one workgroup of LT threads per row:
// thread t owns float4 q = t + LT j of the row (elements 4q .. 4q+3); its
// row, gain, bias, shift and mix values are loaded as float4 before the sums,
// so the only exposed latencies are one round trip and the two sequential
// sums (one lane). 256 threads rather than one wave spread the row's loads
// and the mixes' stores: 9.6 -> 8.4 us per call at D = 768, B = 64.
constexpr int kLnR = 192;                  // float4 of a row held in registers (rows <= 768)
constexpr int kLnT = 256;                  // threads per row

template <int LT>
__global__ __launch_bounds__(LT) void k_rkq_ln(RkqLnArgs A) {
    constexpr int kLnQ = (kLnR + LT - 1) / LT;   // float4 per thread
    __shared__ float4 xs4[kLnMax / 4];
    __shared__ float4 sq4[kLnMax / 4];
    __shared__ float stat[2];
    const int b = blockIdx.x, t = threadIdx.x, D = A.D, n4 = D / 4;
    const float4* src;
    bool ok = true;
    if (A.mode == RKQ_LN_EMBED) {
        const int tk = A.tok[b];
        ok = tk >= 0 && tk < A.vocab;
        src = reinterpret_cast<const float4*>(A.embed + (size_t)(ok ? tk : 0) * D);
    } else {
        src = reinterpret_cast<const float4*>(A.x + (size_t)b * D);
    }
    float4* sh4 = A.shift ? reinterpret_cast<float4*>(A.shift + (size_t)b * A.shift_bstride) : nullptr;
    const float4* g4 = reinterpret_cast<const float4*>(A.g);
    const float4* c4 = reinterpret_cast<const float4*>(A.c);
    const float4* l4 = reinterpret_cast<const float4*>(A.lerp);
    const bool regs = n4 <= LT * kLnQ;
    const bool mix1 = A.mode == RKQ_LN_MIX1, mix2 = A.mode == RKQ_LN_MIX2;
    float4 gv[kLnQ], cv[kLnQ], sv[kLnQ], lv[6][kLnQ];
    for (int q = t; q < n4; q += LT) {
        float4 v = src[q];
        if (!ok) v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
        xs4[q] = v;
    }
    if (regs) {
#pragma unroll
        for (int j = 0; j < kLnQ; ++j) {
            const int q = min(t + LT * j, n4 - 1);
            gv[j] = g4[q];
            cv[j] = c4[q];
            if (mix1 || mix2) sv[j] = sh4[q];
            if (mix1) {
#pragma unroll
                for (int s6 = 0; s6 < 6; ++s6) lv[s6][j] = l4[(size_t)s6 * n4 + q];
            } else if (mix2) {
                lv[0][j] = l4[q];
            }
        }
    }
    __syncthreads();
    // sum = sum + x[i], then vsum = vsum + d * d, in order: lane-sliced in
    // wave 0 (lanesum.h) for rows of 256, 512, 768 or 1024, else by thread 0
    const int kl = D % 256 ? 0 : D / 256;
    if (kl >= 1 && kl <= 4) {
        if (t < 64) {
            auto go = [&](auto k) {
                constexpr int KL4 = decltype(k)::value;
                float v[4 * KL4];
#pragma unroll
                for (int q = 0; q < KL4; ++q) {
                    const float4 x = xs4[t * KL4 + q];
                    v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
                }
                float m, r;
                lane_ln_stats(v, D, A.eps, m, r);
                if (t == 0) {
                    stat[0] = m;
                    stat[1] = r;
                }
            };
            if (kl == 1) go(std::integral_constant<int, 1>{});
            else if (kl == 2) go(std::integral_constant<int, 2>{});
            else if (kl == 3) go(std::integral_constant<int, 3>{});
            else go(std::integral_constant<int, 4>{});
        }
        __syncthreads();
    } else {
        if (t == 0) stat[0] = seq_sum(xs4, n4) / (float)D;
        __syncthreads();
        const float m0 = stat[0];
        for (int q = t; q < n4; q += LT) {
            const float4 v = xs4[q];
            float4 d;
            d.x = v.x - m0; d.y = v.y - m0; d.z = v.z - m0; d.w = v.w - m0;
            d.x = d.x * d.x; d.y = d.y * d.y; d.z = d.z * d.z; d.w = d.w * d.w;
            sq4[q] = d;
        }
        __syncthreads();
        if (t == 0) stat[1] = 1.0f / sqrtf(seq_sum(sq4, n4) / (float)D + A.eps);
        __syncthreads();
    }
    const float mean = stat[0], rstd = stat[1];
    float4* o4 = reinterpret_cast<float4*>(A.out);
    auto norm = [&](float x, float g, float c) { return (x - mean) * rstd * g + c; };
    auto emit = [&](int q, float4 g, float4 c, float4 sh, const float4* lp) {
        const float4 x = xs4[q];
        float4 xn;
        xn.x = norm(x.x, g.x, c.x); xn.y = norm(x.y, g.y, c.y);
        xn.z = norm(x.z, g.z, c.z); xn.w = norm(x.w, g.w, c.w);
        if (mix1) {
            float4 d;
            d.x = sh.x - xn.x; d.y = sh.y - xn.y; d.z = sh.z - xn.z; d.w = sh.w - xn.w;
#pragma unroll
            for (int s6 = 0; s6 < 6; ++s6) {
                float4 r;
                r.x = xn.x + lp[s6].x * d.x; r.y = xn.y + lp[s6].y * d.y;
                r.z = xn.z + lp[s6].z * d.z; r.w = xn.w + lp[s6].w * d.w;
                o4[(size_t)b * 6 * n4 + (size_t)s6 * n4 + q] = r;
            }
            sh4[q] = xn;
        } else if (mix2) {
            float4 r;
            r.x = xn.x + lp[0].x * (sh.x - xn.x); r.y = xn.y + lp[0].y * (sh.y - xn.y);
            r.z = xn.z + lp[0].z * (sh.z - xn.z); r.w = xn.w + lp[0].w * (sh.w - xn.w);
            o4[(size_t)b * n4 + q] = r;
            sh4[q] = xn;
        } else {
            o4[(size_t)b * n4 + q] = xn;
        }
    };
    if (regs) {
#pragma unroll
        for (int j = 0; j < kLnQ; ++j) {
            const int q = t + LT * j;
            if (q < n4) {
                const float4 lp[6] = {lv[0][j], lv[1][j], lv[2][j], lv[3][j], lv[4][j], lv[5][j]};
                emit(q, gv[j], cv[j], sv[j], lp);
            }
        }
    } else {
        for (int q = t; q < n4; q += LT) {   // longer rows: parameters loaded as used
            float4 lp[6], sh = make_float4(0.f, 0.f, 0.f, 0.f);
            if (mix1 || mix2) sh = sh4[q];
            if (mix1) {
                for (int s6 = 0; s6 < 6; ++s6) lp[s6] = l4[(size_t)s6 * n4 + q];
            } else if (mix2) {
                lp[0] = l4[q];
            }
            emit(q, g4[q], c4[q], sh, lp);
        }
    }
}

// ------------------------------------------------------------- products
struct RkqMMArgs {
    RkqJob j[kRkqMaxJobs];
    int start[kRkqMaxJobs + 1];   // first workgroup of each job
    int tiles_out[kRkqMaxJobs];   // 64-row tiles of each job
    int n, B, seq_tiles;
    int xs_per_wave;              // tiled fp32: float4 of LDS per wave
};

__device__ __forceinline__ float dequant_at(const RkqJob& J, int row, int k, int blk) {
    if (blk < 0)   // tiled fp32 (k_rkq_mm_w4)
        return J.w[(((size_t)(row >> 6) * (size_t)(J.Kd >> 2) + (size_t)(k >> 2)) * 64 + (row & 63)) * 4 + (k & 3)];
    if (!blk) return J.w[(size_t)row * J.Kd + k];
    const int half = blk / 2, g = k / blk, e = k % blk;
    const uint8_t byte = J.q[(size_t)row * (J.Kd / 2) + (size_t)g * half + (e % half)];
    const float sc = J.sc[(size_t)row * (J.Kd / blk) + g];
    const int qv = e < half ? (byte & 0x0F) : (byte >> 4);
    return fmaf((float)qv, sc, -8.0f * sc);
}

template <int S>
__device__ __forceinline__ void mfma_k(const float (&xv)[S], float wv, v4f (&acc)[S]) {
#pragma unroll
    for (int s = 0; s < S; ++s) acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xv[s], wv, acc[s], 0, 0, 0);
}

template <int S>
__device__ __forceinline__ void step4(const float4 (&x4)[S], float w0, float w1, float w2, float w3,
                                      v4f (&acc)[S]) {
    float xv[S];
#pragma unroll
    for (int s = 0; s < S; ++s) xv[s] = x4[s].x;
    mfma_k<S>(xv, w0, acc);
#pragma unroll
    for (int s = 0; s < S; ++s) xv[s] = x4[s].y;
    mfma_k<S>(xv, w1, acc);
#pragma unroll
    for (int s = 0; s < S; ++s) xv[s] = x4[s].z;
    mfma_k<S>(xv, w2, acc);
#pragma unroll
    for (int s = 0; s < S; ++s) xv[s] = x4[s].w;
    mfma_k<S>(xv, w3, acc);
}

template <int S>
__device__ __forceinline__ void step4(const v4f (&x4)[S], float w0, float w1, float w2, float w3, v4f (&acc)[S]) {
    float xv[S];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int s = 0; s < S; ++s) xv[s] = x4[s][c];
        mfma_k<S>(xv, c == 0 ? w0 : c == 1 ? w1 : c == 2 ? w2 : w3, acc);
    }
}

// Inputs per chunk staged in LDS at once (X rows; INT4 codes in registers).
constexpr int kRkqKC = 768;
constexpr int kRkqU = 64;                  // INT4: inputs per pipeline unit (two producer halves of 32)
constexpr int kRkqNP = 2;                  // producer waves of an INT4 workgroup

// This workgroup's job (uniform selects: no dynamic index into the arguments).
// The first workgroup of the job is selected in the same pass as the job
// index: selecting it by index afterwards was folded back into an indexed
// read of a local copy of start[], which the compiler kept in scratch memory
// (a store and a dependent load at every launch).
__device__ __forceinline__ void rkq_job_at(const RkqMMArgs& A, int wg, RkqJob& J, int& u0) {
    int ji = 0, j0 = A.start[0];
#pragma unroll
    for (int i = 1; i < kRkqMaxJobs; ++i)
        if (i < A.n && wg >= A.start[i]) { ji = i; j0 = A.start[i]; }
    J = A.j[0];
#pragma unroll
    for (int i = 1; i < kRkqMaxJobs; ++i)
        if (i == ji) J = A.j[i];
    u0 = wg - j0;
}
__device__ __forceinline__ void rkq_job(const RkqMMArgs& A, RkqJob& J, int& u0) {
    rkq_job_at(A, (int)blockIdx.x, J, u0);
}

// Tail columns and the epilogue of one lane's 4 sequences (seq0 .. seq0+3)
// of output column `out`. Columns past the last multiple of 8 take the
// reference's scalar tail (acc + x * w, two roundings).
__device__ __forceinline__ void rkq_finish(const RkqJob& J, int B, int blk, int seq0, int out,
                                           v4f acc) {
    if (out >= J.M) return;
    if (out >= (J.M & ~7)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int sq = seq0 + i;
            if (sq >= B) continue;
            const float* x = J.X + (size_t)sq * J.ldx;
            float a2 = 0.0f;
            for (int k = 0; k < J.Kd; ++k) a2 = a2 + x[k] * dequant_at(J, out, k, blk);
            acc[i] = a2;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int sq = seq0 + i;
        if (sq >= B) continue;
        float* y = J.Y + (size_t)sq * J.ldy + out;
        const float v = acc[i];
        switch (J.epi) {
        case RKQ_ADD: *y = *y + v; break;
        case RKQ_RELU2: { const float r = v > 0.0f ? v : 0.0f; *y = r * r; break; }
        case RKQ_TANH: *y = refmath::tanhf(v); break;
        case RKQ_SIGMOID: *y = refmath::sigmoid(v); break;
        default: *y = v; break;
        }
    }
}

// One output (sequence sq, column out) of a chain sum v: the scalar tail
// past the last multiple of 8 as in rkq_finish, then the epilogue.
__device__ __forceinline__ void rkq_finish1(const RkqJob& J, int B, int blk, int sq, int out, float v) {
    if (out >= J.M || sq >= B) return;
    if (out >= (J.M & ~7)) {
        const float* x = J.X + (size_t)sq * J.ldx;
        float a2 = 0.0f;
        for (int k = 0; k < J.Kd; ++k) a2 = a2 + x[k] * dequant_at(J, out, k, blk);
        v = a2;
    }
    float* y = J.Y + (size_t)sq * J.ldy + out;
    switch (J.epi) {
    case RKQ_ADD: *y = *y + v; break;
    case RKQ_RELU2: { const float r = v > 0.0f ? v : 0.0f; *y = r * r; break; }
    case RKQ_TANH: *y = refmath::tanhf(v); break;
    case RKQ_SIGMOID: *y = refmath::sigmoid(v); break;
    default: *y = v; break;
    }
}

// fp32 weights: one wave per 64 rows x S groups of 4 sequences; X of the
// chunk in LDS, the lane's weight row read 32 inputs ahead.
template <int S>
__global__ __launch_bounds__(64) void k_rkq_mm_f32(const RkqMMArgs A) {
    __shared__ float4 xs4[4 * S * (kRkqKC / 4)];   // X row (4 s + r) at (4 s + r) * KC
    RkqJob J;
    int u0;
    rkq_job(A, J, u0);
    const int ot = u0 / A.seq_tiles, st = u0 % A.seq_tiles;
    const int l = threadIdx.x, r4 = l & 3;
    const int out = ot * 64 + l;
    const int orow = out < J.M ? out : J.M - 1;
    const int seq0 = st * 4 * S;
    v4f acc[S];
#pragma unroll
    for (int s = 0; s < S; ++s) acc[s] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < J.Kd; k0 += kRkqKC) {
        const int kc = min(kRkqKC, J.Kd - k0);
        __syncthreads();
        const int nq = kc / 4;
        for (int idx = l; idx < 4 * S * nq; idx += 64) {
            const int row = idx / nq, q = idx - row * nq;
            const int sq = seq0 + row;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (sq < A.B) v = *reinterpret_cast<const float4*>(J.X + (size_t)sq * J.ldx + k0 + 4 * q);
            xs4[row * (kRkqKC / 4) + q] = v;
        }
        const float4* xl = xs4 + r4 * (kRkqKC / 4);
        const float* wr = J.w + (size_t)orow * J.Kd + k0;
        float4 wc[8], wn[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (4 * i < kc) wc[i] = *reinterpret_cast<const float4*>(wr + 4 * i);
        __syncthreads();
        for (int kb = 0; kb < kc; kb += 32) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (kb + 32 + 4 * i < kc) wn[i] = *reinterpret_cast<const float4*>(wr + kb + 32 + 4 * i);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (kb + 4 * i < kc) {
                    float4 x4[S];
#pragma unroll
                    for (int s = 0; s < S; ++s) x4[s] = xl[4 * s * (kRkqKC / 4) + kb / 4 + i];
                    step4<S>(x4, wc[i].x, wc[i].y, wc[i].z, wc[i].w, acc);
                }
#pragma unroll
            for (int i = 0; i < 8; ++i) wc[i] = wn[i];
        }
    }
#pragma unroll
    for (int s = 0; s < S; ++s) rkq_finish(J, A.B, 0, seq0 + 4 * s, out, acc[s]);
}

// Tiled fp32 weights (block = -1), made at load from the INT4 codes with the
// producers' dequantization, or from fp32 rows: float4 (t * nb + kb) * 64 + l
// holds inputs 4 kb .. 4 kb + 3 of row 64 t + l (rows past M repeat row
// M - 1), nb = Kd / 4, followed by kRkwPad float4 that loads past the end
// may touch. One wave per 64 rows x S groups of 4 sequences (one wave per
// workgroup unless a tuning shape groups NW of an output tile's waves),
// nothing shared between waves, so no barrier paces its chains. A chain
// step is one dependent v_mfma_f32_4x4x1_16b_f32 (~13 cycles on gfx950),
// and every other instruction of the wave lengthens it (measured: X read from
// LDS once per 4 inputs, 13.3 -> 15.3 cycles per input; with 64-bit address
// arithmetic for a weight load added, 21), so a block of 4 inputs issues
// only its MFMAs, one buffer load of the next weights (1 KiB of consecutive
// memory; the scalar offset advances, the lane offset and the immediate stay
// fixed) and one LDS read of X at an immediate offset from the lane's base.
// The wave's X rows go straight into LDS at the start (one load latency);
// its weight blocks run PF blocks ahead in registers. Workgroups are
// renumbered so that consecutive numbers run on one XCD (dispatch is
// round-robin over the 8 XCDs): the sequence tiles of an output tile then
// read its weights from one L2.
// Weight blocks in flight per wave (PF): chosen by the launcher, 48 while
// the launch's waves fit one per CU and 16 beyond, when each CU's loads in
// flight are several waves' worth (measured on the RWKV-7 step, cfg4 INT4:
// at B = 16 48 beat 24 by 2 % and 56 by 1 %; at B = 64, on the launches of
// 656 - 768 waves, 24 beat 48 by 2 % and 16 beat 24 by 0.4 %).
constexpr int kRkwXA = 4;          // X blocks read from LDS ahead of the MFMAs
constexpr int kRkwXMax = 4096;     // float4 of X per workgroup (64 KiB): S * Kd <= this
constexpr int kRkwPad = 64 * 64;   // float4 after a tiled matrix (64 blocks: the stream reads up to PF - 1 past a tile)
// s_waitcnt vmcnt(n) (expcnt, lgkmcnt at their maximum; gfx9 split vmcnt field)
constexpr int rkw_vmcnt(int n) { return ((n >> 4) & 3) << 14 | 0x0F70 | (n & 15); }

// Direct-to-LDS loads the compiler does not see (inline asm): lane l's 16
// (4) bytes at gaddr go to LDS byte lds + 16 l (4 l), lds wave-uniform. M0,
// which holds the LDS base, is saved and restored around the load, and one
// wait state separates its write from the load. Seen by the compiler
// (builtin), these writes to LDS counted as pending at every later LDS read
// of the kernel's chain loop, which then waited for all loads at the top of
// each trip and drained the weight prefetch; in a function of their own,
// the call boundary waited for every load. The caller waits for them itself:
// before its first read of what they bring, and for all of them before the
// wave ends (its LDS may then go to another workgroup).
__device__ __forceinline__ void dma_lds16(const void* gaddr, uint32_t lds) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(gaddr), "s"(lds)
        : "memory");
}
__device__ __forceinline__ void dma_lds4(const void* gaddr, uint32_t lds) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(gaddr), "s"(lds)
        : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) char*)p;
}

// An LDS address (LDS-typed, so reads through it are ds_read, counted by
// lgkmcnt only) held in a vector register as far as the compiler knows, so
// that reads through it keep their whole address in the one register and
// take the rest as an immediate offset.
typedef __attribute__((address_space(3))) const v4f lds_f4;
__device__ __forceinline__ const lds_f4* lds_vbase(const float4* p) {
    uint32_t a = (uint32_t)(size_t)(const lds_f4*)p;
    asm volatile("" : "+v"(a));
    return (const lds_f4*)(size_t)a;
}

template <int S, int NW, int PF>
__global__ __launch_bounds__(64 * NW) void k_rkq_mm_w4(const RkqMMArgs A) {
    constexpr int R = 4 * S;   // sequences of the wave
    static_assert(PF % kRkwXA == 0, "the X ring restarts with each weight group");
    extern __shared__ float4 xsh[];
    // NW independent waves per workgroup (one per SIMD): sequence tiles
    // NW u0 .. NW u0 + NW - 1 of one output tile; a wave past the last tile
    // has no work (nothing here waits on another wave)
    const int T = (int)gridDim.x, b = (int)blockIdx.x, q8 = T / 8, r8 = T % 8, x8 = b % 8;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    RkqJob J;
    int u0;
    rkq_job_at(A, x8 * q8 + min(x8, r8) + b / 8, J, u0);
    const int wg_per_tile = (A.seq_tiles + NW - 1) / NW;
    const int ot = u0 / wg_per_tile, st = (u0 % wg_per_tile) * NW + wv;
    if (st >= A.seq_tiles) return;
    float4* xs = xsh + (size_t)wv * (A.xs_per_wave);
    const int l = threadIdx.x & 63, r4 = l & 3;
    const int out = ot * 64 + l;
    const int seq0 = st * R;
    const int nb = J.Kd / 4;
    // the whole tiled matrix with its padding; block kb of this tile at
    // scalar offset (ot * nb + kb) * 1 KiB, lane offset 16 l
    const uint32_t bytes = (uint32_t)(((size_t)((J.M + 63) / 64) * nb * 64 + kRkwPad) * sizeof(float4));
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(J.w), (short)0, (int)bytes,
                                                                        0x00020000);
    const int vo = 16 * l;
    const int sob = ot * nb * 1024;
    auto ldw = [&](int kb) -> float4 {
        const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(rw, vo, sob + kb * 1024, 0);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
    };
    // The wave's X rows into LDS (float4 f = kb * R + row: lane l of pass f0
    // brings float4 f0 + l; past the end the last one again, into the
    // padding of the launch's LDS size).
    const int nx = nb * R;
    for (int f0 = 0; f0 < nx; f0 += 64) {
        const int f = min(f0 + l, nx - 1);
        const int kb = f / R, row = f - kb * R;
        dma_lds16(J.X + (size_t)min(seq0 + row, A.B - 1) * (size_t)J.ldx + 4 * kb, lds_addr(xs + f0));
    }
    float4 w[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) w[i] = ldw(i);
    // X in: every load but the PF weight loads above
    __builtin_amdgcn_s_waitcnt(rkw_vmcnt(PF));
    __builtin_amdgcn_sched_barrier(0);
    // The L2 prefetch, issued once X is in (so the chains do not wait for
    // it): this sequence tile's share of the output tile's weights past the
    // first PF blocks (at most 63 - PF blocks, so that the wave's loads in
    // flight fit the wait counter; lane l touches bytes 16 l .. + 4 of each
    // 1 KiB block, so every 128-byte line) into a 256-byte LDS slot nothing
    // reads. The sequence tiles of an output tile each take their own part,
    // so its weights leave HBM together rather than block by block as every
    // chain reaches them.
    {
        const int rest = max(nb - PF, 0), share = (rest + A.seq_tiles - 1) / A.seq_tiles;
        const int pf0 = PF + min(st * share, rest);
        // only in the shallow form (several waves per CU): with one wave per
        // CU the deep stream alone was faster (B = 16 1,145 -> 1,125 us/step
        // without it; B = 64 1,304 -> 1,297 with it on the shallow launches only)
        const int npf = PF < 48 ? min(min(share, nb - pf0), 63 - PF) : 0;
        const char* wb = reinterpret_cast<const char*>(J.w) + (size_t)(sob + pf0 * 1024) + 16 * l;
        const uint32_t dump = lds_addr(xs + A.xs_per_wave - 16);
        for (int j = 0; j < npf; ++j) dma_lds4(wb + 1024 * j, dump);
    }
    __builtin_amdgcn_sched_barrier(0);
    v4f xa[kRkwXA][S];
    v4f acc[S];
#pragma unroll
    for (int s = 0; s < S; ++s) acc[s] = v4f{0.f, 0.f, 0.f, 0.f};
    {
        const lds_f4* xq = lds_vbase(xs + r4);   // block kb of group s: xq[kb * R + 4 s]
#pragma unroll
        for (int j = 0; j < kRkwXA; ++j)
#pragma unroll
            for (int s = 0; s < S; ++s) xa[j][s] = xq[j * R + 4 * s];
    }
    // X past block nb - 1 is read from the launch's LDS padding and weights
    // past the tile from the next tile or the padding, never used.
    int b0 = 0;
    for (; b0 + PF <= nb; b0 += PF) {
        const lds_f4* xq = lds_vbase(xs + r4 + b0 * R);
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            step4<S>(xa[i % kRkwXA], w[i].x, w[i].y, w[i].z, w[i].w, acc);
            w[i] = ldw(b0 + PF + i);
#pragma unroll
            for (int s = 0; s < S; ++s) xa[i % kRkwXA][s] = xq[(i + kRkwXA) * R + 4 * s];
            // each block's refill stays with it (the scheduler otherwise sank
            // the group's weight loads below its last MFMA)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const int rem = nb - b0;   // < PF blocks, already in registers
    const lds_f4* xq = lds_vbase(xs + r4 + b0 * R);
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        if (i < rem) {
            step4<S>(xa[i % kRkwXA], w[i].x, w[i].y, w[i].z, w[i].w, acc);
#pragma unroll
            for (int s = 0; s < S; ++s) xa[i % kRkwXA][s] = xq[(i + kRkwXA) * R + 4 * s];
        }
    }
    __builtin_amdgcn_s_waitcnt(rkw_vmcnt(0));   // the L2 prefetch's writes to LDS, before the wave can end
#pragma unroll
    for (int s = 0; s < S; ++s) rkq_finish(J, A.B, -1, seq0 + 4 * s, out, acc[s]);
}

// The tiled form (above) of an M x Kd matrix: each value the one the
// products use (dequant_at: fp32 rows, or INT4 codes dequantized as the
// producers do); the padding is zeroed.
__global__ __launch_bounds__(256) void k_rkq_block4(RkqJob J, int blk, float4* out) {
    const int nb = J.Kd / 4;
    const size_t n = (size_t)((J.M + 63) / 64) * nb * 64;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n + kRkwPad) return;
    if (i >= n) {
        out[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const int l = (int)(i % 64), kb = (int)((i / 64) % nb), t = (int)(i / 64 / nb);
    const int o = min(64 * t + l, J.M - 1);
    float4 v;
    v.x = dequant_at(J, o, 4 * kb, blk);
    v.y = dequant_at(J, o, 4 * kb + 1, blk);
    v.z = dequant_at(J, o, 4 * kb + 2, blk);
    v.w = dequant_at(J, o, 4 * kb + 3, blk);
    out[i] = v;
}

// INT4 weights: a workgroup of kRkqNP producer waves and NC consumer waves
// per 64 rows x 4 S NC sequences.
//
// Producer wave h dequantizes half h (32 inputs) of every 64-input unit of
// the rows: at step t it converts unit t from codes and scales it loaded
// kRkqPF units earlier into slot t % 3 of an LDS ring ([block][row] float4,
// conflict-free). Consumer c multiplies unit t - 2 at step t, S independent
// k-ordered MFMA chains of 4 sequences each sharing the weight operand. Its
// weight window runs kRkqWD blocks of 4 inputs ahead of the MFMAs and
// crosses into unit t - 1 (complete since the previous step), and its X
// operands come from global memory one unit ahead, so the chains wait on
// neither LDS nor global memory. One workgroup barrier per step, waiting on
// LDS only; every weight is dequantized once per workgroup.
constexpr int kRkqPF = 4;     // producer code prefetch, units
constexpr int kRkqWD = 8;     // consumer weight window, blocks of 4 inputs (a half unit)

// Producer wave h (0 or 1) of an INT4 product workgroup: converts half h of
// every 64-input unit of rows orow.. into slot t % 3 of the LDS ring at
// step t, one workgroup barrier per step, nsteps steps in all.
template <int BLK>
__device__ __forceinline__ void rkq_produce(const RkqJob& J, int h, int l, int orow, int nu, int nsteps,
                                            float4 (*wring)[kRkqU / 4][64]) {
    const int Kd = J.Kd;
    constexpr int NQ = BLK / 32;
    const uint8_t* qrow = J.q + (size_t)orow * (size_t)(Kd / 2);
    const float* srow = J.sc + (size_t)orow * (size_t)(Kd / BLK);
    uint4 qw[kRkqPF][NQ];
    float sw[kRkqPF];
    // Branch-free loads: a unit past the end reads the last half again
    // (never converted), so no wait depends on control flow.
    auto load = [&](int u, uint4 (&q)[NQ], float& s) {
        const int k = min(u * kRkqU + 32 * h, Kd - 32);
        if (BLK == 32) {
            q[0] = *reinterpret_cast<const uint4*>(qrow + k / 2);
            s = srow[k / 32];
        } else {
            const int g = k / 64;
#pragma unroll
            for (int i = 0; i < NQ; ++i) q[i] = *reinterpret_cast<const uint4*>(qrow + g * 32 + 16 * i);
            s = srow[g];
        }
    };
#pragma unroll
    for (int p = 0; p < kRkqPF; ++p) load(p, qw[p], sw[p]);
    // Groups of kRkqPF steps: a group first issues the loads of the next
    // group's units, then converts its own (loaded one group earlier), so
    // every wait on codes covers loads a whole group old.
    for (int t0 = 0; t0 < nsteps; t0 += kRkqPF) {
        uint4 qn[kRkqPF][NQ];
        float sn[kRkqPF];
#pragma unroll
        for (int p = 0; p < kRkqPF; ++p) load(t0 + kRkqPF + p, qn[p], sn[p]);
#pragma unroll
        for (int p = 0; p < kRkqPF; ++p) {
            const int t = t0 + p;
            // Converted unconditionally: past the last unit (or the
            // missing half of a half unit) this writes leftovers to slot
            // t % 3, which the consumers do not read at or after step t.
            const float scg = sw[p], m8 = -8.0f * scg;
            // Block i of the half: inputs 4i .. 4i+3. BLK 64: nibble h of
            // bytes 4i .. 4i+3; BLK 32: low nibbles of word i for i < 4,
            // high nibbles of word i - 4 after.
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 v = BLK == 32 ? qw[p][0] : qw[p][(i >> 2) % NQ];
                const int wi = i & 3;
                const uint32_t word = wi == 0 ? v.x : wi == 1 ? v.y : wi == 2 ? v.z : v.w;
                const bool hi = BLK == 32 ? i >= 4 : h == 1;
                uint32_t nib = (hi ? (word >> 4) : word) & 0x0F0F0F0Fu;
                // Opaque to the compiler, so that each byte converts with
                // one v_cvt_f32_ubyteN (no field extraction).
                asm volatile("" : "+v"(nib));
                float4 w;
                w.x = fmaf((float)(nib & 0xFFu), scg, m8);
                w.y = fmaf((float)((nib >> 8) & 0xFFu), scg, m8);
                w.z = fmaf((float)((nib >> 16) & 0xFFu), scg, m8);
                w.w = fmaf((float)(nib >> 24), scg, m8);
                wring[t % 3][8 * h + i][l] = w;
            }
            __syncthreads();
            // keep each step's conversion after its barrier
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int p = 0; p < kRkqPF; ++p) {
#pragma unroll
            for (int i = 0; i < NQ; ++i) qw[p][i] = qn[p][i];
            sw[p] = sn[p];
        }
    }
}

// X rows staged in LDS (XD = 0) take at most 64 KiB: rows of up to
// kRkqXLF / (sequences per workgroup) inputs.
constexpr int kRkqXLF = 16384;

template <int BLK, int NC, int S, int XD>
__global__ __launch_bounds__(64 * (NC + kRkqNP)) void k_rkq_mm_q4(const RkqMMArgs A) {
    constexpr int U4 = kRkqU / 4;                      // blocks per unit
    static_assert(U4 % kRkqWD == 0 && kRkqWD == U4 / 2, "the weight window is a half unit");
    constexpr int XR = XD > 0 ? XD : 1;                // X register sets
    constexpr int NSQ = 4 * S * NC;                    // sequences of the workgroup
    __shared__ float4 wring[3][U4][64];
    constexpr int XLK = kRkqXLF / NSQ;                 // inputs per staged row
    constexpr int XLS = XLK / 4 + 1;                   // row stride in float4 (padded: rows on distinct banks)
    __shared__ float4 xlds[XD == 0 ? NSQ * XLS : 1];
    RkqJob J;
    int u0;
    rkq_job(A, J, u0);
    const int ot = u0 / A.seq_tiles, st = u0 % A.seq_tiles;
    // wave index in a scalar register: every branch on the role is uniform
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, r4 = l & 3;
    const int out = ot * 64 + l;
    const int orow = out < J.M ? out : J.M - 1;
    const int Kd = J.Kd;
    const int nu = (Kd + kRkqU - 1) / kRkqU;            // the last unit is half when Kd % 64 == 32
    const bool half_last = (Kd % kRkqU) != 0;
    // Steps (one barrier each) for both roles: units 0 .. nu - 1 are written
    // at steps 0 .. nu - 1 and multiplied at steps 2 .. nu + 1; the count is
    // rounded up to the producer's prefetch depth (idle steps at the end).
    const int nsteps = (nu + 2 + kRkqPF - 1) / kRkqPF * kRkqPF;
    if constexpr (XD == 0) {
        // The X rows of the workgroup's sequences into LDS, by every wave
        // (Kd <= XLK; rows past the batch repeat the last sequence's).
        const int kq = Kd / 4;
        for (int idx = threadIdx.x; idx < NSQ * kq; idx += 64 * (NC + kRkqNP)) {
            const int sq = idx / kq, q = idx - sq * kq;
            xlds[sq * XLS + q] =
                *reinterpret_cast<const float4*>(J.X + (size_t)min(st * NSQ + sq, A.B - 1) * (size_t)J.ldx + 4 * q);
        }
        __syncthreads();
    }
    if (wv < kRkqNP) {
        rkq_produce<BLK>(J, wv, l, orow, nu, nsteps, wring);
        return;
    }
    // ---- consumer c: sequences seqb + 4 s + (0..3), lane row r4 of each chain.
    // Rows past the batch read the last sequence's X (their outputs are not
    // stored), and loads past the end re-read the last block, so every load
    // is unconditional and no wait depends on control flow.
    const int c = wv - kRkqNP;
    const int seqb = st * (4 * S * NC) + c * (4 * S);
    const float* xr[S];
#pragma unroll
    for (int s = 0; s < S; ++s)
        xr[s] = J.X + (size_t)min(seqb + 4 * s + r4, A.B - 1) * (size_t)J.ldx;
    // X operands run XR units ahead of the MFMAs, from global memory (XD = 1;
    // XD = 2 in launches of at most one workgroup per CU, whose chains then
    // wait on X less: the second set's registers would keep larger grids
    // from residing at three workgroups per CU) or from the rows staged in
    // LDS (XD = 0).
    static_assert(XD >= 0 && XD <= 2, "X depth");
    auto ldx = [&](int s, int k) -> float4 {
        if constexpr (XD == 0) return xlds[(c * 4 * S + 4 * s + r4) * XLS + (k >> 2)];
        else return *reinterpret_cast<const float4*>(xr[s] + k);
    };
    float4 xw[XR][S][U4];   // unit u's block i in xw[u % XR]; refilled with unit u + XR's
    float4 ww[kRkqWD];      // weight blocks, slot = block % kRkqWD
    v4f acc[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        acc[s] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < XR; ++d)
#pragma unroll
            for (int i = 0; i < U4; ++i) xw[d][s][i] = ldx(s, min(d * kRkqU + 4 * i, Kd - 4));
    }
    // Steps 0 and 1: the producers write units 0 and 1; the window takes
    // unit 0's first half once it is complete.
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRkqWD; ++j) ww[j] = wring[0][j][l];
    __syncthreads();
    // One full unit from X set P: block i's MFMAs, then its refills (weight
    // block i + kRkqWD, from the next unit's slot for the last half; X block i
    // of unit u + XD). Straight-line, so the window stays in place.
    auto full_unit = [&](auto par, int slot, int nslot, int knext) {
        constexpr int P = decltype(par)::value;
#pragma unroll
        for (int i = 0; i < U4; ++i) {
            const float4 wc = ww[i % kRkqWD];
#pragma unroll
            for (int s = 0; s < S; ++s) acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].x, wc.x, acc[s], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < S; ++s) acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].y, wc.y, acc[s], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < S; ++s) acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].z, wc.z, acc[s], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < S; ++s) acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].w, wc.w, acc[s], 0, 0, 0);
            ww[i % kRkqWD] = i + kRkqWD < U4 ? wring[slot][i + kRkqWD][l] : wring[nslot][i + kRkqWD - U4][l];
            const int kx = min(knext + 4 * i, Kd - 4);
#pragma unroll
            for (int s = 0; s < S; ++s) xw[P][s][i] = ldx(s, kx);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto half_unit = [&](auto par) {
        constexpr int P = decltype(par)::value;
#pragma unroll
        for (int i = 0; i < U4 / 2; ++i) {
            const float4 wc = ww[i % kRkqWD];
#pragma unroll
            for (int s = 0; s < S; ++s) {
                acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].x, wc.x, acc[s], 0, 0, 0);
                acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].y, wc.y, acc[s], 0, 0, 0);
                acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].z, wc.z, acc[s], 0, 0, 0);
                acc[s] = __builtin_amdgcn_mfma_f32_4x4x1f32(xw[P][s][i].w, wc.w, acc[s], 0, 0, 0);
            }
        }
    };
    constexpr std::integral_constant<int, 0> x0{};
    constexpr std::integral_constant<int, XR - 1> x1{};
    // Steps 2 .. nu: units 0 .. nu - 2, each followed by another; two at a
    // time, so that the X set of each is fixed at compile time.
    int u = 0;
    for (; u + 2 <= nu - 1; u += 2) {
        full_unit(x0, u % 3, (u + 1) % 3, (u + XR) * kRkqU);
        __syncthreads();
        full_unit(x1, (u + 1) % 3, (u + 2) % 3, (u + 1 + XR) * kRkqU);
        __syncthreads();
    }
    if (u < nu - 1) {   // one more (u even: set 0)
        full_unit(x0, u % 3, (u + 1) % 3, (u + XR) * kRkqU);
        __syncthreads();
        ++u;
    }
    // Step nu + 1: the last unit, u = nu - 1 (its refills read in-bounds
    // leftovers).
    if ((u & 1) == 0 || XR == 1) {
        if (!half_last) full_unit(x0, u % 3, (u + 1) % 3, Kd);
        else half_unit(x0);
    } else {
        if (!half_last) full_unit(x1, u % 3, (u + 1) % 3, Kd);
        else half_unit(x1);
    }
    __syncthreads();
    for (int t = nu + 2; t < nsteps; ++t) __syncthreads();
#pragma unroll
    for (int s = 0; s < S; ++s) rkq_finish(J, A.B, BLK, seqb + 4 * s, out, acc[s]);
}

// INT4 weights, wide form: as k_rkq_mm_q4, but each consumer wave runs one
// chain of v_mfma_f32_16x16x1_4b_f32 over 16 sequences. That instruction also
// holds one product per output per instruction and rounds once (checked on
// gfx950: a chain of them in k order equals the sequential fmaf chain), and
// one chain of it keeps a SIMD's matrix pipe busy (a dependent one issues
// every ~32.5 cycles, independent ones every ~32), so a wave covers 16
// sequences x 64 rows with one accumulator. Lane l supplies weight row
// out0 + l (B, block l / 16, column l % 16) and the input of sequence l % 16
// (A, the same rows in every block); it then holds, in register 4 b + r,
// sequence 4 (l / 16) + r of row out0 + 16 b + l % 16.
template <int BLK, int NC>
__global__ __launch_bounds__(64 * (NC + kRkqNP)) void k_rkq_mm_q4w(const RkqMMArgs A) {
    constexpr int U4 = kRkqU / 4;
    __shared__ float4 wring[3][U4][64];
    RkqJob J;
    int u0;
    rkq_job(A, J, u0);
    const int ot = u0 / A.seq_tiles, st = u0 % A.seq_tiles;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
    const int out = ot * 64 + l;
    const int orow = out < J.M ? out : J.M - 1;
    const int Kd = J.Kd;
    const int nu = (Kd + kRkqU - 1) / kRkqU;
    const bool half_last = (Kd % kRkqU) != 0;
    const int nsteps = (nu + 2 + kRkqPF - 1) / kRkqPF * kRkqPF;
    if (wv < kRkqNP) {
        rkq_produce<BLK>(J, wv, l, orow, nu, nsteps, wring);
        return;
    }
    const int c = wv - kRkqNP;
    const int seqb = st * (16 * NC) + 16 * c;
    const float* xr = J.X + (size_t)min(seqb + (l & 15), A.B - 1) * (size_t)J.ldx;
    // (X rows staged in LDS, as the one-chain kernel does for large grids,
    // made the channel-mix key at B = 64 slower: its chains wait on the
    // 16x16x1 issue rate, not on X.)
    float4 xw[U4];
    float4 ww[kRkqWD];
    v16f acc = {};
#pragma unroll
    for (int i = 0; i < U4; ++i) xw[i] = *reinterpret_cast<const float4*>(xr + min(4 * i, Kd - 4));
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kRkqWD; ++j) ww[j] = wring[0][j][l];
    __syncthreads();
    auto full_unit = [&](int slot, int nslot, int knext) {
#pragma unroll
        for (int i = 0; i < U4; ++i) {
            const float4 wc = ww[i % kRkqWD];
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].x, wc.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].y, wc.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].z, wc.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].w, wc.w, acc, 0, 0, 0);
            ww[i % kRkqWD] = i + kRkqWD < U4 ? wring[slot][i + kRkqWD][l] : wring[nslot][i + kRkqWD - U4][l];
            xw[i] = *reinterpret_cast<const float4*>(xr + min(knext + 4 * i, Kd - 4));
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    for (int u = 0; u < nu - 1; ++u) {
        full_unit(u % 3, (u + 1) % 3, (u + 1) * kRkqU);
        __syncthreads();
    }
    const int ul = nu - 1;
    if (!half_last) {
        full_unit(ul % 3, (ul + 1) % 3, Kd);
    } else {
#pragma unroll
        for (int i = 0; i < U4 / 2; ++i) {
            const float4 wc = ww[i % kRkqWD];
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].x, wc.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].y, wc.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].z, wc.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xw[i].w, wc.w, acc, 0, 0, 0);
        }
    }
    __syncthreads();
    for (int t = nu + 2; t < nsteps; ++t) __syncthreads();
    const int sq0 = seqb + 4 * (l >> 4), col = ot * 64 + (l & 15);
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) rkq_finish1(J, A.B, BLK, sq0 + r, col + 16 * b, acc[4 * b + r]);
}

// ---------------------------------------------------------------- heads
// One group of an INT4 row (BLK inputs; the codes in BLK / 32 chunks of 16
// bytes, scale sc) on top of acc: acc = fmaf(x[i], w[i], acc) for i in order,
// w[i] dequantized as fma(q, sc, -8 sc) (dequant_at's value). Input i is
// byte i % (BLK / 2) of the group, low nibble for the first half.
template <int BLK>
__device__ __forceinline__ float up_group(float acc, const uint4* qv, float sc, const float* x) {
    constexpr int HALF = BLK / 2;
    const float m8 = -8.0f * sc;
#pragma unroll
    for (int i = 0; i < BLK; ++i) {
        const int bi = i % HALF, ch = bi / 16, by = bi % 16;
        const uint32_t word = by < 4 ? qv[ch].x : by < 8 ? qv[ch].y : by < 12 ? qv[ch].z : qv[ch].w;
        const uint32_t bt = (word >> (8 * (by % 4))) & 0xFFu;
        const uint32_t q = i < HALF ? (bt & 0xFu) : (bt >> 4);
        acc = fmaf(x[i], fmaf((float)q, sc, m8), acc);
    }
    return acc;
}

// LoRA up-projection m of channel c for sequence b (see RkqHeadArgs): every
// code chunk is loaded first (up to 4, clamped so that no load depends on the
// rank), then the output is one sequential chain from 0 over its inputs, as
// the products compute it.
template <int BLK>
__device__ __forceinline__ float up_one(const RkqHeadArgs& A, int b, int c, int m) {
    constexpr int NQ = BLK / 32, CH = 4;   // chunks per group; chunks per matrix at most
    // rank 0 (layer 0's v2 slot, naming another matrix): one group's loads of
    // row c of that matrix, in bounds, never used
    const int Kr = A.up_k[m], K = Kr > 0 ? Kr : BLK, nch = K / 32;
    const uint4* q = reinterpret_cast<const uint4*>(A.up_q[m] + (size_t)c * (size_t)(K / 2));
    const float* sp = A.up_sc[m] + (size_t)c * (size_t)(K / BLK);
    uint4 qv[CH];
    float sc[CH / NQ];
#pragma unroll
    for (int j = 0; j < CH; ++j) qv[j] = q[min(j, nch - 1)];
#pragma unroll
    for (int g = 0; g < CH / NQ; ++g) sc[g] = sp[min(g, K / BLK - 1)];
    float acc = 0.0f;
    const float* x = A.up_x[m] + (size_t)b * (size_t)A.up_ldx;
#pragma unroll
    for (int g = 0; g < CH / NQ; ++g)
        if (g < Kr / BLK) acc = up_group<BLK>(acc, &qv[g * NQ], sc[g], x + g * BLK);
    return acc;
}

// NWV = 4 (the up-projections fused in): waves 1..3 compute them into LDS
// (wave 1: w2; wave 2: a2, then v2; wave 3: g2) while wave 0 loads its state
// row; after one workgroup barrier they end and wave 0 runs the rest alone.
// NWV = 1: one wave, the up-projections read from dw, da, g, dv.
template <int NWV>
__global__ __launch_bounds__(64 * NWV) void k_rkq_heads(RkqHeadArgs A) {
    __shared__ float w_[kHS], k_[kHS], v_[kHS], a_[kHS], kn_[kHS], r_[kHS], y_[kHS], dt_[kHS],
        sq_[kHS], part[8], stat[3];
    __shared__ float upv[NWV > 1 ? 4 : 1][kHS];
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x & 63;
    // The workgroup's syncs after the up-projections: with NWV > 1 wave 0 is
    // the only wave left, and its LDS operations complete in program order,
    // so a fence that keeps the compiler from moving them across is enough
    // (no barrier waits on the waves that have ended).
    auto sync = [] {
        if constexpr (NWV > 1) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        } else {
            __syncthreads();
        }
    };
    const size_t row = (size_t)b * A.D;
    const int c = h * kHS + t;
    if constexpr (NWV > 1) {
        const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if (wv != 0) {
            auto one = [&](int m) {
                upv[m][t] = A.up_blk == 32 ? up_one<32>(A, b, c, m) : up_one<64>(A, b, c, m);
            };
            if (wv == 1) one(0);
            else if (wv == 2) { one(1); one(3); }
            else one(2);
            __syncthreads();
            return;
        }
    }
    // Every input of the wave is loaded before any is used: the state row,
    // the channel's products and parameters, and the epilogue's.
    float* Sr = A.S + (size_t)b * A.s_bstride + (size_t)h * kHS * kHS + (size_t)t * kHS;
    float s[kHS];
#pragma unroll
    for (int q = 0; q < kHS; q += 4) {
        const float4 v4 = *reinterpret_cast<const float4*>(Sr + q);
        s[q] = v4.x; s[q + 1] = v4.y; s[q + 2] = v4.z; s[q + 3] = v4.w;
    }
    float dw, da, dv, gv;
    if constexpr (NWV > 1) {
        __syncthreads();   // the up-projections in
        dw = upv[0][t]; da = upv[1][t]; gv = upv[2][t]; dv = A.first ? 0.0f : upv[3][t];
        A.g_out[row + c] = gv;
    } else {
        dw = A.dw[row + c]; da = A.da[row + c]; gv = A.g[row + c];
        dv = A.first ? 0.0f : A.dv[row + c];
    }
    const float w0 = A.w0[c], v_in = A.v[row + c];
    const float vf = A.first ? 0.0f : A.vfirst[row + c];
    const float v0 = A.v0[c], a0 = A.a0[c], kv = A.k[row + c];
    const float kkw = A.kk_w[c], kaw = A.ka_w[c], rv = A.r[row + c], rkw = A.rk_w[c];
    const float lnw = A.lnx_w[c], lnb = A.lnx_b[c];
    // Channel terms (rwkv7.c:236-260).
    const float ww = refmath::expf(-refmath::sigmoid(dw + w0) * kR2);
    float vv = v_in;
    if (A.first) {
        A.vfirst[row + c] = vv;
    } else {
        const float mix = refmath::sigmoid(dv + v0);
        vv = vv + (vf - vv) * mix;
    }
    const float av = refmath::sigmoid(da + a0);
    const float kkv = kv * kkw;
    const float k2 = kv + kv * (av - 1.0f) * kaw;
    if (A.dbg && b == 0) {
        A.dbg[(size_t)2 * A.D + c] = k2;
        A.dbg[(size_t)3 * A.D + c] = vv;
        A.dbg[(size_t)4 * A.D + c] = av;
        A.dbg[(size_t)6 * A.D + c] = ww;
    }
    w_[t] = ww; k_[t] = k2; v_[t] = vv; a_[t] = av; kn_[t] = kkv; r_[t] = rv;
    dt_[t] = rv * k2 * rkw;
    sync();
    // |kk|: eight stride-8 partial sums of squares (rwkv7.c:156-162).
    if (t < 8) {
        float ss = 0.0f;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const float e = kn_[8 * m + t];
            ss = fmaf(e, e, ss);
        }
        part[t] = ss;
    }
    sync();
    if (t == 0) {
        float nrm = sqrtf(hsum8(part));
        if (!(nrm > 1e-12f)) nrm = 1e-12f;
        stat[0] = 1.0f / nrm;
    }
    sync();
    const float kn = kkv * stat[0];
    sync();
    kn_[t] = kn;
    sync();
    // State row t (rwkv7.c:165-187).
    float proj[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kHS; j += 8)
#pragma unroll
        for (int q = 0; q < 8; ++q) proj[q] = fmaf(s[j + q], kn_[j + q], proj[q]);
    const float pv = hsum8(proj);
    float yacc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kHS; j += 8)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float kka = kn_[j + q] * a_[j + q];
            const float vk = vv * k_[j + q];
            const float ns = fmaf(s[j + q], w_[j + q], vk - pv * kka);
            s[j + q] = ns;
            yacc[q] = fmaf(ns, r_[j + q], yacc[q]);
        }
#pragma unroll
    for (int q = 0; q < kHS; q += 4)
        *reinterpret_cast<float4*>(Sr + q) = make_float4(s[q], s[q + 1], s[q + 2], s[q + 3]);
    y_[t] = hsum8(yacc);
    sync();
    // Group norm, bonus, gate (rwkv7.c:266-288): the mean and the bonus dot
    // as sequential sums (lanes 0 and 1 side by side), then the variance.
    if (t < 2) {
        const float* src = t == 0 ? y_ : dt_;
        float acc = 0.0f;
#pragma unroll 8
        for (int i = 0; i < kHS; ++i) acc = acc + src[i];
        stat[1 + t] = acc;
    }
    sync();
    const float mean = stat[1] / (float)kHS, dot = stat[2];
    const float yy = y_[t];
    const float dd = yy - mean;
    sq_[t] = dd * dd;
    sync();
    if (t == 0) {
        float var = 0.0f;
#pragma unroll 8
        for (int i = 0; i < kHS; ++i) var = var + sq_[i];
        stat[0] = 1.0f / sqrtf(var / (float)kHS + kEpsGroup);
    }
    sync();
    const float n = (yy - mean) * stat[0] * lnw + lnb;
    A.y[row + c] = (n + dot * vv) * gv;
}

__global__ void k_refmath(const float* __restrict__ x, float* __restrict__ e, float* __restrict__ th,
                          int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        e[i] = refmath::expf(x[i]);
        th[i] = refmath::tanhf(x[i]);
    }
}

}  // namespace

snhip_status launch_rkq_ln(const RkqLnArgs& a, int B, hipStream_t st) {
    if (a.D <= 0 || a.D > kLnMax || a.D % 4 || B <= 0) return SNHIP_E_INVAL;
    hipLaunchKernelGGL(k_rkq_ln<kLnT>, dim3(B), dim3(kLnT), 0, st, a);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

snhip_status launch_rkq_heads(const RkqHeadArgs& a, int B, hipStream_t st) {
    if (a.D != a.NH * kHS || B <= 0) return SNHIP_E_INVAL;
    if (a.up_blk) {
        if ((a.up_blk != 32 && a.up_blk != 64) || !a.g_out) return SNHIP_E_INVAL;
        // every slot names a matrix the loads may read (an unused v2 slot in
        // layer 0: any of the others, rank 0, so its chain is empty)
        for (int m = 0; m < 4; ++m) {
            const int K = a.up_k[m];
            if (!a.up_q[m] || !a.up_sc[m] || !a.up_x[m] || K < 0 || K > 128 || K % a.up_blk ||
                (K == 0 && !(m == 3 && a.first)))
                return SNHIP_E_INVAL;
        }
    }
    if (a.up_blk) hipLaunchKernelGGL(k_rkq_heads<4>, dim3(a.NH, B), dim3(256), 0, st, a);
    else hipLaunchKernelGGL(k_rkq_heads<1>, dim3(a.NH, B), dim3(64), 0, st, a);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// Compute units of the current device (queried once per device).
int cu_count() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        cached[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
                          ? n
                          : 256;
    }
    return cached[dev];
}

// nc, s: INT4 consumer waves per workgroup and chains per consumer (0: chosen
// here); fp32 rows: s groups of 4 sequences per wave; tiled fp32: nc waves
// per workgroup, s groups of 4 sequences per wave.
snhip_status launch_rkq_mm_cfg(const RkqJob* jobs, int n, int B, int block, int nc, int s,
                               hipStream_t st) {
    if (n <= 0 || n > kRkqMaxJobs || B <= 0 || (block != -1 && block != 0 && block != 32 && block != 64))
        return SNHIP_E_INVAL;
    RkqMMArgs a{};
    int tiles1 = 0, kmax = 0;
    for (int i = 0; i < n; ++i) {
        const RkqJob& J = jobs[i];
        const int kq = block > 0 ? block : 4;
        if (J.M <= 0 || J.Kd <= 0 || J.Kd % kq || J.ldx % 4 || !J.X || !J.Y ||
            (block > 0 ? (!J.q || !J.sc || J.Kd % 32) : !J.w))
            return SNHIP_E_INVAL;
        a.j[i] = J;
        a.tiles_out[i] = (J.M + 63) / 64;
        tiles1 += a.tiles_out[i];
        kmax = std::max(kmax, J.Kd);
    }
    int per;   // sequences per workgroup
    int S = 1, NC = 1;
    bool xl = false;   // INT4: four one-chain consumers per workgroup, X staged in LDS
    size_t shm = 0;
    int NW = 1;   // tiled fp32: waves per workgroup
    bool wdeep = true;   // tiled fp32: the deeper weight stream (at most one wave per CU)
    if (block < 0) {
        // One chain per wave; the waves of one output tile's sequence tiles
        // in workgroups of NW (one per SIMD) once there are more waves than
        // CUs; more than four per CU: two chains per wave, and so on.
        const long cus = cu_count();
        auto waves = [&](int s_) { return (long)tiles1 * ((B + 4 * s_ - 1) / (4 * s_)); };
        // SNHIP_RKQ_W4_SHAPE=S,NW (tuning): that shape wherever it fits
        if (!s && !nc)
            if (const char* e = getenv("SNHIP_RKQ_W4_SHAPE")) {
                int s_ = 0, n_ = 0;
                if (sscanf(e, "%d,%d", &s_, &n_) == 2 && (s_ == 1 || s_ == 2 || s_ == 4) &&
                    (n_ == 1 || n_ == 2 || n_ == 4) && s_ * kmax <= kRkwXMax &&
                    (size_t)n_ * ((s_ * kmax + 63) / 64 * 64 + kRkwXA * 4 * s_ + 16) * sizeof(float4) <= 65536) {
                    s = s_;
                    nc = n_;
                }
            }
        S = 1;
        if (s) S = s;
        else
            while (S < 4 && waves(S) > 4 * cus) S *= 2;
        while (!s && S > 1 && S * kmax > kRkwXMax) S /= 2;
        if ((S != 1 && S != 2 && S != 4) || S * kmax > kRkwXMax) return SNHIP_E_INVAL;
        // One wave per workgroup (grouping an output tile's waves 2 or 4 per
        // workgroup measured 2 % slower at B = 64 once the stream depth
        // follows the waves per CU); NW only when forced.
        NW = nc ? nc : 1;
        wdeep = waves(S) <= cus;
        // per wave: X (S Kd float4, rounded up to the staging's 64) and the
        // read-ahead past the last block; at most 64 KiB per workgroup
        a.xs_per_wave = (S * kmax + 63) / 64 * 64 + kRkwXA * 4 * S + 16;   // + the prefetch's dump slot
        while (!nc && NW > 1 && (size_t)NW * a.xs_per_wave * sizeof(float4) > 65536) NW /= 2;
        shm = (size_t)NW * a.xs_per_wave * sizeof(float4);
        if ((NW != 1 && NW != 2 && NW != 4) || shm > 65536) return SNHIP_E_INVAL;
        per = 4 * S;
    } else if (block == 0) {
        const long waves1 = (long)tiles1 * ((B + 3) / 4);
        S = s ? s : (B > 8 && waves1 / 4 >= 1024) ? 4 : (B > 4 && waves1 / 2 >= 1024) ? 2 : 1;
        if (S != 1 && S != 2 && S != 4) return SNHIP_E_INVAL;
        per = 4 * S;
    } else {
        // Measured on MI355X (K = 768 / 3072 products, B = 1 / 8 / 64): one
        // consumer of one chain is fastest while the grid of such workgroups
        // stays within ~1024 (up to 3 reside per CU); larger grids (the
        // vocabulary head) share the dequantized units among more chains.
        // S = 16 selects the wide kernel (one 16x16x1 chain of 16 sequences
        // per consumer), used from B = 8 once the one-chain grid exceeds 256
        // workgroups (SNHIP_RKQ_WIDE_GRID): the products are then bound by
        // matrix-core throughput, not chain latency. NC then keeps the grid at
        // >= ~512 workgroups. Measured on the RWKV-7 step (B = 64): head
        // 376 -> 112 us, channel-mix key 26 -> 21 us.
        const long wg11 = (long)tiles1 * ((B + 3) / 4);
        int nc0 = wg11 <= 1024 ? 1 : 2, s0 = wg11 <= 1024 || B < 16 ? 1 : 2;
        // Not for launches with a tanh / sigmoid epilogue (a wide lane finishes
        // 16 outputs, not 4) or with a short K (fill-bound).
        bool wide_ok = true;
        for (int i = 0; i < n; ++i)
            wide_ok = wide_ok && jobs[i].Kd >= 256 && jobs[i].epi != RKQ_TANH && jobs[i].epi != RKQ_SIGMOID;
        if (wide_ok && B >= 8 && wg11 > (long)env_unsigned("SNHIP_RKQ_WIDE_GRID", 256, 0)) {
            s0 = 16;
            nc0 = B > 32 ? 4 : B > 16 ? 2 : 1;   // chains of 16 per workgroup: 1, 2 or 4 (instantiated)
            while (nc0 > 1 && (long)tiles1 * ((B + 16 * nc0 - 1) / (16 * nc0)) < 512) nc0 /= 2;
        }
        NC = nc ? nc : nc0;
        S = s ? s : s0;
        if (!((NC == 1 || NC == 2 || NC == 4) && (S == 1 || S == 2 || S == 16)) || (NC == 4 && S == 2))
            return SNHIP_E_INVAL;
        // One-chain launches of more than one workgroup per CU instead run
        // one workgroup of four consumers per 16 sequences with their X rows
        // staged in LDS once (each consumer lane otherwise loads its X from
        // global memory one unit ahead, and at three workgroups per CU those
        // loads' latency held the chains back). Measured on the RWKV-7 step
        // at B = 64 (r, k, v and the LoRA downs, 656 -> 164 workgroups):
        // 31.3 -> 21.9 us; the LoRA ups 7.3 -> 6.5. Staging the rows of
        // smaller grids (one workgroup of one consumer per CU) was slower
        // (B = 8 step 1384 -> 1504 us).
        if (!nc && !s && NC == 1 && S == 1 && B >= 16 && wg11 > (long)cu_count() &&
            env_unsigned("SNHIP_RKQ_XL", 1, 0)) {
            bool fits = true;
            for (int i = 0; i < n; ++i) fits = fits && jobs[i].Kd <= kRkqXLF / 16;
            if (fits) {
                NC = 4;
                xl = true;
            }
        }
        per = (S == 16 ? 16 : 4 * S) * NC;
    }
    a.n = n;
    a.B = B;
    a.seq_tiles = (B + per - 1) / per;
    int total = 0;
    for (int i = 0; i < n; ++i) {
        a.start[i] = total;
        total += a.tiles_out[i] * ((a.seq_tiles + NW - 1) / NW);
    }
    a.start[n] = total;
    for (int i = n + 1; i <= kRkqMaxJobs; ++i) a.start[i] = total;
    // Measured on the RWKV-7 step at B = 64: X two units ahead takes W_o and
    // the channel-mix value (192 workgroups) 1.5 us faster each, and makes
    // the 656- and 768-workgroup launches 1.9 us slower.
    const bool deep = total <= cu_count();
#define SNHIP_RKQ_F32(S_) hipLaunchKernelGGL((k_rkq_mm_f32<S_>), dim3(total), dim3(64), 0, st, a)
#define SNHIP_RKQ_Q4(B_, N_, S_) \
    hipLaunchKernelGGL((k_rkq_mm_q4<B_, N_, S_, 1>), dim3(total), dim3(64 * (N_ + kRkqNP)), 0, st, a)
#define SNHIP_RKQ_Q4D(B_) \
    hipLaunchKernelGGL((k_rkq_mm_q4<B_, 1, 1, 2>), dim3(total), dim3(64 * (1 + kRkqNP)), 0, st, a)
#define SNHIP_RKQ_Q4L(B_, N_) \
    hipLaunchKernelGGL((k_rkq_mm_q4<B_, N_, 1, 0>), dim3(total), dim3(64 * (N_ + kRkqNP)), 0, st, a)
#define SNHIP_RKQ_Q4W(B_, N_) \
    hipLaunchKernelGGL((k_rkq_mm_q4w<B_, N_>), dim3(total), dim3(64 * (N_ + kRkqNP)), 0, st, a)
#define SNHIP_RKQ_Q4B(B_)                                 \
    do {                                                  \
        if (S == 16) {                                    \
            if (NC == 1) SNHIP_RKQ_Q4W(B_, 1);            \
            else if (NC == 2) SNHIP_RKQ_Q4W(B_, 2);       \
            else SNHIP_RKQ_Q4W(B_, 4);                    \
        } else if (xl) SNHIP_RKQ_Q4L(B_, 4);             \
        else if (NC == 1 && S == 1 && deep) SNHIP_RKQ_Q4D(B_); \
        else if (NC == 1 && S == 1) SNHIP_RKQ_Q4(B_, 1, 1); \
        else if (NC == 2 && S == 1) SNHIP_RKQ_Q4(B_, 2, 1); \
        else if (NC == 4) SNHIP_RKQ_Q4(B_, 4, 1);        \
        else if (NC == 1) SNHIP_RKQ_Q4(B_, 1, 2);        \
        else SNHIP_RKQ_Q4(B_, 2, 2);                     \
    } while (0)
    if (block < 0) {
#define SNHIP_RKW(S_, N_, P_) \
    hipLaunchKernelGGL((k_rkq_mm_w4<S_, N_, P_>), dim3(total), dim3(64 * N_), shm, st, a)
        if (S == 1) {
            if (NW == 1) {
                if (wdeep) SNHIP_RKW(1, 1, 48);
                else SNHIP_RKW(1, 1, 16);
            } else if (NW == 2) {
                SNHIP_RKW(1, 2, 40);
            } else {
                SNHIP_RKW(1, 4, 24);
            }
        } else if (S == 2) {
            if (NW == 1) SNHIP_RKW(2, 1, 40);
            else if (NW == 2) SNHIP_RKW(2, 2, 40);
            else SNHIP_RKW(2, 4, 40);
        } else {
            if (NW == 1) SNHIP_RKW(4, 1, 24);
            else if (NW == 2) SNHIP_RKW(4, 2, 24);
            else SNHIP_RKW(4, 4, 24);
        }
#undef SNHIP_RKW
    } else if (block == 0) {
        if (S == 1) SNHIP_RKQ_F32(1);
        else if (S == 2) SNHIP_RKQ_F32(2);
        else SNHIP_RKQ_F32(4);
    } else if (block == 32) {
        SNHIP_RKQ_Q4B(32);
    } else {
        SNHIP_RKQ_Q4B(64);
    }
#undef SNHIP_RKQ_F32
#undef SNHIP_RKQ_Q4
#undef SNHIP_RKQ_Q4D
#undef SNHIP_RKQ_Q4L
#undef SNHIP_RKQ_Q4B
#undef SNHIP_RKQ_Q4W
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

snhip_status launch_rkq_mm(const RkqJob* jobs, int n, int B, int block, hipStream_t st) {
    return launch_rkq_mm_cfg(jobs, n, B, block, 0, 0, st);
}

size_t rkq_tiled_floats(int M, int Kd) {
    return ((size_t)((M + 63) / 64) * (size_t)(Kd / 4) * 64 + kRkwPad) * 4;
}

snhip_status launch_rkq_block4(const float* w, const uint8_t* q, const float* sc, int block, int M, int Kd,
                               float* out, hipStream_t st) {
    if (M <= 0 || Kd <= 0 || Kd % 4 || !out || (block != 0 && block != 32 && block != 64) ||
        (block ? (!q || !sc || Kd % block) : !w))
        return SNHIP_E_INVAL;
    RkqJob J{};
    J.w = w; J.q = q; J.sc = sc; J.M = M; J.Kd = Kd;
    const size_t n = rkq_tiled_floats(M, Kd) / 4;
    hipLaunchKernelGGL(k_rkq_block4, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, J, block,
                       reinterpret_cast<float4*>(out));
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

}  // namespace snhip

extern "C" {

snhip_status snhip_refmath_host(const float* x, float* e, float* t, int32_t n) {
    if (!x || !e || !t || n <= 0) return SNHIP_E_INVAL;
    for (int32_t i = 0; i < n; ++i) {
        e[i] = snhip::refmath::expf(x[i]);
        t[i] = snhip::refmath::tanhf(x[i]);
    }
    return SNHIP_OK;
}

snhip_status snhip_refmath_dev(const float* x, float* e, float* t, int32_t n, void* stream) {
    if (!x || !e || !t || n <= 0) return SNHIP_E_INVAL;
    hipLaunchKernelGGL(snhip::k_refmath, dim3((n + 255) / 256), dim3(256), 0,
                       snhip::as_stream(stream), x, e, t, n);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

}  // extern "C"
