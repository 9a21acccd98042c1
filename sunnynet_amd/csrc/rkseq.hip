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
#include <cstring>

#include "refmath.h"
#include "rkseq.h"
#include "snhip_rwkv7.h"

namespace snhip {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr float kR2 = 0.6065306597126334f;   // 1/sqrt(e), rwkv7.c:38
constexpr float kEpsGroup = 6.4e-4f;          // rwkv7.c:39
constexpr int kHS = 64;
constexpr int kLnMax = 4096;

__device__ __forceinline__ float hsum8(const float* v) {
    const float c0 = v[0] + v[4], c1 = v[1] + v[5], c2 = v[2] + v[6], c3 = v[3] + v[7];
    return (c0 + c1) + (c2 + c3);
}

// ------------------------------------------------------------------ rows
// Sequential fp32 sum of n4 float4 in LDS (element order), by one lane. Rows
// whose length is a multiple of 64 take blocks of 64 values with the next
// block's reads in flight while the current block is added; only the chain
// of dependent adds is exposed.
__device__ __forceinline__ float seq_sum(const float4* v, int n4) {
    float s = 0.0f;
    if (n4 % 16 == 0) {
        float4 cur[16], nxt[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) cur[i] = v[i];
        for (int base = 0; base < n4; base += 16) {
            if (base + 16 < n4) {
#pragma unroll
                for (int i = 0; i < 16; ++i) nxt[i] = v[base + 16 + i];
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s = s + cur[i].x; s = s + cur[i].y; s = s + cur[i].z; s = s + cur[i].w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) cur[i] = nxt[i];
        }
        return s;
    }
    for (int i = 0; i < n4; ++i) {
        const float4 b = v[i];
        s = s + b.x; s = s + b.y; s = s + b.z; s = s + b.w;
    }
    return s;
}

// Row LayerNorm of rows up to kLnMax (= 64 lanes x kLnQ float4): lane t owns
// float4 q = t + 64 j of the row (elements 4q .. 4q+3); its row, gain, bias,
// shift and mix values are loaded as float4 before the sums, so the only
// exposed latencies are one round trip and the two sequential sums.
constexpr int kLnQ = 3;                    // float4 per lane with everything in registers (rows <= 768)

__global__ __launch_bounds__(64) void k_rkq_ln(RkqLnArgs A) {
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
    const bool regs = n4 <= 64 * kLnQ;
    const bool mix1 = A.mode == RKQ_LN_MIX1, mix2 = A.mode == RKQ_LN_MIX2;
    float4 xv[kLnQ], gv[kLnQ], cv[kLnQ], sv[kLnQ], lv[6][kLnQ];
    for (int q = t; q < n4; q += 64) {
        float4 v = src[q];
        if (!ok) v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
        xs4[q] = v;
    }
    if (regs) {
#pragma unroll
        for (int j = 0; j < kLnQ; ++j) {
            const int q = min(t + 64 * j, n4 - 1);
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
    if (t == 0) stat[0] = seq_sum(xs4, n4) / (float)D;   // sum = sum + x[i], in order
    __syncthreads();
    const float mean = stat[0];
    for (int q = t; q < n4; q += 64) {
        const float4 v = xs4[q];
        float4 d;
        d.x = v.x - mean; d.y = v.y - mean; d.z = v.z - mean; d.w = v.w - mean;
        d.x = d.x * d.x; d.y = d.y * d.y; d.z = d.z * d.z; d.w = d.w * d.w;
        sq4[q] = d;
    }
    __syncthreads();
    if (t == 0)                         // vsum = vsum + d * d, in order
        stat[1] = 1.0f / sqrtf(seq_sum(sq4, n4) / (float)D + A.eps);
    __syncthreads();
    const float rstd = stat[1];
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
            const int q = t + 64 * j;
            if (q < n4) {
                const float4 lp[6] = {lv[0][j], lv[1][j], lv[2][j], lv[3][j], lv[4][j], lv[5][j]};
                emit(q, gv[j], cv[j], sv[j], lp);
            }
        }
    } else {
        for (int q = t; q < n4; q += 64) {   // longer rows: parameters loaded as used
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
};

__device__ __forceinline__ float dequant_at(const RkqJob& J, int row, int k, int blk) {
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

// Inputs per chunk staged in LDS at once (X rows; INT4 codes in registers).
constexpr int kRkqKC = 768;
constexpr int kRkqU = 64;                  // inputs per pipeline unit (two producer halves of 32)
constexpr int kRkqNP = 2;                  // producer waves of an INT4 workgroup

// This workgroup's job (uniform selects: no dynamic index into the arguments).
__device__ __forceinline__ void rkq_job(const RkqMMArgs& A, RkqJob& J, int& u0) {
    int ji = 0;
#pragma unroll
    for (int i = 1; i < kRkqMaxJobs; ++i)
        if (i < A.n && (int)blockIdx.x >= A.start[i]) ji = i;
    J = A.j[0];
    int j0 = A.start[0];
#pragma unroll
    for (int i = 1; i < kRkqMaxJobs; ++i)
        if (i == ji) { J = A.j[i]; j0 = A.start[i]; }
    u0 = (int)blockIdx.x - j0;
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

// INT4 weights: a workgroup of 1 + NC waves (one per SIMD) per 64 rows x
// 4 NC sequences. Wave 0 (producer) holds the rows' codes and scales of the
// chunk in registers and dequantizes one unit of 32 inputs per step into a
// three-slot LDS ring ([k/4][row] float4, conflict-free). Consumer wave c runs
// the k-ordered MFMA chains of sequences 4c .. 4c+3. Step t ends with one
// workgroup barrier: the producer writes unit t; a consumer reads unit t-1
// into registers (alternating between two register sets) and multiplies unit
// t-2 from the other set, so its MFMA chain never waits on LDS or on VALU work
// of its own. Every weight is dequantized once per workgroup.
template <int BLK, int NC>
__global__ __launch_bounds__(64 * (NC + kRkqNP)) void k_rkq_mm_q4(const RkqMMArgs A) {
    constexpr int U4 = kRkqU / 4;
    __shared__ float4 xs4[NC][4][kRkqKC / 4];          // consumer c's X rows
    __shared__ float4 wring[2][U4][64];                // dequantized units
    __shared__ uint4 cq[kRkqKC / 32][64];              // producer: codes, [16-byte slot][row]
    __shared__ float cs[kRkqKC / BLK][64];             // producer: scales, [group][row]
    RkqJob J;
    int u0;
    rkq_job(A, J, u0);
    const int ot = u0 / A.seq_tiles, st = u0 % A.seq_tiles;
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63, r4 = l & 3;
    const int out = ot * 64 + l;
    const int orow = out < J.M ? out : J.M - 1;
    const int cw_ = wv - kRkqNP;                      // consumer index (< 0: producer)
    const int seqw = st * 4 * NC + 4 * cw_;            // consumer's first sequence
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < J.Kd; k0 += kRkqKC) {
        const int kc = min(kRkqKC, J.Kd - k0);
        const int nu = (kc + kRkqU - 1) / kRkqU;
        __syncthreads();
        if (cw_ >= 0) {
            // Consumer: stage its 4 X rows of the chunk (zero rows past the batch).
            const int nq = kc / 4;
            for (int idx = l; idx < 4 * nq; idx += 64) {
                const int row = idx / nq, q = idx - row * nq;
                const int sq = seqw + row;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (sq < A.B) v = *reinterpret_cast<const float4*>(J.X + (size_t)sq * J.ldx + k0 + 4 * q);
                xs4[cw_][row][q] = v;
            }
            __syncthreads();
            const float4* xl = xs4[cw_][r4];
            for (int t = 0; t < nu + 1; ++t) {
                if (t >= 1) {
                    const int u = t - 1;
                    const int n4 = min(U4, (kc - u * kRkqU) / 4);   // a last unit may be half
                    float4 w[U4], x[U4];
                    if (n4 == U4) {
#pragma unroll
                        for (int i = 0; i < U4; ++i) {
                            w[i] = wring[u & 1][i][l];
                            x[i] = xl[u * U4 + i];
                        }
#pragma unroll
                        for (int i = 0; i < U4; ++i) {
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(x[i].x, w[i].x, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(x[i].y, w[i].y, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(x[i].z, w[i].z, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(x[i].w, w[i].w, acc, 0, 0, 0);
                        }
                    } else {
                        for (int i = 0; i < n4; ++i) {
                            const float4 wi = wring[u & 1][i][l], xi = xl[u * U4 + i];
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(xi.x, wi.x, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(xi.y, wi.y, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(xi.z, wi.z, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_4x4x1f32(xi.w, wi.w, acc, 0, 0, 0);
                        }
                    }
                }
                __syncthreads();
            }
        } else {
            // Producer: stage row orow's codes and scales of the chunk in LDS
            // (every load in flight at once; the lane reads back only its own),
            // then dequantize unit t at step t from there.
            const int ng = kc / BLK;
            const uint4* qr = reinterpret_cast<const uint4*>(J.q + (size_t)orow * (J.Kd / 2) + k0 / 2);
            const float* sr = J.sc + (size_t)orow * (J.Kd / BLK) + k0 / BLK;
            // (both producers stage every slot; each reads back its own lane's)
            for (int i = 0; i < kc / 32; ++i) cq[i][l] = qr[i];
            for (int g = 0; g < ng; ++g) cs[g][l] = sr[g];
            __syncthreads();
            // Unit t: inputs 64 t .. 64 t + 63 of the chunk, from the 16-byte
            // code slots 4 t .. 4 t + 3 (element e of a group is byte
            // e % (BLK/2), low nibble for e < BLK/2).
            for (int t = 0; t < nu + 1; ++t) {
                if (t < nu) {
                    if (t * kRkqU + 32 * wv < kc) {            // this producer's 32-input half
                        const int h = wv;
                        const int k = t * kRkqU + 32 * h;
                        const int g = k / BLK;
                        const float scg = cs[g][l], m8 = -8.0f * scg;
                        uint32_t cw[BLK / 8];
#pragma unroll
                        for (int i = 0; i < BLK / 32; ++i) {
                            const uint4 v = cq[g * (BLK / 32) + i][l];
                            cw[4 * i] = v.x; cw[4 * i + 1] = v.y; cw[4 * i + 2] = v.z; cw[4 * i + 3] = v.w;
                        }
                        const int e0 = k % BLK;
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const int e = e0 + 4 * i;
                            const int by = e % (BLK / 2);
                            const uint32_t word = cw[by / 4];
                            uint32_t nib = (e >= BLK / 2 ? (word >> 4) : word) & 0x0F0F0F0Fu;
                            // Opaque to the compiler, so that each byte converts
                            // with one v_cvt_f32_ubyteN (no field extraction).
                            asm volatile("" : "+v"(nib));
                            float4 w;
                            w.x = fmaf((float)(nib & 0xFFu), scg, m8);
                            w.y = fmaf((float)((nib >> 8) & 0xFFu), scg, m8);
                            w.z = fmaf((float)((nib >> 16) & 0xFFu), scg, m8);
                            w.w = fmaf((float)(nib >> 24), scg, m8);
                            wring[t & 1][8 * h + i][l] = w;
                        }
                    }
                }
                __syncthreads();
            }
        }
    }
    if (cw_ >= 0) rkq_finish(J, A.B, BLK, seqw, out, acc);
}

// ---------------------------------------------------------------- heads
__global__ __launch_bounds__(64) void k_rkq_heads(RkqHeadArgs A) {
    __shared__ float w_[kHS], k_[kHS], v_[kHS], a_[kHS], kn_[kHS], r_[kHS], y_[kHS], dt_[kHS],
        sq_[kHS], part[8], stat[3];
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const size_t row = (size_t)b * A.D;
    const int c = h * kHS + t;
    // Every input of the wave is loaded before any is used: the state row,
    // the channel's products and parameters, and the epilogue's.
    float* Sr = A.S + (size_t)b * A.s_bstride + (size_t)h * kHS * kHS + (size_t)t * kHS;
    float s[kHS];
#pragma unroll
    for (int q = 0; q < kHS; q += 4) {
        const float4 v4 = *reinterpret_cast<const float4*>(Sr + q);
        s[q] = v4.x; s[q + 1] = v4.y; s[q + 2] = v4.z; s[q + 3] = v4.w;
    }
    const float dw = A.dw[row + c], w0 = A.w0[c], v_in = A.v[row + c];
    const float vf = A.first ? 0.0f : A.vfirst[row + c];
    const float dv = A.first ? 0.0f : A.dv[row + c];
    const float v0 = A.v0[c], da = A.da[row + c], a0 = A.a0[c], kv = A.k[row + c];
    const float kkw = A.kk_w[c], kaw = A.ka_w[c], rv = A.r[row + c], rkw = A.rk_w[c];
    const float lnw = A.lnx_w[c], lnb = A.lnx_b[c], gv = A.g[row + c];
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
    w_[t] = ww; k_[t] = k2; v_[t] = vv; a_[t] = av; kn_[t] = kkv; r_[t] = rv;
    dt_[t] = rv * k2 * rkw;
    __syncthreads();
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
    __syncthreads();
    if (t == 0) {
        float nrm = sqrtf(hsum8(part));
        if (!(nrm > 1e-12f)) nrm = 1e-12f;
        stat[0] = 1.0f / nrm;
    }
    __syncthreads();
    const float kn = kkv * stat[0];
    __syncthreads();
    kn_[t] = kn;
    __syncthreads();
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
    __syncthreads();
    // Group norm, bonus, gate (rwkv7.c:266-288): the mean and the bonus dot
    // as sequential sums (lanes 0 and 1 side by side), then the variance.
    if (t < 2) {
        const float* src = t == 0 ? y_ : dt_;
        float acc = 0.0f;
#pragma unroll 8
        for (int i = 0; i < kHS; ++i) acc = acc + src[i];
        stat[1 + t] = acc;
    }
    __syncthreads();
    const float mean = stat[1] / (float)kHS, dot = stat[2];
    const float yy = y_[t];
    const float dd = yy - mean;
    sq_[t] = dd * dd;
    __syncthreads();
    if (t == 0) {
        float var = 0.0f;
#pragma unroll 8
        for (int i = 0; i < kHS; ++i) var = var + sq_[i];
        stat[0] = 1.0f / sqrtf(var / (float)kHS + kEpsGroup);
    }
    __syncthreads();
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
    hipLaunchKernelGGL(k_rkq_ln, dim3(B), dim3(64), 0, st, a);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

snhip_status launch_rkq_heads(const RkqHeadArgs& a, int B, hipStream_t st) {
    if (a.D != a.NH * kHS || B <= 0) return SNHIP_E_INVAL;
    hipLaunchKernelGGL(k_rkq_heads, dim3(a.NH, B), dim3(64), 0, st, a);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

snhip_status launch_rkq_mm(const RkqJob* jobs, int n, int B, int block, hipStream_t st) {
    if (n <= 0 || n > kRkqMaxJobs || B <= 0 || (block != 0 && block != 32 && block != 64))
        return SNHIP_E_INVAL;
    RkqMMArgs a{};
    int tiles1 = 0;
    for (int i = 0; i < n; ++i) {
        const RkqJob& J = jobs[i];
        const int kq = block ? block : 4;
        if (J.M <= 0 || J.Kd <= 0 || J.Kd % kq || J.ldx % 4 || !J.X || !J.Y ||
            (block ? (!J.q || !J.sc || J.Kd % 32) : !J.w))
            return SNHIP_E_INVAL;
        a.j[i] = J;
        a.tiles_out[i] = (J.M + 63) / 64;
        tiles1 += a.tiles_out[i];
    }
    // fp32: groups of 4 sequences per wave (S); INT4: consumer waves per
    // workgroup (NC), 4 sequences each.
    int per;   // sequences per workgroup
    int S = 1, NC = 1;
    if (block == 0) {
        const long waves1 = (long)tiles1 * ((B + 3) / 4);
        S = (B > 8 && waves1 / 4 >= 1024) ? 4 : (B > 4 && waves1 / 2 >= 1024) ? 2 : 1;
        per = 4 * S;
    } else {
        // One wave per SIMD: two producers and one or two consumers.
        NC = B <= 4 ? 1 : 2;
        per = 4 * NC;
    }
    a.n = n;
    a.B = B;
    a.seq_tiles = (B + per - 1) / per;
    int total = 0;
    for (int i = 0; i < n; ++i) {
        a.start[i] = total;
        total += a.tiles_out[i] * a.seq_tiles;
    }
    a.start[n] = total;
    for (int i = n + 1; i <= kRkqMaxJobs; ++i) a.start[i] = total;
#define SNHIP_RKQ_F32(S_) hipLaunchKernelGGL((k_rkq_mm_f32<S_>), dim3(total), dim3(64), 0, st, a)
#define SNHIP_RKQ_Q4(B_, N_) hipLaunchKernelGGL((k_rkq_mm_q4<B_, N_>), dim3(total), dim3(64 * (N_ + kRkqNP)), 0, st, a)
    if (block == 0) {
        if (S == 1) SNHIP_RKQ_F32(1);
        else if (S == 2) SNHIP_RKQ_F32(2);
        else SNHIP_RKQ_F32(4);
    } else if (block == 32) {
        if (NC == 1) SNHIP_RKQ_Q4(32, 1);
        else SNHIP_RKQ_Q4(32, 2);
    } else {
        if (NC == 1) SNHIP_RKQ_Q4(64, 1);
        else SNHIP_RKQ_Q4(64, 2);
    }
#undef SNHIP_RKQ_F32
#undef SNHIP_RKQ_Q4
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
