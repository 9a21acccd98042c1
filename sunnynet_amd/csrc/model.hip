// SunnyNet whole-model decode on gfx950 (include/snhip.h).
//
// The math is the reference's decode step, sunnynet/runtime/sunnynet.c:212-334
// (= SunnyNet.forward_step, sunnynet/model.py:113-124, sunnynet/layers.py:287-326):
//   raw = LN(x); at = raw + conv(raw, hist); v = V at; q = U v
//   u = u_raw * sig(g_i - g_{i+1}) * sig(g_i - g_{i+2})   (groups of 8)
//   p = 1 - delta (1 - sig(g)); sfb = W_eff s; s' = p s + (1 - p) u
//   z = W_z u; y = LN_I(z (1 + a/2 / (1 + |z|))); out = W_c y + b s' + sfb + x
//   logits = E LN(x_L)
//
// One step is a short sequence of kernels on the handle's stream; every
// kernel processes all B sequences. Weights live row-major (out, in) in HBM,
// fp32 or INT4 (quant.c's packing, dequantized in registers and bit-identical
// to sn_dequant_i4). Elementwise work keeps the reference's operation order;
// the GEMV reductions use a parallel (wavefront) order, so logits agree with
// the reference to float rounding, not bit for bit.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include <hip/hip_fp16.h>

#include "common.h"
#include "decode.h"
#include "gemm.h"
#include "gemv.h"
#include "snhip.h"

namespace snhip {
namespace {

constexpr int kMagic = 0x4E4E5355;   // "USNN", sunnynet.c:33
constexpr int kMaxTaps = 8;

// ------------------------------------------------------------------ device
__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum within aligned segments of `seg` lanes (seg a power of two <= 64).
__device__ __forceinline__ float seg_sum(float v, int seg) {
    for (int o = seg >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// 256-thread block sum (4 waves); `red` holds 4 floats of LDS.
__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Largest LayerNorm row: 16 values per thread of a 256-thread block.
constexpr int kLnPer = 16;
// Prefill: up to this many channels (max_batch x dim) the gates are computed
// for every row in parallel and the scan only multiplies and adds
// (k_gate_rows + k_scan_rows); above it k_core_scan fuses them.
constexpr size_t kSplitScanChannels = 16384;

__global__ void k_round_f16(float* __restrict__ x, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = __half2float(__float2half_rn(x[i]));
}

__global__ void k_embed(const int32_t* __restrict__ tok, const float* __restrict__ embed,
                        float* __restrict__ x, int D, int vocab) {
    const int b = blockIdx.x;
    const int t = tok[b];
    const bool ok = t >= 0 && t < vocab;
    for (int i = threadIdx.x; i < D; i += blockDim.x)
        x[(size_t)b * D + i] = ok ? embed[(size_t)t * D + i] : __builtin_nanf("");
}

// Two-pass LayerNorm statistics (sunnynet.c:198-210 form) over n values held
// in registers, PER per thread of a 256-thread block (element k*256+tid).
template <int PER>
__device__ __forceinline__ void ln_stats_t(const float (&xv)[PER], int n, float eps, float* red,
                                           float& mean, float& rstd) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (k * 256 + (int)threadIdx.x < n) sum += xv[k];
    mean = block_sum256(sum, red) / (float)n;
    float vs = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (k * 256 + (int)threadIdx.x < n) {
            const float d = xv[k] - mean;
            vs += d * d;
        }
    rstd = 1.0f / sqrtf(block_sum256(vs, red) / (float)n + eps);
}

// raw = LN(x); at = raw + conv(raw, hist); hist <- [raw, hist[0..K-3]] in place.
// One block per sequence; conv order as sunnynet.c:227-237. Every load (x,
// gains, taps, history) is issued before the statistics are reduced.
template <int PER>
__global__ __launch_bounds__(256) void k_ln_conv(
        const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ c,
        const float* __restrict__ dw, float* __restrict__ hist, size_t hist_bstride,
        float* __restrict__ at, int D, int K, float eps) {
    __shared__ float red[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float* xb = x + (size_t)b * D;
    float* hb = hist + (size_t)b * hist_bstride;
    float xv[PER], gv[PER], cv[PER], h[kMaxTaps - 1][PER], dv[kMaxTaps][PER];
#pragma unroll
    for (int kk = 0; kk < PER; ++kk) {
        const int i = min(kk * 256 + tid, D - 1);   // lanes past D load a valid element
        xv[kk] = xb[i];
        gv[kk] = g[i];
        cv[kk] = c[i];
#pragma unroll
        for (int t = 0; t < kMaxTaps - 1; ++t) h[t][kk] = t < K - 1 ? hb[(size_t)t * D + i] : 0.0f;
#pragma unroll
        for (int t = 0; t < kMaxTaps; ++t) dv[t][kk] = t < K ? dw[(size_t)t * D + i] : 0.0f;
    }
    float mean, rstd;
    ln_stats_t<PER>(xv, D, eps, red, mean, rstd);
#pragma unroll
    for (int kk = 0; kk < PER; ++kk) {
        const int i = kk * 256 + tid;
        if (i >= D) continue;
        const float raw = (xv[kk] - mean) * rstd * gv[kk] + cv[kk];
        if (K > 1) {
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < kMaxTaps; ++t)
                if (t == K - 1) acc = raw * dv[t][kk];
#pragma unroll
            for (int t = 0; t < kMaxTaps - 1; ++t)
                if (t < K - 1) {
#pragma unroll
                    for (int u = 0; u < kMaxTaps; ++u)
                        if (u == K - 2 - t) acc = acc + h[t][kk] * dv[u][kk];
                }
            at[(size_t)b * D + i] = raw + acc;
#pragma unroll
            for (int t = kMaxTaps - 2; t >= 1; --t)
                if (t <= K - 2) hb[(size_t)t * D + i] = h[t - 1][kk];
            hb[i] = raw;
        } else {
            at[(size_t)b * D + i] = raw;
        }
    }
}

// y = LN(x) per sequence (norm_mix and norm_out); loads issued up front.
template <int PER>
__global__ __launch_bounds__(256) void k_ln(const float* __restrict__ x, int ldx,
                                            const float* __restrict__ g,
                                            const float* __restrict__ c, float* __restrict__ y,
                                            int ldy, int n, float eps) {
    __shared__ float red[4];
    const int b = blockIdx.x, tid = threadIdx.x;
    float xv[PER], gv[PER], cv[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = min(k * 256 + tid, n - 1);
        xv[k] = x[(size_t)b * ldx + i];
        gv[k] = g[i];
        cv[k] = c[i];
    }
    float mean, rstd;
    ln_stats_t<PER>(xv, n, eps, red, mean, rstd);
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = k * 256 + tid;
        if (i < n) y[(size_t)b * ldy + i] = (xv[k] - mean) * rstd * gv[k] + cv[k];
    }
}

// Per-thread element count for a row of n (<= 4096) values.
int ln_per(int n) {
    const int p = (n + 255) / 256;
    return p <= 1 ? 1 : p <= 2 ? 2 : p <= 4 ? 4 : p <= 6 ? 6 : p <= 8 ? 8 : 16;
}

void launch_ln(int rows, const float* x, int ldx, const float* g, const float* c, float* y,
               int ldy, int n, float eps, hipStream_t st) {
    const dim3 grid((unsigned)rows), blk(256);
    switch (ln_per(n)) {
    case 1: hipLaunchKernelGGL(k_ln<1>, grid, blk, 0, st, x, ldx, g, c, y, ldy, n, eps); break;
    case 2: hipLaunchKernelGGL(k_ln<2>, grid, blk, 0, st, x, ldx, g, c, y, ldy, n, eps); break;
    case 4: hipLaunchKernelGGL(k_ln<4>, grid, blk, 0, st, x, ldx, g, c, y, ldy, n, eps); break;
    case 6: hipLaunchKernelGGL(k_ln<6>, grid, blk, 0, st, x, ldx, g, c, y, ldy, n, eps); break;
    case 8: hipLaunchKernelGGL(k_ln<8>, grid, blk, 0, st, x, ldx, g, c, y, ldy, n, eps); break;
    default: hipLaunchKernelGGL(k_ln<16>, grid, blk, 0, st, x, ldx, g, c, y, ldy, n, eps); break;
    }
}

void launch_ln_conv(int rows, const float* x, const float* g, const float* c, const float* dw,
                    float* hist, size_t hist_bstride, float* at, int D, int K, float eps,
                    hipStream_t st) {
    const dim3 grid((unsigned)rows), blk(256);
#define SNHIP_LNC(P) hipLaunchKernelGGL(k_ln_conv<P>, grid, blk, 0, st, x, g, c, dw, hist, \
                                        hist_bstride, at, D, K, eps)
    switch (ln_per(D)) {
    case 1: SNHIP_LNC(1); break;
    case 2: SNHIP_LNC(2); break;
    case 4: SNHIP_LNC(4); break;
    case 6: SNHIP_LNC(6); break;
    case 8: SNHIP_LNC(8); break;
    default: SNHIP_LNC(16); break;
    }
#undef SNHIP_LNC
}

// Competitive gate, decay gate and state update for every (b, channel):
// sunnynet.c:252-266 (groups of 8, state update after the feedback GEMV).
// q rows are in the qrow_u / qrow_g order.
__global__ void k_compete_state(const float* __restrict__ q, const float* __restrict__ delta,
                                float* __restrict__ s, size_t s_bstride, float* __restrict__ u,
                                int B, int D, int clamp, float p_floor) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)B * D) return;
    const int b = (int)(idx / D), i = (int)(idx - (long)b * D);
    const float* qb = q + (size_t)b * 2 * D;
    const int base = i & ~7, off = i - base;
    const float gi = qb[qrow_g(i)];
    const float uu = qb[qrow_u(i)] * (sgm(gi - qb[qrow_g(base + ((off + 1) & 7))]) *
                                      sgm(gi - qb[qrow_g(base + ((off + 2) & 7))]));
    float p = 1.0f - delta[i] * (1.0f - sgm(gi));
    if (clamp && p < p_floor) p = p_floor;
    float* sp = s + (size_t)b * s_bstride + i;
    *sp = p * *sp + (1.0f - p) * uu;
    u[(size_t)b * D + i] = uu;
}

// Greedy token from the per-block maxima (first maximal index, the
// torch.argmax convention of sunnynet/cli.py:41). One block per sequence
// reduces the nblk partial keys; next[b] = token, and the token is appended to
// hist_tok at the device step counter. The last block to finish advances the
// counter (a done-count keeps the counter read and its update in order).
__global__ __launch_bounds__(256) void k_finalize_tok(const unsigned long long* __restrict__ part,
                                                      int nblk, int B, int32_t* __restrict__ next,
                                                      int32_t* __restrict__ hist_tok,
                                                      int32_t* __restrict__ counter,
                                                      int32_t* __restrict__ done, int cap) {
    __shared__ unsigned long long red[256];
    const int b = blockIdx.x;
    unsigned long long k = 0ull;
    for (int i = threadIdx.x; i < nblk; i += 256) k = max(k, part[(size_t)b * nblk + i]);
    red[threadIdx.x] = k;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int32_t t = (int32_t)(0xFFFFFFFFu - (uint32_t)(red[0] & 0xFFFFFFFFull));
        const int step = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        next[b] = t;
        if ((long)step * B + b < (long)cap) hist_tok[(size_t)step * B + b] = t;
        __threadfence();
        if (atomicAdd(done, 1) == B - 1) {
            *done = 0;
            __hip_atomic_store(counter, step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// (in, out) row-major -> (out, in) row-major, 32x32 tiles through LDS.
__global__ void k_transpose(const float* __restrict__ src, float* __restrict__ dst, int in,
                            int out) {
    __shared__ float tile[32][33];
    const int bo = blockIdx.x * 32, bi = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int i = bi + r, o = bo + tx;
        if (i < in && o < out) tile[r][tx] = src[(size_t)i * out + o];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int o = bo + r, i = bi + tx;
        if (o < out && i < in) dst[(size_t)o * in + i] = tile[tx][r];
    }
}

// Rows of U (2D, R) into the qrow_u / qrow_g order: dst[perm(o)] = src[o].
__global__ void k_permute_u(const float* __restrict__ src, float* __restrict__ dst, int D, int R) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= 2L * D * R) return;
    const int o = (int)(idx / R), k = (int)(idx % R);
    const int po = o < D ? qrow_u(o) : qrow_g(o - D);
    dst[(size_t)po * R + k] = src[idx];
}

// ------------------------------------------------------------------- host
struct Mat {
    int M = 0, Kd = 0;
    float* w = nullptr;
    uint8_t* q = nullptr;
    float* sc = nullptr;
    uint16_t* h = nullptr;    // fp16 bits of w (the fp16 format; read by the B=1 persistent kernel)
};

struct Layer {
    const float *ni_g, *ni_c, *nm_g, *nm_c, *dw, *delta;
    float a_tanh, b_gain;
    Mat V, U, Wz, Wc, Ws;
};

// ---------------------------------------------------------------- prefill
// x[b*T + t] = embed[tokens[b*T + t]]  (NaN rows for out-of-range ids).
__global__ void k_gather_embed(const int32_t* __restrict__ tok, const float* __restrict__ embed,
                               float* __restrict__ x, int D, int vocab) {
    const long row = blockIdx.x;
    const int t = tok[row];
    const bool ok = t >= 0 && t < vocab;
    for (int i = threadIdx.x; i < D; i += blockDim.x)
        x[row * D + i] = ok ? embed[(size_t)t * D + i] : __builtin_nanf("");
}

// at[b,t] = raw[b,t] + conv: the depthwise causal conv of the step form
// (sunnynet.c:227-233) applied to every row, with raw[b, t-1-k] taken from the
// carried history (newest first) when t-1-k < 0.
__global__ void k_conv_rows(const float* __restrict__ raw, const float* __restrict__ hist,
                            size_t hist_bstride, const float* __restrict__ dw,
                            float* __restrict__ at, int B, int T, int D, int K) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)B * T * D) return;
    const int i = (int)(idx % D);
    const long row = idx / D;
    const int b = (int)(row / T), t = (int)(row % T);
    const float r = raw[idx];
    float acc = r * dw[(size_t)(K - 1) * D + i];
    for (int k = 0; k < K - 1; ++k) {
        const int j = t - 1 - k;
        const float prev = j >= 0 ? raw[((long)b * T + j) * D + i]
                                  : hist[(size_t)b * hist_bstride + (size_t)(k - t) * D + i];
        acc = acc + prev * dw[(size_t)(K - 2 - k) * D + i];
    }
    at[idx] = r + acc;
}

// hist' = the K-1 newest raw rows (newest first), shifting in older history
// when the chunk is shorter than K-1. Runs after k_conv_rows.
__global__ void k_hist_update(const float* __restrict__ raw, float* __restrict__ hist,
                              size_t hist_bstride, int B, int T, int D, int kh) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long)B * D) return;
    const int b = (int)(idx / D), i = (int)(idx % D);
    float* hb = hist + (size_t)b * hist_bstride;
    for (int k = kh - 1; k >= 0; --k) {
        const int j = T - 1 - k;
        hb[(size_t)k * D + i] = j >= 0 ? raw[((long)b * T + j) * D + i] : hb[(size_t)(k - T) * D + i];
    }
}

// Fused competitive gate + decay gate + exact sequential scan over T for the
// prefill (the core of sunnynet/layers.py:194-206 with the recurrence of
// layers.py:314, in the operation order of the decode step). Same slot
// pipeline as the standalone scan: wave w owns TC steps of every W*TC tile;
// the wave whose slot is next prepares p and (1-p)*u (and writes u) while
// the active wave runs the chain s = p*s + (1-p)*u from registers and hands
// the state on through LDS. One lane per channel; D % 64 == 0.
template <int W, int TC>
__global__ __launch_bounds__(64 * W) void k_core_scan(
        const float* __restrict__ q, const float* __restrict__ delta,
        const float* __restrict__ s_in, size_t s_bstride, float* __restrict__ s_out,
        size_t out_bstride, float* __restrict__ u_out, float* __restrict__ states, int T, int D,
        int clamp, float p_floor) {
    __shared__ float carry[64];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gpr = D / 64;
    const int b = blockIdx.x / gpr;
    const int i = (blockIdx.x - b * gpr) * 64 + lane;
    const long row0 = (long)b * T;
    const float dl = delta[i];
    const int base = lane & ~7, off = lane & 7;
    const int n1 = base + ((off + 1) & 7), n2 = base + ((off + 2) & 7);
    constexpr int TILE = W * TC;
    const int ntiles = (T + TILE - 1) / TILE;
    const int nfull = T / TILE;
    float ur[TC], gt[TC], pa[TC], pb[TC];

    auto load_slot = [&](int tile) {
        const int t0 = tile * TILE + w * TC;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const long r = row0 + min(t0 + k, T - 1);
            ur[k] = q[r * 2 * D + qrow_u(i)];
            gt[k] = q[r * 2 * D + qrow_g(i)];
        }
    };
    auto prep = [&](int tile) {
        const int t0 = tile * TILE + w * TC;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const float gi = gt[k];
            const float g1 = __shfl(gi, n1, 64), g2 = __shfl(gi, n2, 64);
            const float uu = ur[k] * (sgm(gi - g1) * sgm(gi - g2));
            float p = 1.0f - dl * (1.0f - sgm(gi));
            if (clamp && p < p_floor) p = p_floor;
            pa[k] = p;
            pb[k] = (1.0f - p) * uu;
            if (t0 + k < T) u_out[(row0 + t0 + k) * D + i] = uu;
        }
    };

    if (w == 0) carry[lane] = s_in[(size_t)b * s_bstride + i];
    load_slot(0);
    if (w == 0) prep(0);
    __syncthreads();
    for (int tile = 0; tile < ntiles; ++tile) {
        const bool full = tile < nfull;
        for (int j = 0; j < W; ++j) {
            if (w == j) {
                float s = carry[lane];
                const int t0 = tile * TILE + j * TC;
#pragma unroll
                for (int k = 0; k < TC; ++k) {
                    if (full || t0 + k < T) {
                        s = pa[k] * s + pb[k];
                        states[(row0 + t0 + k) * D + i] = s;
                    }
                }
                carry[lane] = s;
                if (tile + 1 < ntiles) load_slot(tile + 1);
            } else if (w == j + 1) {
                prep(tile);
            } else if (j == W - 1 && w == 0 && tile + 1 < ntiles) {
                prep(tile + 1);
            }
            barrier_lds();
        }
    }
    if (w == 0) s_out[(size_t)b * out_bstride + i] = carry[lane];
}

// The per-element part of k_core_scan for every row of a prefill chunk, for
// batches too small to hide it behind the scan (sunnynet.c:248-262, same
// arithmetic as k_core_scan's prep): u = u_raw sigmoid(g - g_{+1})
// sigmoid(g - g_{+2}) within the group of 8, p = 1 - delta (1 - sigmoid(g))
// (clamped), and the scan input b = (1 - p) u.
__global__ __launch_bounds__(256) void k_gate_rows(const float* __restrict__ q, const float* __restrict__ delta,
                                                   float* __restrict__ u_out, float* __restrict__ pa,
                                                   float* __restrict__ pb, long n, int D, int clamp,
                                                   float p_floor) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n) return;
    const long r = idx / D;
    const int i = (int)(idx - r * D);
    const float* qr = q + r * 2 * D;
    const int base = i & ~7, off = i & 7;
    const float gi = qr[qrow_g(i)];
    const float g1 = qr[qrow_g(base + ((off + 1) & 7))], g2 = qr[qrow_g(base + ((off + 2) & 7))];
    const float uu = qr[qrow_u(i)] * (sgm(gi - g1) * sgm(gi - g2));
    float p = 1.0f - delta[i] * (1.0f - sgm(gi));
    if (clamp && p < p_floor) p = p_floor;
    u_out[idx] = uu;
    pa[idx] = p;
    pb[idx] = (1.0f - p) * uu;
}

// s_t = p_t s_{t-1} + b_t per channel (two roundings, as the decode step) over
// the T rows of each sequence, for 64 channels per block: in each tile of
// W TC steps wave w holds steps [w TC, (w + 1) TC), loaded before the tile's
// hand-off chain starts; the state passes wave to wave through LDS, and a wave
// loads its slice of the next tile right after its turn.
template <int W, int TC>
__global__ __launch_bounds__(64 * W) void k_scan_rows(
        const float* __restrict__ pa, const float* __restrict__ pb, const float* __restrict__ s_in,
        size_t s_bstride, float* __restrict__ s_out, size_t out_bstride, float* __restrict__ states, int T,
        int D) {
    __shared__ float carry[64];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gpr = D / 64;
    const int b = __builtin_amdgcn_readfirstlane(blockIdx.x / gpr);
    const int i = (blockIdx.x - b * gpr) * 64 + lane;
    // This sequence's rows as buffer resources: 32-bit byte offsets from a
    // scalar base (raw buffer addressing, dword 3 = 0x00020000 on gfx950).
    const size_t o = (size_t)b * T * D;
    const int bytes = T * D * 4;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(pa + o), (short)0, bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(pb + o), (short)0, bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(states + o, (short)0, bytes, 0x00020000);
    constexpr int TILE = W * TC;
    float P[TC], Bv[TC];
    auto load = [&](int t0) {
        const int ts = min(t0 + w * TC, T - 1);
        const int kmax = T - 1 - ts;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int vo = ((ts + min(k, kmax)) * D + i) * 4;
            P[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ra, vo, 0, 0));
            Bv[k] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, vo, 0, 0));
        }
    };
    if (w == 0) carry[lane] = s_in[(size_t)b * s_bstride + i];
    load(0);
    for (int t0 = 0; t0 < T; t0 += TILE) {
        const int ts = t0 + w * TC;
        for (int j = 0; j < W; ++j) {
            barrier_lds();
            if (w == j) {
                float s = carry[lane];
#pragma unroll
                for (int k = 0; k < TC; ++k)
                    if (ts + k < T) {
                        s = P[k] * s + Bv[k];
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(s), rs, ((ts + k) * D + i) * 4, 0, 0);
                    }
                carry[lane] = s;
                if (t0 + TILE < T) load(t0 + TILE);
            }
        }
    }
    barrier_lds();
    if (w == 0) s_out[(size_t)b * out_bstride + i] = carry[lane];
}

// Rows t = T-1 of each sequence: dst[b] = src[b*T + T-1].
__global__ void k_last_rows(const float* __restrict__ src, float* __restrict__ dst, int T, int D) {
    const int b = blockIdx.x;
    for (int i = threadIdx.x; i < D; i += blockDim.x)
        dst[(size_t)b * D + i] = src[((size_t)b * T + T - 1) * D + i];
}

// Per-block partial maxima of logits rows (packed keys as argmax_key), for
// the greedy token after a GEMM-computed head: grid (nblk, B).
__global__ __launch_bounds__(256) void k_argmax_partial(const float* __restrict__ logits, int V,
                                                        unsigned long long* __restrict__ part) {
    __shared__ unsigned long long red[256];
    const int b = blockIdx.y, nblk = gridDim.x;
    const int chunk = (V + nblk - 1) / nblk;
    const int lo = blockIdx.x * chunk, hi = min(V, lo + chunk);
    unsigned long long k = 0ull;
    for (int i = lo + (int)threadIdx.x; i < hi; i += 256)
        k = max(k, argmax_key(logits[(size_t)b * V + i], i));
    red[threadIdx.x] = k;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    if (threadIdx.x == 0) part[(size_t)b * nblk + blockIdx.x] = red[0];
}

}  // namespace
}  // namespace snhip

struct SnHipModel {
    int vocab = 0, D = 0, I = 0, R = 0, K = 0, L = 0, G = 0, tied = 0, clamp = 0, kh = 0;
    float eps = 0.f, p_floor = 0.f;
    int max_batch = 1, wfmt = 0, block = 32;
    std::vector<snhip::Layer> layers;
    const float *no_g = nullptr, *no_c = nullptr, *embed = nullptr;
    snhip::Mat head;
    float* s = nullptr;       // (maxB, L, D)
    float* hist = nullptr;    // (maxB, L, kh, D)
    float *x = nullptr, *at = nullptr, *v = nullptr, *q = nullptr, *u = nullptr, *z = nullptr,
          *yn = nullptr, *sfb = nullptr, *nrm = nullptr, *logits = nullptr;
    int32_t* tok = nullptr;
    unsigned long long* best = nullptr;   // (maxB, 4096) per-block packed argmax keys
    int32_t* counter = nullptr;           // device step counter of greedy decoding
    int32_t* done = nullptr;              // blocks finished in the current finalize
    int32_t* tok_hist = nullptr;          // greedy tokens, step-major rows of B
    int hist_cap = 0;                     // capacity of tok_hist in tokens
    std::vector<void*> allocs;
    hipStream_t stream = nullptr;         // caller's stream
    hipStream_t work = nullptr;           // internal stream that runs the step graphs
    hipEvent_t ev_in = nullptr, ev_out = nullptr;
    // Captured step graphs keyed by (B, logits pointer, greedy).
    std::map<std::tuple<int, const void*, int>, hipGraphExec_t> graphs;
    bool use_graphs = true;
    // Decode batches of at least this many sequences run their matmuls on the
    // MFMA GEMM; smaller batches use the GEMV kernels.
    int gemm_min_batch = 3;
    bool gemm_ok = true;
    float* gemm_work = nullptr;           // split-K partials
    size_t gemm_work_floats = 0;
    unsigned* gemm_cnt = nullptr;         // skinny-GEMM tile counters (zero between launches)
    int gemm_ncnt = 0;
    // Chunked prefill workspace for (max_batch x pf_chunk) rows, on first use.
    int pf_chunk = 0;
    float *pf_x = nullptr, *pf_raw = nullptr, *pf_at = nullptr, *pf_v = nullptr, *pf_q = nullptr,
          *pf_u = nullptr, *pf_st = nullptr, *pf_z = nullptr, *pf_yn = nullptr, *pf_sfb = nullptr,
          *pf_send = nullptr, *pf_pa = nullptr, *pf_pb = nullptr;
    int32_t* pf_tok = nullptr;
    // Persistent single-sequence decode (persist.hip): grid size, 0 when the
    // model's shape or the device does not allow it.
    int persist_wg = 0;
    // The same kernel stepping 2..mi_max sequences at once, each on its own
    // slice of mi_grid[B] workgroups (0: off); pex / psx hold mi_max
    // sequences' words and pring one ring per workgroup of the largest grid.
    int mi_max = 0;
    int mi_grid[snhip::kPersistMiMax + 1] = {};
    snhip::PLayer* dlayers = nullptr;     // device copy of the layer table
    unsigned long long* pex = nullptr;    // exchange words (2 x kPersistExWords)
    unsigned long long* psx = nullptr;    // new-state words (L x 2 x D)
    float* pring = nullptr;               // per-workgroup LN_in history rings
    unsigned* perr = nullptr;             // time-out flag
    unsigned* h_err = nullptr;            // pinned copies of the time-out flags: [0] perr, [1] berr
    unsigned persist_spin = 1u << 22;     // poll limit (SNHIP_PERSIST_SPIN)
    unsigned persist_stall = 0;           // SNHIP_PERSIST_STALL: forces time-outs (tests), read per call
    // A persistent step timed out after some workgroups had written their part
    // of the state: sequences [0, poisoned) may be part-stepped, and every
    // stepping call fails until snhip_reset, or snhip_set_state_dev over at
    // least that many sequences, gives them a valid state.
    int poisoned = 0;
    // Persistent batched step (batch.hip) for batches of gemm_min_batch ..
    // batch_max sequences: grid size, 0 when the shape or device does not allow it.
    int batch_wg = 0;
    int batch_max = 64;
    float* bbuf = nullptr;                // per-layer slabs: xs, at, v, sfb, u, z, sn
    unsigned* bflags = nullptr;           // dataflow flags (zeroed once)
    size_t bflag_words = 0;
    unsigned* berr = nullptr;             // time-out flag
    unsigned batch_epoch = 0;             // epoch of the last batched launch
    bool half = false;                    // matrices rounded to fp16 at load (sn_load_h)
    int ready = 0;
};

namespace snhip {
namespace {

template <typename T>
T* dalloc(SnHipModel* m, size_t n) {
    void* p = nullptr;
    if (hipMalloc(&p, n * sizeof(T) > 0 ? n * sizeof(T) : 4) != hipSuccess) return nullptr;
    m->allocs.push_back(p);
    return static_cast<T*>(p);
}

void free_model(SnHipModel* m) {
    if (!m) return;
    if (m->h_err) (void)hipHostFree(m->h_err);
    for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
    if (m->ev_in) (void)hipEventDestroy(m->ev_in);
    if (m->ev_out) (void)hipEventDestroy(m->ev_out);
    if (m->work) (void)hipStreamDestroy(m->work);
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

// Reads the blob like sn_load (sunnynet.c:358-454): same header check,
// same float count, NULL on any mismatch.
bool read_blob(const char* path, const int32_t want[9], std::vector<float>& payload,
               int32_t& clamp) {
    FILE* f = fopen(path, "rb");
    if (!f) { set_last_error(std::string("cannot open ") + path); return false; }
    int32_t h[10];
    if (fread(h, sizeof(int32_t), 10, f) != 10 || h[0] != kMagic) {
        fclose(f); set_last_error("bad blob header (magic)"); return false;
    }
    for (int i = 0; i < 8; ++i)
        if (h[i + 1] != want[i]) { fclose(f); set_last_error("blob header does not match the given dimensions"); return false; }
    clamp = h[9];
    const size_t D = want[1], I = want[2], R = want[3], K = want[4], L = want[5], V = want[0];
    const size_t per_layer = 2 * D + 2 * I + K * D + D * R + R * 2 * D + D * I + I * D + D * D + D + 2;
    const size_t total = L * per_layer + 2 + 2 * D + V * D + D * V;
    payload.resize(total);
    const size_t got = fread(payload.data(), sizeof(float), total, f);
    fclose(f);
    if (got != total) { set_last_error("blob is truncated"); return false; }
    return true;
}

// INT4 blob (no counterpart in the reference, which stores fp32 only):
// 12 x int32 header (magic 'SNQ4', version 1, vocab, dim, inner, rank, taps,
// layers, group, tied, clamp, block), then the fp32 blob's fields in its
// order with V, U, W_z, W_c, W_s_eff and the head as (out, in) quant.c codes
// followed by their scales; the lookup embedding stays fp32.
constexpr int32_t kMagicI4 = 0x34514E53, kVersionI4 = 1;

int32_t peek_magic(const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) return 0;
    int32_t h = 0;
    const bool ok = fread(&h, sizeof(int32_t), 1, f) == 1;
    fclose(f);
    return ok ? h : 0;
}

// Reads an INT4 blob whole and checks its header and size against the shape.
bool read_blob_i4(const char* path, const int32_t want[8], int block, std::vector<uint8_t>& raw,
                  int32_t& clamp) {
    FILE* f = fopen(path, "rb");
    if (!f) { set_last_error(std::string("cannot open ") + path); return false; }
    int32_t h[12];
    if (fread(h, sizeof(int32_t), 12, f) != 12 || h[0] != kMagicI4 || h[1] != kVersionI4) {
        fclose(f); set_last_error("bad INT4 blob header (magic or version)"); return false;
    }
    for (int i = 0; i < 8; ++i)
        if (h[i + 2] != want[i]) { fclose(f); set_last_error("INT4 blob header does not match the given dimensions"); return false; }
    if (h[11] != block) { fclose(f); set_last_error("INT4 blob group size differs from the requested block"); return false; }
    clamp = h[10];
    const size_t V = want[0], D = want[1], I = want[2], R = want[3], K = want[4], L = want[5], B = block;
    auto qbytes = [&](size_t out, size_t in) { return out * in / 2 + out * (in / B) * 4; };
    const size_t per_layer = 4 * (2 * D + 2 * I + K * D + D + 2) + qbytes(R, D) + qbytes(2 * D, R) +
                             qbytes(I, D) + qbytes(D, I) + qbytes(D, D);
    const size_t total = L * per_layer + 4 * (2 + 2 * D + V * D) + qbytes(V, D);
    raw.resize(total + 1);
    const size_t got = fread(raw.data(), 1, total + 1, f);
    fclose(f);
    if (got != total) { set_last_error(got < total ? "INT4 blob is truncated" : "INT4 blob has trailing bytes"); return false; }
    raw.resize(total);
    return true;
}

bool upload(SnHipModel* m, float*& dst, const float* src, size_t n) {
    dst = dalloc<float>(m, n);
    return dst && hipMemcpy(dst, src, n * sizeof(float), hipMemcpyHostToDevice) == hipSuccess;
}

// Storage of one weight matrix, (out, in) rows: fp32 w, or INT4 q + sc.
struct MatStore {
    float* w = nullptr;
    uint8_t* q = nullptr;
    float* sc = nullptr;
};

MatStore alloc_mat(SnHipModel* m, size_t rows, size_t in) {
    MatStore S;
    if (m->wfmt == SNHIP_WEIGHTS_F32) {
        S.w = dalloc<float>(m, rows * in);
    } else {
        S.q = dalloc<uint8_t>(m, rows * in / 2);
        S.sc = dalloc<float>(m, rows * in / m->block);
    }
    return S;
}

bool store_ok(const SnHipModel* m, const MatStore& S) {
    return m->wfmt == SNHIP_WEIGHTS_F32 ? S.w != nullptr : (S.q && S.sc);
}

// Codes and scales of an (out, in) INT4 matrix into rows row0.. of storage S;
// perm_u: U's rows go to the qrow_u / qrow_g order.
bool upload_q(SnHipModel* m, Mat& M, const uint8_t* codes, const float* scales, int in, int out,
              const MatStore& S, size_t row0, bool perm_u = false) {
    M.M = out;
    M.Kd = in;
    const size_t cb = (size_t)in / 2, sb = (size_t)in / m->block;
    M.q = S.q + row0 * cb;
    M.sc = S.sc + row0 * sb;
    if (!perm_u)
        return hipMemcpy(M.q, codes, (size_t)out * cb, hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(M.sc, scales, (size_t)out * sb * sizeof(float), hipMemcpyHostToDevice) == hipSuccess;
    std::vector<uint8_t> qc((size_t)out * cb);
    std::vector<float> sc((size_t)out * sb);
    const int half = out / 2;
    for (int i = 0; i < out; ++i) {
        const int r = i < half ? qrow_u(i) : qrow_g(i - half);
        memcpy(qc.data() + (size_t)r * cb, codes + (size_t)i * cb, cb);
        memcpy(sc.data() + (size_t)r * sb, scales + (size_t)i * sb, sb * sizeof(float));
    }
    return hipMemcpy(M.q, qc.data(), qc.size(), hipMemcpyHostToDevice) == hipSuccess &&
           hipMemcpy(M.sc, sc.data(), sc.size() * sizeof(float), hipMemcpyHostToDevice) == hipSuccess;
}


// Upload an (in,out) blob matrix as (out,in) rows starting at row `row0` of
// the storage S (quantized to INT4 for that format). perm_u: U's rows go to
// the qrow_u / qrow_g order (in = R, out = 2D).
bool upload_mat(SnHipModel* m, Mat& M, const float* src, int in, int out, float* tmp_in,
                float* tmp_out, const MatStore& S, size_t row0, bool perm_u = false) {
    M.M = out;
    M.Kd = in;
    const size_t n = (size_t)in * out;
    if (hipMemcpy(tmp_in, src, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) return false;
    dim3 grid((out + 31) / 32, (in + 31) / 32);
    hipLaunchKernelGGL(k_transpose, grid, dim3(256), 0, nullptr, tmp_in, tmp_out, in, out);
    const float* rows = tmp_out;
    if (perm_u) {
        hipLaunchKernelGGL(k_permute_u, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nullptr,
                           tmp_out, tmp_in, out / 2, in);
        rows = tmp_in;
    }
    if (m->half) {
        // _cvtss_sh(x, 0) (sunnynet.c:517,570): round to the nearest fp16, ties to even
        hipLaunchKernelGGL(k_round_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nullptr,
                           const_cast<float*>(rows), (long)n);
    }
    if (hipGetLastError() != hipSuccess) return false;
    if (m->wfmt == SNHIP_WEIGHTS_F32) {
        M.w = S.w + row0 * in;
        if (hipMemcpy(M.w, rows, n * sizeof(float), hipMemcpyDeviceToDevice) != hipSuccess) return false;
    } else {
        M.q = S.q + row0 * in / 2;
        M.sc = S.sc + row0 * in / m->block;
        if (launch_quant_i4(rows, M.q, M.sc, out, in, m->block, nullptr) != SNHIP_OK) return false;
    }
    return hipDeviceSynchronize() == hipSuccess;
}

bool upload_new(SnHipModel* m, Mat& M, const float* src, int in, int out, float* tmp_in,
                float* tmp_out, bool perm_u = false) {
    const MatStore S = alloc_mat(m, out, in);
    return store_ok(m, S) && upload_mat(m, M, src, in, out, tmp_in, tmp_out, S, 0, perm_u);
}

PMat pmat(const Mat& W) { return PMat{W.w, W.q, W.sc, W.M, W.h}; }

__global__ void k_f32_to_f16(const float* __restrict__ x, uint16_t* __restrict__ h, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = __builtin_bit_cast(uint16_t, (_Float16)x[i]);
}

// fp16 storage of rows x in values of w (already rounded to fp16 values, so
// the conversion is exact) into M.h.
bool make_f16(SnHipModel* m, Mat& M, const float* w, size_t rows, size_t in) {
    const long n = (long)(rows * in);
    M.h = dalloc<uint16_t>(m, (size_t)n);
    if (!M.h) return false;
    hipLaunchKernelGGL(k_f32_to_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, nullptr, w, M.h, n);
    return hipGetLastError() == hipSuccess;
}

// The fp16 format: the five matrices and the head held as fp16 for the
// single-sequence persistent step (half the bytes it streams, as sn_load_h
// holds them, sunnynet.c:455-579); the other paths multiply the same values
// from the fp32 copy.
bool make_f16_copies(SnHipModel* m) {
    for (Layer& A : m->layers) {
        // V and W_eff share one storage: V's rows, then W_eff's
        if (!make_f16(m, A.V, A.V.w, (size_t)A.V.M + A.Ws.M, A.V.Kd) ||
            !make_f16(m, A.U, A.U.w, A.U.M, A.U.Kd) || !make_f16(m, A.Wz, A.Wz.w, A.Wz.M, A.Wz.Kd) ||
            !make_f16(m, A.Wc, A.Wc.w, A.Wc.M, A.Wc.Kd))
            return false;
    }
    return make_f16(m, m->head, m->head.w, m->head.M, m->head.Kd) && hipDeviceSynchronize() == hipSuccess;
}

// Weight-format code of the B=1 persistent kernel: 0 fp32, 16 fp16, else the INT4 group.
int persist_blk(const SnHipModel* m) {
    return m->wfmt == SNHIP_WEIGHTS_INT4 ? m->block : (m->half && m->head.h ? 16 : 0);
}

// The device layer table of the persistent kernels (built once).
bool layer_table(SnHipModel* m) {
    if (m->dlayers) return true;
    std::vector<PLayer> hl(m->L);
    for (int l = 0; l < m->L; ++l) {
        const Layer& A = m->layers[l];
        PLayer& P = hl[l];
        P.ni_g = A.ni_g; P.ni_c = A.ni_c; P.nm_g = A.nm_g; P.nm_c = A.nm_c;
        P.dw = A.dw; P.delta = A.delta; P.a_tanh = A.a_tanh; P.b_gain = A.b_gain;
        P.VW = pmat(A.V);
        P.VW.M = A.V.M + A.Ws.M;      // W_eff's rows follow V's in one storage
        P.U = pmat(A.U); P.Wz = pmat(A.Wz); P.Wc = pmat(A.Wc);
    }
    PLayer* d = dalloc<PLayer>(m, m->L);
    if (!d || hipMemcpy(d, hl.data(), hl.size() * sizeof(PLayer), hipMemcpyHostToDevice) != hipSuccess)
        return false;
    m->dlayers = d;
    return true;
}

// Pinned host copies of the persistent kernels' time-out flags.
bool host_err(SnHipModel* m) {
    if (m->h_err) return true;
    if (hipHostMalloc((void**)&m->h_err, 2 * sizeof(unsigned), 0) != hipSuccess) {
        m->h_err = nullptr;
        return false;
    }
    m->h_err[0] = m->h_err[1] = 0;
    return true;
}

// Grids of the single-sequence kernel stepping B = 2..mi_max sequences in one
// launch: each sequence gets the largest grid the kernel accepts (at most cap,
// the one-sequence grid, and ncu / B, so the whole launch is one workgroup per
// CU). Workgroup w of every sequence sits on the same XCD (slices are
// multiples of 8 workgroups) and reads the same weight rows in the same phase,
// so most rows reach the other sequences from that XCD's L2: eight sequences
// of SunnyNet-100M INT4 fetch 131 MB per step from HBM (rocprofv3 FETCH_SIZE),
// against 87 MB for one sequence alone. mi_max defaults to the
// sizes measured faster than the batched kernel (SunnyNet-100M, one MI355X,
// us/step): INT4 g32 up to 16 (B=2 183.7 against 281.5, B=4 206.4 / 349.6,
// B=8 252.5 / 369.7, B=16 359.2 / 400.3; B=24 541.3 against 430.1), fp32 and
// fp16 rows up to 4 (B=2 253.1 / 731.1, B=4 351.7 / 379.2; B=8 513.9 against
// 399.8). SNHIP_PERSIST_MI sets it (1: off). Returns the sequences the
// exchange words must hold.
int setup_persist_mi(SnHipModel* m, int ncu, int cap) {
    const unsigned dflt = m->wfmt == SNHIP_WEIGHTS_INT4 ? 16 : 4;
    int lim = std::min(m->max_batch, kPersistMiMax);
    lim = std::min(lim, (int)std::min(env_unsigned("SNHIP_PERSIST_MI", dflt, 0), (unsigned)kPersistMiMax));
    m->mi_max = 0;
    for (int b = 2; b <= lim; ++b) {
        int g = 0;
        for (int c = std::min(cap, ncu / b); c >= 1 && !g; --c)
            if (persist_grid_ok(c, m->D, m->I, m->R, m->vocab)) g = c;
        if (g < 1) break;
        m->mi_grid[b] = g;
        m->mi_max = b;
    }
    return std::max(1, m->mi_max);
}

// Enables the persistent single-sequence decode when the shape fits it and the
// device supports cooperative launches (SNHIP_PERSIST=0 turns it off;
// SNHIP_PERSIST_WG caps the grid size). The grid is the largest size the
// kernel accepts for the shape (persist_grid_ok) up to one workgroup per CU
// and per four channels (fp32 / fp16 rows) or eight (INT4 rows): measured
// fastest at dim 1024, 256 workgroups for fp32 (225.2 us/step against 250.4
// at 128) and 128 for INT4 (180.2 against 184.0 at 256: half the workgroups
// poll each exchange).
void setup_persist(SnHipModel* m) {
    if (const char* e = getenv("SNHIP_PERSIST"))
        if (e[0] == '0') return;
    if (m->D > kPersistMaxD || m->I > kPersistMaxK || m->R > kPersistMaxK ||
        m->K != kPersistTaps || m->D % 8 || m->L > kPersistMaxL)
        return;
    int dev = 0, coop = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return;
    const int occ = persist_occupancy(persist_blk(m));
    if (occ < 1) return;
    int cap = std::min(m->D / (m->wfmt == SNHIP_WEIGHTS_INT4 ? 8 : 4), ncu);
    if (const char* e = getenv("SNHIP_PERSIST_WG")) cap = atoi(e);
    cap = std::min(std::min(cap, ncu * occ), kPersistMaxGrid);
    int nwg = 0;
    for (int g = cap; g >= 1 && !nwg; --g)
        if (persist_grid_ok(g, m->D, m->I, m->R, m->vocab)) nwg = g;
    if (nwg < 1) return;
    const int nseq = setup_persist_mi(m, ncu, cap);
    int ring_wg = nwg;
    for (int b = 2; b <= m->mi_max; ++b) ring_wg = std::max(ring_wg, b * m->mi_grid[b]);
    m->pex = dalloc<unsigned long long>(m, 2 * (size_t)kPersistExWords * nseq);
    m->psx = dalloc<unsigned long long>(m, (size_t)m->L * 2 * m->D * nseq);
    m->pring = dalloc<float>(m, (size_t)ring_wg * m->L * m->kh * m->D);
    m->perr = dalloc<unsigned>(m, 1);
    if (!m->pex || !m->psx || !m->pring || !m->perr || !layer_table(m) || !host_err(m)) {
        m->mi_max = 0;
        return;
    }
    m->persist_wg = nwg;
}

// Enables the persistent batched step (batch.hip) when the shape fits it and
// the device supports cooperative launches (SNHIP_BATCH_PERSIST=0 turns it
// off). Its per-layer slabs are sized for min(max_batch, batch_max) rows.
void setup_batch(SnHipModel* m) {
    if (const char* e = getenv("SNHIP_BATCH_PERSIST"))
        if (e[0] == '0') return;
    if (!m->gemm_ok || m->max_batch < m->gemm_min_batch || !batch_shape_ok(m->D, m->I, m->R, m->K, m->L) ||
        m->kh != kPersistTaps - 1)
        return;
    const int G = batch_grid(m->wfmt == SNHIP_WEIGHTS_INT4 ? m->block : 0, m->D, m->I, m->R);
    if (G < 8) return;
    const size_t B = (size_t)std::min(m->max_batch, m->batch_max);
    const size_t per = (size_t)m->L * (5 * (size_t)m->D + m->R + m->I);
    m->bbuf = dalloc<float>(m, B * per);
    m->bflag_words = batch_flag_words(m->L, (int)B, m->D, m->I, m->R);
    m->bflags = dalloc<unsigned>(m, m->bflag_words);
    m->berr = dalloc<unsigned>(m, 1);
    if (!m->bbuf || !m->bflags || !m->berr || !layer_table(m) || !host_err(m) ||
        hipMemset(m->berr, 0, sizeof(unsigned)) != hipSuccess ||
        hipMemset(m->bflags, 0, m->bflag_words * sizeof(unsigned)) != hipSuccess)
        return;
    m->batch_wg = G;
}

// Every weight of an INT4 blob (past its header) onto the device.
bool load_layers_i4(SnHipModel* m, const uint8_t* raw) {
    const size_t D = m->D, I = m->I, R = m->R, K = m->K, V = m->vocab, BL = m->block;
    const uint8_t* o = raw;
    auto f32 = [&](size_t n) {
        const float* a = reinterpret_cast<const float*>(o);
        o += 4 * n;
        return a;
    };
    auto mat = [&](size_t out, size_t in, const uint8_t*& q, const float*& sc) {
        q = o;
        o += out * in / 2;
        sc = reinterpret_cast<const float*>(o);
        o += out * (in / BL) * 4;
    };
    bool ok = true;
    for (int l = 0; l < m->L && ok; ++l) {
        Layer& A = m->layers[l];
        float* t;
        ok &= upload(m, t, f32(D), D); A.ni_g = t;
        ok &= upload(m, t, f32(D), D); A.ni_c = t;
        ok &= upload(m, t, f32(I), I); A.nm_g = t;
        ok &= upload(m, t, f32(I), I); A.nm_c = t;
        ok &= upload(m, t, f32(K * D), K * D); A.dw = t;
        const uint8_t* q;
        const float* sc;
        const MatStore vw = alloc_mat(m, R + D, D);        // V's rows, then W_eff's
        ok = ok && store_ok(m, vw);
        mat(R, D, q, sc); ok = ok && upload_q(m, A.V, q, sc, (int)D, (int)R, vw, 0);
        mat(2 * D, R, q, sc);
        const MatStore us = alloc_mat(m, 2 * D, R);
        ok = ok && store_ok(m, us) && upload_q(m, A.U, q, sc, (int)R, (int)(2 * D), us, 0, true);
        mat(I, D, q, sc);
        const MatStore zs = alloc_mat(m, I, D);
        ok = ok && store_ok(m, zs) && upload_q(m, A.Wz, q, sc, (int)D, (int)I, zs, 0);
        mat(D, I, q, sc);
        const MatStore cs = alloc_mat(m, D, I);
        ok = ok && store_ok(m, cs) && upload_q(m, A.Wc, q, sc, (int)I, (int)D, cs, 0);
        mat(D, D, q, sc); ok = ok && upload_q(m, A.Ws, q, sc, (int)D, (int)D, vw, R);
        ok &= upload(m, t, f32(D), D); A.delta = t;
        const float* ab = f32(2);
        A.a_tanh = ab[0]; A.b_gain = ab[1];
    }
    if (!ok) return false;
    const float* ep = f32(2);
    m->eps = ep[0]; m->p_floor = ep[1];
    float* t;
    ok &= upload(m, t, f32(D), D); m->no_g = t;
    ok &= upload(m, t, f32(D), D); m->no_c = t;
    ok &= upload(m, t, f32(V * D), V * D); m->embed = t;
    const uint8_t* q;
    const float* sc;
    mat(V, D, q, sc);
    const MatStore hs = alloc_mat(m, V, D);
    return ok && store_ok(m, hs) && upload_q(m, m->head, q, sc, (int)D, (int)V, hs, 0);
}

SnHipModel* load_model(const char* path, int vocab, int dim, int inner, int rank, int taps,
                       int layers, int group, int tied, int max_batch, int wfmt, int block) {
    if (!path || vocab <= 0 || dim <= 0 || inner <= 0 || rank <= 0 || taps <= 0 || layers <= 0 ||
        max_batch <= 0) {
        set_last_error("invalid arguments");
        return nullptr;
    }
    if (group != 8 || dim % 8 || taps > kMaxTaps) {
        set_last_error("unsupported shape: group must be 8, dim a multiple of 8, taps <= 8");
        return nullptr;
    }
    if (dim % 4 || inner % 4 || rank % 4) { set_last_error("dim, inner, rank must be multiples of 4"); return nullptr; }
    if (dim > kLnPer * 256 || inner > kLnPer * 256) { set_last_error("dim and inner must be <= 4096"); return nullptr; }
    if (max_batch > 1024) { set_last_error("max_batch must be <= 1024"); return nullptr; }
    if (wfmt == SNHIP_WEIGHTS_INT4) {
        if (block != 32 && block != 64) { set_last_error("INT4 block must be 32 or 64"); return nullptr; }
        if (dim % block || inner % block || rank % block) {
            set_last_error("INT4 block must divide dim, inner and rank");
            return nullptr;
        }
    } else if (wfmt != SNHIP_WEIGHTS_F32 && wfmt != SNHIP_WEIGHTS_F16) {
        set_last_error("unknown weight format");
        return nullptr;
    }
    // fp16 values (sn_load_h) are held as fp32: every kernel takes the fp32 path.
    const bool half = wfmt == SNHIP_WEIGHTS_F16;
    if (half) wfmt = SNHIP_WEIGHTS_F32;
    const int32_t want[9] = {vocab, dim, inner, rank, taps, layers, group, tied, 0};
    std::vector<float> P;
    std::vector<uint8_t> Q;                  // an INT4 blob, read whole
    int32_t clamp = 0;
    const bool i4blob = peek_magic(path) == kMagicI4;
    if (i4blob) {
        if (wfmt != SNHIP_WEIGHTS_INT4) {
            set_last_error("an INT4 blob needs weight format SNHIP_WEIGHTS_INT4");
            return nullptr;
        }
        if (!read_blob_i4(path, want, block, Q, clamp)) return nullptr;
    } else if (!read_blob(path, want, P, clamp)) {
        return nullptr;
    }

    SnHipModel* m = new SnHipModel();
    m->vocab = vocab; m->D = dim; m->I = inner; m->R = rank; m->K = taps; m->L = layers;
    m->G = group; m->tied = tied; m->clamp = clamp; m->kh = taps > 1 ? taps - 1 : 0;
    m->max_batch = max_batch; m->wfmt = wfmt; m->block = block; m->half = half;
    const size_t D = dim, I = inner, R = rank, K = taps, V = vocab;
    const size_t big = std::max(std::max(D * R, R * 2 * D), std::max(D * I, std::max(D * D, D * V)));
    float* tmp_in = dalloc<float>(m, big);
    float* tmp_out = dalloc<float>(m, big);
    if (!tmp_in || !tmp_out) { free_model(m); set_last_error("out of device memory"); return nullptr; }

    const float* p = P.data();
    bool ok = true;
    m->layers.resize(layers);
    if (i4blob) ok = load_layers_i4(m, Q.data());
    for (int l = 0; l < layers && ok && !i4blob; ++l) {
        Layer& A = m->layers[l];
        float* t;
        ok &= upload(m, t, p, D); A.ni_g = t; p += D;
        ok &= upload(m, t, p, D); A.ni_c = t; p += D;
        ok &= upload(m, t, p, I); A.nm_g = t; p += I;
        ok &= upload(m, t, p, I); A.nm_c = t; p += I;
        ok &= upload(m, t, p, K * D); A.dw = t; p += K * D;
        // V and W_eff share one (R + D, D) storage: V's rows, then W_eff's.
        const MatStore vw = alloc_mat(m, R + D, D);
        ok = ok && store_ok(m, vw);
        ok = ok && upload_mat(m, A.V, p, dim, rank, tmp_in, tmp_out, vw, 0); p += D * R;
        ok = ok && upload_new(m, A.U, p, rank, 2 * dim, tmp_in, tmp_out, true); p += R * 2 * D;
        ok = ok && upload_new(m, A.Wz, p, dim, inner, tmp_in, tmp_out); p += D * I;
        ok = ok && upload_new(m, A.Wc, p, inner, dim, tmp_in, tmp_out); p += I * D;
        ok = ok && upload_mat(m, A.Ws, p, dim, dim, tmp_in, tmp_out, vw, R); p += D * D;
        ok &= upload(m, t, p, D); A.delta = t; p += D;
        A.a_tanh = p[0]; A.b_gain = p[1]; p += 2;
    }
    if (ok && !i4blob) {
        m->eps = p[0]; m->p_floor = p[1]; p += 2;
        float* t;
        ok &= upload(m, t, p, D); m->no_g = t; p += D;
        ok &= upload(m, t, p, D); m->no_c = t; p += D;
        ok &= upload(m, t, p, V * D); m->embed = t; p += V * D;
        ok = ok && upload_new(m, m->head, p, dim, vocab, tmp_in, tmp_out);
    }
    const size_t B = max_batch;
    if (ok) {
        m->s = dalloc<float>(m, B * layers * D);
        m->hist = dalloc<float>(m, B * layers * (m->kh ? m->kh : 1) * D);
        m->x = dalloc<float>(m, B * D);
        m->at = dalloc<float>(m, B * D);
        m->v = dalloc<float>(m, B * R);
        m->q = dalloc<float>(m, B * 2 * D);
        m->u = dalloc<float>(m, B * D);
        m->z = dalloc<float>(m, B * I);
        m->yn = dalloc<float>(m, B * I);
        m->sfb = dalloc<float>(m, B * D);
        m->nrm = dalloc<float>(m, B * D);
        m->logits = dalloc<float>(m, B * V);
        m->tok = dalloc<int32_t>(m, B);
        m->best = dalloc<unsigned long long>(m, B * 4096);
        m->counter = dalloc<int32_t>(m, 1);
        m->done = dalloc<int32_t>(m, 1);
        ok = m->s && m->hist && m->x && m->at && m->v && m->q && m->u && m->z && m->yn && m->sfb &&
             m->nrm && m->logits && m->tok && m->best && m->counter && m->done;
    }
    if (!ok) {
        if (last_error().empty()) set_last_error("device allocation or upload failed");
        free_model(m);
        return nullptr;
    }
    // The transpose staging buffers are no longer needed.
    for (auto it = m->allocs.begin(); it != m->allocs.end();) {
        if (*it == tmp_in || *it == tmp_out) { (void)hipFree(*it); it = m->allocs.erase(it); }
        else ++it;
    }
    if (hipMemset(m->s, 0, B * layers * D * sizeof(float)) != hipSuccess ||
        hipMemset(m->hist, 0, B * layers * (m->kh ? m->kh : 1) * D * sizeof(float)) != hipSuccess ||
        hipMemset(m->counter, 0, sizeof(int32_t)) != hipSuccess ||
        hipMemset(m->done, 0, sizeof(int32_t)) != hipSuccess ||
        hipStreamCreateWithFlags(&m->work, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_in, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_out, hipEventDisableTiming) != hipSuccess) {
        set_last_error("device setup failed");
        free_model(m);
        return nullptr;
    }
    if (const char* e = getenv("SNHIP_NO_GRAPH")) m->use_graphs = !(e[0] == '1');
    if (const char* e = getenv("SNHIP_GEMM_MIN_BATCH")) m->gemm_min_batch = std::max(1, atoi(e));
    // The MFMA GEMM needs every contraction length to be a multiple of 32.
    m->gemm_ok = dim % 32 == 0 && inner % 32 == 0 && rank % 32 == 0;
    if (!m->gemm_ok) m->gemm_min_batch = 1 << 30;
    m->gemm_work_floats = (size_t)16 << 20;
    m->gemm_work = dalloc<float>(m, m->gemm_work_floats);
    m->gemm_ncnt = 4096;
    m->gemm_cnt = dalloc<unsigned>(m, m->gemm_ncnt);
    if (!m->gemm_work || !m->gemm_cnt ||
        hipMemset(m->gemm_cnt, 0, m->gemm_ncnt * sizeof(unsigned)) != hipSuccess) {
        set_last_error("out of device memory");
        free_model(m);
        return nullptr;
    }
    m->persist_spin = env_unsigned("SNHIP_PERSIST_SPIN", m->persist_spin, 1);
    if (m->half && m->wfmt == SNHIP_WEIGHTS_F32 && !make_f16_copies(m)) {
        set_last_error("fp16 weight copies: device allocation or conversion failed");
        free_model(m);
        return nullptr;
    }
    setup_persist(m);
    setup_batch(m);
    m->ready = 1;
    return m;
}

GemvJob make_job(const Mat& W, int B, const float* X, int ldx, float* Y, int ldy) {
    GemvJob j{};
    j.w = W.w; j.q = W.q; j.sc = W.sc;
    j.M = W.M; j.Kd = W.Kd; j.B = B;
    j.X = X; j.ldx = ldx; j.Y = Y; j.ldy = ldy;
    j.epi = EPI_STORE;
    return j;
}

// One or two GEMV jobs in one launch (j1.M == 0: one job).
hipError_t launch_gemv(const SnHipModel* m, GemvJob j0, GemvJob j1, hipStream_t st) {
    GemvJob js[2] = {j0, j1};
    return launch_gemv(js, j1.M > 0 ? 2 : 1, m->wfmt == SNHIP_WEIGHTS_INT4 ? m->block : 0, st);
}

GemmArgs gemm_for(const SnHipModel* m, const Mat& W, const float* X, long ldx, int M, float* Y,
                  long ldy) {
    GemmArgs g{};
    g.X = X; g.ldx = ldx;
    g.w = W.w; g.q = W.q; g.sc = W.sc;
    g.block = W.q ? m->block : 0;
    g.M = M; g.N = W.M; g.K = W.Kd;
    g.Y = Y; g.ldy = ldy;
    g.epi = GEPI_STORE;
    return g;
}

GemmWork gemm_work(const SnHipModel* m) {
    GemmWork w;
    w.part = m->gemm_work; w.part_floats = m->gemm_work_floats;
    w.cnt = m->gemm_cnt; w.ncnt = m->gemm_ncnt;
    return w;
}

snhip_status run_gemm(SnHipModel* m, const GemmArgs& g, hipStream_t st) {
    return launch_gemm(g, gemm_work(m), st);
}

__global__ void k_copy_rows(const float* __restrict__ src, long lds, float* __restrict__ dst,
                            long ldd, int D) {
    const int b = blockIdx.x;
    for (int i = threadIdx.x; i < D; i += blockDim.x) dst[b * ldd + i] = src[b * lds + i];
}

// Final norm, LM head and (greedy) token selection for B rows of x.
// Does a step of B sequences run as the batched persistent kernel?
bool uses_batch(const SnHipModel* m, int B) {
    return m->batch_wg > 0 && B >= m->gemm_min_batch && B <= std::min(m->max_batch, m->batch_max);
}

snhip_status enqueue_head(SnHipModel* m, int B, const float* x, float* logits_out, bool greedy,
                          hipStream_t st, bool normed = false) {
    const int D = m->D;
    if (!normed) launch_ln(B, x, D, m->no_g, m->no_c, m->nrm, D, D, m->eps, st);
    if (B >= m->gemm_min_batch) {
        const snhip_status rc = run_gemm(m, gemm_for(m, m->head, m->nrm, D, B, logits_out, m->vocab), st);
        if (rc != SNHIP_OK) return rc;
        if (greedy) {
            const int nblk = 64;
            hipLaunchKernelGGL(k_argmax_partial, dim3(nblk, B), dim3(256), 0, st, logits_out,
                               m->vocab, m->best);
            hipLaunchKernelGGL(k_finalize_tok, dim3(B), dim3(256), 0, st, m->best, nblk, B, m->tok,
                               m->tok_hist, m->counter, m->done, m->hist_cap);
        }
    } else {
        GemvJob jh = make_job(m->head, B, m->nrm, D, logits_out, m->vocab);
        if (greedy) {
            jh.epi = EPI_ARGMAX;
            jh.best = m->best;
        }
        GemvJob none{};
        SNHIP_CHECK(launch_gemv(m, jh, none, st));
        if (greedy)
            hipLaunchKernelGGL(k_finalize_tok, dim3(B), dim3(256), 0, st, m->best,
                               gemv_blocks(jh, m->wfmt == SNHIP_WEIGHTS_INT4 ? m->block : 0), B, m->tok, m->tok_hist,
                               m->counter, m->done, m->hist_cap);
    }
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// Layer l of the GEMV step for sequences [0, B), after LN_in + conv wrote
// m->at: v = V at and sfb = W_eff s_old (one launch), q = U v, the gates and
// the state update (m->u, s'), z = wedge(W_z u), yn = LN_I(z), and
// x' = W_c yn + b s' + sfb + x into m->x (sunnynet.c:239-276). Every
// intermediate stays in its buffer until the next layer (snhip_dbg_layer
// reads them).
snhip_status enqueue_layer_gemv(SnHipModel* m, int B, int l, hipStream_t st) {
    const int D = m->D, I = m->I, R = m->R, L = m->L;
    const size_t sbs = (size_t)L * D;
    const Layer& A = m->layers[l];
    float* s_l = m->s + (size_t)l * D;
    const long n = (long)B * D;
    GemvJob jv = make_job(A.V, B, m->at, D, m->v, R);
    GemvJob js = make_job(A.Ws, B, s_l, (int)sbs, m->sfb, D);
    SNHIP_CHECK(launch_gemv(m, jv, js, st));
    GemvJob ju = make_job(A.U, B, m->v, R, m->q, 2 * D);
    GemvJob none{};
    SNHIP_CHECK(launch_gemv(m, ju, none, st));
    hipLaunchKernelGGL(k_compete_state, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       m->q, A.delta, s_l, sbs, m->u, B, D, m->clamp, m->p_floor);
    GemvJob jz = make_job(A.Wz, B, m->u, D, m->z, I);
    jz.epi = EPI_WEDGE;
    jz.a_tanh = A.a_tanh;
    SNHIP_CHECK(launch_gemv(m, jz, none, st));
    launch_ln(B, m->z, I, A.nm_g, A.nm_c, m->yn, I, I, m->eps, st);
    GemvJob jc = make_job(A.Wc, B, m->yn, I, m->x, D);
    jc.epi = EPI_RESID;
    jc.b_gain = A.b_gain;
    jc.s = s_l; jc.lds = (int)sbs;
    jc.sfb = m->sfb; jc.ldf = D;
    SNHIP_CHECK(launch_gemv(m, jc, none, st));
    return SNHIP_OK;
}

// Enqueue one decode step for sequences [0, B) on `st`; tokens in m->tok.
// greedy: the head also reduces the first maximal logit per sequence and a
// final kernel writes it to m->tok (the next step's input) and m->tok_hist.
snhip_status enqueue_step(SnHipModel* m, int B, float* logits_out, bool greedy, hipStream_t st) {
    const int D = m->D, I = m->I, R = m->R, L = m->L;
    const size_t sbs = (size_t)L * D;                               // s batch stride
    const size_t hbs = (size_t)L * (m->kh ? m->kh : 1) * D;         // hist batch stride
    if (uses_batch(m, B)) {
        // Every layer in one cooperative launch (the embedding rows gathered
        // inside), then the head.
        BatchArgs a{};
        a.layers = m->dlayers;
        a.L = L; a.B = B; a.D = D; a.I = I; a.R = R; a.K = m->K; a.kh = m->kh;
        a.clamp = m->clamp; a.eps = m->eps; a.p_floor = m->p_floor;
        a.no_g = m->no_g; a.no_c = m->no_c;
        a.tok = m->tok; a.embed = m->embed; a.vocab = m->vocab;
        float* p = m->bbuf;
        const size_t LB = (size_t)L * B;
        a.xs = p; p += LB * D;
        a.at = p; p += LB * D;
        a.v = p; p += LB * R;
        a.sfb = p; p += LB * D;
        a.u = p; p += LB * D;
        a.z = p; p += LB * I;
        a.sn = p;
        a.s = m->s; a.hist = m->hist; a.nrm = m->nrm;
        a.flags = m->bflags; a.err = m->berr; a.spin_limit = m->persist_spin; a.stall = m->persist_stall;
        if (m->batch_epoch == 0xFFFFFFFFu) {
            // epochs start over from clean flags
            SNHIP_CHECK(hipMemsetAsync(m->bflags, 0, m->bflag_words * sizeof(unsigned), st));
            m->batch_epoch = 0;
        }
        a.epoch = ++m->batch_epoch;
        const snhip_status rc = launch_decode_batch(a, m->batch_wg, m->wfmt == SNHIP_WEIGHTS_INT4 ? m->block : 0, st);
        if (rc != SNHIP_OK) return rc;
        return enqueue_head(m, B, nullptr, logits_out, greedy, st, true);
    }
    hipLaunchKernelGGL(k_embed, dim3(B), dim3(256), 0, st, m->tok, m->embed, m->x, D, m->vocab);
    const bool mm = B >= m->gemm_min_batch;
    for (int l = 0; l < L; ++l) {
        const Layer& A = m->layers[l];
        float* s_l = m->s + (size_t)l * D;
        float* h_l = m->hist + (size_t)l * (m->kh ? m->kh : 1) * D;
        launch_ln_conv(B, m->x, A.ni_g, A.ni_c, A.dw, h_l, hbs, m->at, D, m->K, m->eps, st);
        const long n = (long)B * D;
        if (mm) {
            snhip_status rc;
            // v = V at and sfb = W_eff s (old state) in one launch.
            if ((rc = launch_gemm2(gemm_for(m, A.V, m->at, D, B, m->v, R),
                                   gemm_for(m, A.Ws, s_l, (long)sbs, B, m->sfb, D), gemm_work(m),
                                   st)) != SNHIP_OK)
                return rc;
            GemmArgs gu = gemm_for(m, A.U, m->v, R, B, m->q, 2 * D);
            if (gemm_fuses_compete(gu, gemm_work(m))) {
                // Gate and state update in the U product's epilogue.
                gu.epi = GEPI_COMPETE;
                gu.Y = m->u; gu.ldy = D;
                gu.s = s_l; gu.lds = (long)sbs;
                gu.delta = A.delta; gu.clamp = m->clamp; gu.p_floor = m->p_floor;
                if ((rc = run_gemm(m, gu, st)) != SNHIP_OK) return rc;
            } else {
                if ((rc = run_gemm(m, gu, st)) != SNHIP_OK) return rc;
                hipLaunchKernelGGL(k_compete_state, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                                   st, m->q, A.delta, s_l, sbs, m->u, B, D, m->clamp, m->p_floor);
            }
            GemmArgs gz = gemm_for(m, A.Wz, m->u, D, B, m->z, I);
            gz.epi = GEPI_WEDGE;
            gz.a_tanh = A.a_tanh;
            if ((rc = run_gemm(m, gz, st)) != SNHIP_OK) return rc;
            launch_ln(B, m->z, I, A.nm_g, A.nm_c, m->yn, I, I, m->eps, st);
            GemmArgs gc = gemm_for(m, A.Wc, m->yn, I, B, m->x, D);
            gc.epi = GEPI_RESID;
            gc.b_gain = A.b_gain;
            gc.s = s_l; gc.lds = (long)sbs;
            gc.sfb = m->sfb; gc.ldf = D;
            if ((rc = run_gemm(m, gc, st)) != SNHIP_OK) return rc;
            continue;
        }
        const snhip_status rc = enqueue_layer_gemv(m, B, l, st);
        if (rc != SNHIP_OK) return rc;
    }
    return enqueue_head(m, B, m->x, logits_out, greedy, st);
}

// After a synchronization: did a persistent launch over sequences [0, rows)
// time out at a wait? Its workgroups stop independently: one that passed its
// last wait before another timed out has already written its channels' state
// (single sequence) or its layers' state (batched). Those rows are then
// refused for stepping until their state is reset or set.
snhip_status persist_status(SnHipModel* m, int rows) {
    const bool single = m->h_err && m->h_err[0];
    const bool batched = m->h_err && m->h_err[1];
    if (!single && !batched) return SNHIP_OK;
    m->h_err[0] = m->h_err[1] = 0;
    m->poisoned = std::max(m->poisoned, rows);
    set_last_error(single ? "persistent decode: exchange wait timed out"
                          : "batched persistent decode: a dataflow wait timed out");
    return SNHIP_E_DEVICE;
}

// Stepping calls refuse a handle whose state a timed-out step left part-written.
snhip_status check_usable(const SnHipModel* m) {
    if (m->poisoned) {
        set_last_error("the sequence state was left part-stepped by a timed-out step; "
                       "call snhip_reset, or snhip_set_state_dev over every sequence it stepped, first");
        return SNHIP_E_DEVICE;
    }
    return SNHIP_OK;
}

// Runs `reps` decode steps on the internal stream, ordered after the work
// already queued on the caller's stream and before anything queued on it
// later. The step's kernels are captured once per (B, logits, greedy) into a
// HIP graph and replayed.
snhip_status run_steps(SnHipModel* m, int B, float* logits_out, bool greedy, int reps) {
    SNHIP_CHECK(hipEventRecord(m->ev_in, m->stream));
    SNHIP_CHECK(hipStreamWaitEvent(m->work, m->ev_in, 0));
    const bool batch = uses_batch(m, B);
    if (!m->use_graphs || batch) {
        // The batched persistent step is a handful of launches per step: they
        // are queued directly (a cooperative launch is not captured).
        if (batch) {
            m->persist_stall = env_unsigned("SNHIP_PERSIST_STALL", 0, 0);
            SNHIP_CHECK(hipMemsetAsync(m->berr, 0, sizeof(unsigned), m->work));
        }
        for (int i = 0; i < reps; ++i) {
            const snhip_status rc = enqueue_step(m, B, logits_out, greedy, m->work);
            if (rc != SNHIP_OK) return rc;
        }
        if (batch) {
            // The call returns once its launches have finished, so that a
            // barrier time-out is reported by this call, not a later one.
            SNHIP_CHECK(hipMemcpyAsync(m->h_err + 1, m->berr, sizeof(unsigned), hipMemcpyDeviceToHost, m->work));
            SNHIP_CHECK(hipStreamSynchronize(m->work));
            const snhip_status st = persist_status(m, B);
            if (st != SNHIP_OK) return st;
        }
    } else {
        const auto key = std::make_tuple(B, (const void*)logits_out, greedy ? 1 : 0);
        auto it = m->graphs.find(key);
        if (it == m->graphs.end()) {
            if (m->graphs.size() >= 16) {
                for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
                m->graphs.clear();
            }
            hipGraph_t g = nullptr;
            SNHIP_CHECK(hipStreamBeginCapture(m->work, hipStreamCaptureModeThreadLocal));
            const snhip_status rc = enqueue_step(m, B, logits_out, greedy, m->work);
            const hipError_t ec = hipStreamEndCapture(m->work, &g);
            if (rc != SNHIP_OK) { if (g) (void)hipGraphDestroy(g); return rc; }
            SNHIP_CHECK(ec);
            hipGraphExec_t ex = nullptr;
            const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            SNHIP_CHECK(ei);
            it = m->graphs.emplace(key, ex).first;
        }
        for (int i = 0; i < reps; ++i) SNHIP_CHECK(hipGraphLaunch(it->second, m->work));
    }
    SNHIP_CHECK(hipEventRecord(m->ev_out, m->work));
    SNHIP_CHECK(hipStreamWaitEvent(m->stream, m->ev_out, 0));
    return SNHIP_OK;
}

// Copies B tokens into m->tok on the caller's stream.
snhip_status put_tokens(SnHipModel* m, const int32_t* t, int B, hipMemcpyKind kind) {
    SNHIP_CHECK(hipMemcpyAsync(m->tok, t, B * sizeof(int32_t), kind, m->stream));
    return SNHIP_OK;
}

// Workspace of the chunked prefill for max_batch x chunk rows.
snhip_status ensure_prefill_ws(SnHipModel* m, int chunk) {
    if (m->pf_chunk >= chunk) return SNHIP_OK;
    SNHIP_CHECK(hipStreamSynchronize(m->stream));
    SNHIP_CHECK(hipStreamSynchronize(m->work));
    float** bufs[] = {&m->pf_x, &m->pf_raw, &m->pf_at, &m->pf_v, &m->pf_q, &m->pf_u,
                      &m->pf_st, &m->pf_z, &m->pf_yn, &m->pf_sfb, &m->pf_send, &m->pf_pa, &m->pf_pb};
    for (float** b : bufs)
        if (*b) {
            (void)hipFree(*b);
            for (auto it = m->allocs.begin(); it != m->allocs.end(); ++it)
                if (*it == *b) { m->allocs.erase(it); break; }
            *b = nullptr;
        }
    if (m->pf_tok) {
        (void)hipFree(m->pf_tok);
        for (auto it = m->allocs.begin(); it != m->allocs.end(); ++it)
            if (*it == m->pf_tok) { m->allocs.erase(it); break; }
        m->pf_tok = nullptr;
    }
    const size_t rows = (size_t)m->max_batch * chunk, D = m->D, I = m->I, R = m->R;
    m->pf_x = dalloc<float>(m, rows * D);
    m->pf_raw = dalloc<float>(m, rows * D);
    m->pf_at = dalloc<float>(m, rows * D);
    m->pf_v = dalloc<float>(m, rows * R);
    m->pf_q = dalloc<float>(m, rows * 2 * D);
    m->pf_u = dalloc<float>(m, rows * D);
    m->pf_st = dalloc<float>(m, rows * D);
    m->pf_z = dalloc<float>(m, rows * I);
    m->pf_yn = dalloc<float>(m, rows * I);
    m->pf_sfb = dalloc<float>(m, rows * D);
    m->pf_send = dalloc<float>(m, (size_t)m->max_batch * D);
    // scan inputs of the small-batch path (kSplitScanChannels)
    const size_t prow = (size_t)m->max_batch * D <= kSplitScanChannels ? rows * D : 1;
    m->pf_pa = dalloc<float>(m, prow);
    m->pf_pb = dalloc<float>(m, prow);
    m->pf_tok = dalloc<int32_t>(m, rows);
    for (float** b : bufs)
        if (!*b) { m->pf_chunk = 0; set_last_error("out of device memory (prefill)"); return SNHIP_E_NOMEM; }
    if (!m->pf_tok) { m->pf_chunk = 0; return SNHIP_E_NOMEM; }
    m->pf_chunk = chunk;
    return SNHIP_OK;
}

// One chunk of Tc tokens for sequences [0, B), all layers, carrying s and
// hist. Tokens already in m->pf_tok (B x Tc). If logits_out, also the last
// token's logits. If all_logits, the logits of every token of the chunk go to
// all_logits (B, T, vocab) at positions [c0, c0 + Tc) of each sequence (the
// reference's forward, model.py:89-111, returns them for every position).
snhip_status enqueue_prefill_chunk(SnHipModel* m, int B, int Tc, float* logits_out,
                                   hipStream_t st, float* all_logits = nullptr, int T = 0,
                                   int c0 = 0) {
    const int D = m->D, I = m->I, R = m->R, L = m->L;
    const long rows = (long)B * Tc;
    const size_t sbs = (size_t)L * D;
    const size_t hbs = (size_t)L * (m->kh ? m->kh : 1) * D;
    snhip_status rc;
    hipLaunchKernelGGL(k_gather_embed, dim3((unsigned)rows), dim3(256), 0, st, m->pf_tok, m->embed,
                       m->pf_x, D, m->vocab);
    for (int l = 0; l < L; ++l) {
        const Layer& A = m->layers[l];
        float* s_l = m->s + (size_t)l * D;
        float* h_l = m->hist + (size_t)l * (m->kh ? m->kh : 1) * D;
        launch_ln((int)rows, m->pf_x, D, A.ni_g, A.ni_c, m->pf_raw, D, D, m->eps, st);
        const float* at = m->pf_raw;
        if (m->K > 1) {
            const long n = rows * D;
            hipLaunchKernelGGL(k_conv_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                               m->pf_raw, h_l, hbs, A.dw, m->pf_at, B, Tc, D, m->K);
            hipLaunchKernelGGL(k_hist_update, dim3((unsigned)(((long)B * D + 255) / 256)), dim3(256),
                               0, st, m->pf_raw, h_l, hbs, B, Tc, D, m->kh);
            at = m->pf_at;
        }
        if ((rc = run_gemm(m, gemm_for(m, A.V, at, D, (int)rows, m->pf_v, R), st)) != SNHIP_OK) return rc;
        if ((rc = run_gemm(m, gemm_for(m, A.U, m->pf_v, R, (int)rows, m->pf_q, 2 * D), st)) != SNHIP_OK) return rc;
        if ((size_t)m->max_batch * D <= kSplitScanChannels) {
            // Few channels: the gates of every row in parallel, then a scan
            // that only multiplies and adds.
            const long n = rows * D;
            hipLaunchKernelGGL(k_gate_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, m->pf_q,
                               A.delta, m->pf_u, m->pf_pa, m->pf_pb, n, D, m->clamp, m->p_floor);
            hipLaunchKernelGGL((k_scan_rows<16, 16>), dim3((unsigned)(B * (D / 64))), dim3(1024), 0, st,
                               m->pf_pa, m->pf_pb, s_l, sbs, m->pf_send, (size_t)D, m->pf_st, Tc, D);
        } else {
            hipLaunchKernelGGL((k_core_scan<4, 16>), dim3((unsigned)(B * (D / 64))), dim3(256), 0, st,
                               m->pf_q, A.delta, s_l, sbs, m->pf_send, (size_t)D, m->pf_u, m->pf_st,
                               Tc, D, m->clamp, m->p_floor);
        }
        GemmArgs gz = gemm_for(m, A.Wz, m->pf_u, D, (int)rows, m->pf_z, I);
        gz.epi = GEPI_WEDGE;
        gz.a_tanh = A.a_tanh;
        if ((rc = run_gemm(m, gz, st)) != SNHIP_OK) return rc;
        launch_ln((int)rows, m->pf_z, I, A.nm_g, A.nm_c, m->pf_yn, I, I, m->eps, st);
        // sfb_t = W_eff s_{t-1}, with s_{-1} the carried state (layers.py:208-217,243-250)
        GemmArgs gs = gemm_for(m, A.Ws, m->pf_st, D, (int)rows, m->pf_sfb, D);
        gs.X0 = s_l; gs.ldx0 = (long)sbs; gs.shift_T = Tc;
        if ((rc = run_gemm(m, gs, st)) != SNHIP_OK) return rc;
        GemmArgs gc = gemm_for(m, A.Wc, m->pf_yn, I, (int)rows, m->pf_x, D);
        gc.epi = GEPI_RESID;
        gc.b_gain = A.b_gain;
        gc.s = m->pf_st; gc.lds = D;
        gc.sfb = m->pf_sfb; gc.ldf = D;
        if ((rc = run_gemm(m, gc, st)) != SNHIP_OK) return rc;
        hipLaunchKernelGGL(k_copy_rows, dim3(B), dim3(256), 0, st, m->pf_send, (long)D, s_l,
                           (long)sbs, D);
    }
    if (all_logits) {
        // Final norm of every row into pf_raw (free once the layers are done),
        // then the tied head over those rows. Chunk rows are (b, t) with t
        // fastest, so one product covers every sequence when the chunk is the
        // whole prompt; otherwise each sequence's Tc rows are one product.
        launch_ln((int)rows, m->pf_x, D, m->no_g, m->no_c, m->pf_raw, D, D, m->eps, st);
        const size_t V = (size_t)m->vocab;
        if (Tc == T) {
            if ((rc = run_gemm(m, gemm_for(m, m->head, m->pf_raw, D, (int)rows, all_logits, (long)V), st)) != SNHIP_OK)
                return rc;
        } else {
            for (int b = 0; b < B; ++b) {
                GemmArgs gh = gemm_for(m, m->head, m->pf_raw + (size_t)b * Tc * D, D, Tc,
                                       all_logits + ((size_t)b * T + c0) * V, (long)V);
                if ((rc = run_gemm(m, gh, st)) != SNHIP_OK) return rc;
            }
        }
    }
    if (logits_out) {
        hipLaunchKernelGGL(k_last_rows, dim3(B), dim3(256), 0, st, m->pf_x, m->x, Tc, D);
        if ((rc = enqueue_head(m, B, m->x, logits_out, false, st)) != SNHIP_OK) return rc;
    }
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// Chunked prefill of tokens (B, T) (row-major, device) from the current state;
// logits_out (B, vocab) gets the last token's logits, all_logits (B, T, vocab)
// every token's (either may be NULL).
snhip_status run_prefill(SnHipModel* m, const int32_t* tokens_dev, int B, int T,
                         float* logits_out, float* all_logits = nullptr) {
    if (!m->gemm_ok || m->D % 64) {
        set_last_error("chunked prefill needs dim % 64 == 0 and dim, inner, rank % 32 == 0");
        return SNHIP_E_UNSUPPORTED;
    }
    // 512-token chunks, longer for small batches so the products have at
    // least ~2048 rows (the workspace is sized for max_batch x chunk rows).
    int chunk = std::max(512, std::min(2048, 2048 / std::max(1, m->max_batch)));
    if (const char* e = getenv("SNHIP_PREFILL_CHUNK")) chunk = std::max(1, atoi(e));
    chunk = std::min(chunk, T);
    snhip_status rc = ensure_prefill_ws(m, chunk);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipEventRecord(m->ev_in, m->stream));
    SNHIP_CHECK(hipStreamWaitEvent(m->work, m->ev_in, 0));
    for (int c0 = 0; c0 < T; c0 += chunk) {
        const int Tc = std::min(chunk, T - c0);
        SNHIP_CHECK(hipMemcpy2DAsync(m->pf_tok, (size_t)Tc * sizeof(int32_t), tokens_dev + c0,
                                     (size_t)T * sizeof(int32_t), (size_t)Tc * sizeof(int32_t), B,
                                     hipMemcpyDeviceToDevice, m->work));
        rc = enqueue_prefill_chunk(m, B, Tc, c0 + Tc >= T ? logits_out : nullptr, m->work,
                                   all_logits, T, c0);
        if (rc != SNHIP_OK) return rc;
    }
    SNHIP_CHECK(hipEventRecord(m->ev_out, m->work));
    SNHIP_CHECK(hipStreamWaitEvent(m->stream, m->ev_out, 0));
    return SNHIP_OK;
}

// n_steps decode steps of sequences [0, B) in persistent launches on the
// internal stream (ordered like run_steps): B = 1 on the persist_wg grid, else
// (2 <= B <= mi_max) each sequence on its own mi_grid[B] workgroups of one
// launch. The first input tokens are in m->tok. greedy: out_tok (n_steps, B)
// receives each step's argmax tokens, fed to the next step; otherwise n_steps
// must be 1. logits (B, vocab, device), if not NULL, gets the last step's.
// The call returns once the launches have finished and reports an exchange
// time-out as SNHIP_E_DEVICE. Each workgroup writes its channels' state back
// after its own last wait, so a time-out can leave the sequences part-stepped:
// the handle then refuses steps until reset or set. *launch_failed is set when the
// first cooperative launch could not be queued at all (nothing ran).
snhip_status run_persist(SnHipModel* m, int B, int n_steps, bool greedy, int32_t* out_tok,
                         float* logits, bool* launch_failed) {
    constexpr int kMaxStepsPerLaunch = 1 << 20;   // keeps exchange epochs far from wrapping
    SNHIP_CHECK(hipEventRecord(m->ev_in, m->stream));
    SNHIP_CHECK(hipStreamWaitEvent(m->work, m->ev_in, 0));
    SNHIP_CHECK(hipMemsetAsync(m->perr, 0, sizeof(unsigned), m->work));
    PersistArgs a{};
    a.layers = m->dlayers;
    a.L = m->L; a.D = m->D; a.I = m->I; a.R = m->R; a.K = m->K; a.kh = m->kh;
    a.vocab = m->vocab; a.clamp = m->clamp; a.eps = m->eps; a.p_floor = m->p_floor;
    a.embed = m->embed; a.no_g = m->no_g; a.no_c = m->no_c;
    a.head = pmat(m->head);
    a.s = m->s; a.hist = m->hist;
    a.ring = m->pring; a.ex = m->pex; a.sx = m->psx; a.err = m->perr;
    a.greedy = greedy ? 1 : 0;
    a.spin_limit = m->persist_spin;
    a.stall = env_unsigned("SNHIP_PERSIST_STALL", 0, 0);
    a.ni = B;
    const int blk = persist_blk(m);
    const int grid = B == 1 ? m->persist_wg : B * m->mi_grid[B];
    for (int done = 0; done < n_steps;) {
        const int n = std::min(n_steps - done, kMaxStepsPerLaunch);
        // Epochs restart at 1 in every launch: clear the words of the last one.
        SNHIP_CHECK(hipMemsetAsync(m->pex, 0, 2 * (size_t)kPersistExWords * B * sizeof(unsigned long long), m->work));
        SNHIP_CHECK(hipMemsetAsync(m->psx, 0, (size_t)m->L * 2 * m->D * B * sizeof(unsigned long long), m->work));
        a.tok_in = done == 0 ? m->tok : out_tok + (size_t)(done - 1) * B;
        a.out_tok = greedy ? out_tok + (size_t)done * B : nullptr;
        a.logits = done + n == n_steps ? logits : nullptr;
        a.n_steps = n;
        const snhip_status rc = launch_decode_persist(a, grid, blk, m->work);
        if (rc != SNHIP_OK) {
            if (done == 0 && launch_failed) *launch_failed = true;
            return rc;
        }
        done += n;
    }
    SNHIP_CHECK(hipMemcpyAsync(m->h_err, m->perr, sizeof(unsigned), hipMemcpyDeviceToHost, m->work));
    SNHIP_CHECK(hipEventRecord(m->ev_out, m->work));
    SNHIP_CHECK(hipStreamWaitEvent(m->stream, m->ev_out, 0));
    SNHIP_CHECK(hipStreamSynchronize(m->work));
    return persist_status(m, B);
}

// Does a step of B >= 2 sequences run as B instances of the single-sequence
// persistent kernel in one launch?
bool uses_mi(const SnHipModel* m, int B) { return m->persist_wg > 0 && B >= 2 && B <= m->mi_max; }

// One step of sequences [0, B), B >= 2 (tokens in m->tok): the single-sequence
// persistent kernel on a slice of the grid per sequence when it takes B, else
// the per-kernel or batched step. A failed cooperative launch turns the
// persistent path for B >= 2 off and falls back.
snhip_status step_many(SnHipModel* m, int B, float* logits_out) {
    if (uses_mi(m, B)) {
        bool launch_failed = false;
        const snhip_status rc = run_persist(m, B, 1, false, nullptr, logits_out, &launch_failed);
        if (!launch_failed) return rc;
        m->mi_max = 0;
        (void)hipGetLastError();
    }
    return run_steps(m, B, logits_out, false, 1);
}

// One step of sequence 0 (tokens already in m->tok): the persistent kernel
// when enabled, else the captured per-kernel step. A failed cooperative launch
// turns the persistent path off for this handle and falls back.
snhip_status step_one(SnHipModel* m, float* logits_out) {
    if (m->persist_wg) {
        bool launch_failed = false;
        const snhip_status rc = run_persist(m, 1, 1, false, nullptr, logits_out, &launch_failed);
        if (!launch_failed) return rc;
        m->persist_wg = 0;
        (void)hipGetLastError();
    }
    return run_steps(m, 1, logits_out, false, 1);
}

bool tokens_ok(const SnHipModel* m, const int32_t* t, int n) {
    for (int i = 0; i < n; ++i)
        if (t[i] < 0 || t[i] >= m->vocab) return false;
    return true;
}

}  // namespace
}  // namespace snhip

using namespace snhip;

extern "C" {

SnHipModel* snhip_load(const char* path, int vocab, int dim, int inner, int rank, int taps,
                       int layers, int group, int tied) {
    return load_model(path, vocab, dim, inner, rank, taps, layers, group, tied, 1,
                      SNHIP_WEIGHTS_F32, 32);
}

SnHipModel* snhip_load_h(const char* path, int vocab, int dim, int inner, int rank, int taps,
                         int layers, int group, int tied) {
    return load_model(path, vocab, dim, inner, rank, taps, layers, group, tied, 1,
                      SNHIP_WEIGHTS_F16, 32);
}

SnHipModel* snhip_load_ex(const char* path, int vocab, int dim, int inner, int rank, int taps,
                          int layers, int group, int tied, int32_t max_batch,
                          int32_t weight_format, int32_t block) {
    return load_model(path, vocab, dim, inner, rank, taps, layers, group, tied, max_batch,
                      weight_format, block);
}

void snhip_free(SnHipModel* m) {
    if (!m) return;
    // Only this handle's work is waited for: its internal stream and the
    // caller's stream it was bound to (NULL = the null stream).
    if (m->work) (void)hipStreamSynchronize(m->work);
    (void)hipStreamSynchronize(m->stream);
    free_model(m);
}

void snhip_reset(SnHipModel* m) {
    if (!m) return;
    const size_t B = m->max_batch;
    (void)hipMemsetAsync(m->s, 0, B * m->L * m->D * sizeof(float), m->stream);
    (void)hipMemsetAsync(m->hist, 0, B * m->L * (m->kh ? m->kh : 1) * m->D * sizeof(float),
                         m->stream);
    (void)hipStreamSynchronize(m->stream);
    m->poisoned = 0;
}

int snhip_vocab(const SnHipModel* m) { return m ? m->vocab : 0; }
int snhip_ready(const SnHipModel* m) { return m && m->ready; }
int32_t snhip_max_batch(const SnHipModel* m) { return m ? m->max_batch : 0; }
int32_t snhip_persistent_grid(const SnHipModel* m) { return m ? m->persist_wg : 0; }

int32_t snhip_persistent_grid_batch(const SnHipModel* m, int32_t B) {
    if (!m || B < 1 || B > m->max_batch) return 0;
    if (B == 1) return m->persist_wg;
    return uses_mi(m, B) ? B * m->mi_grid[B] : 0;
}

int32_t snhip_batch_grid(const SnHipModel* m) { return m ? m->batch_wg : 0; }

snhip_status snhip_set_stream(SnHipModel* m, void* stream) {
    if (!m) return SNHIP_E_INVAL;
    m->stream = as_stream(stream);
    return SNHIP_OK;
}

snhip_status snhip_step_batch_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                  float* logits_dev) {
    if (!m || !tokens_dev || !logits_dev || B <= 0 || B > m->max_batch) return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    const snhip_status rc = put_tokens(m, tokens_dev, B, hipMemcpyDeviceToDevice);
    if (rc != SNHIP_OK) return rc;
    return B == 1 ? step_one(m, logits_dev) : step_many(m, B, logits_dev);
}

snhip_status snhip_step_batch(SnHipModel* m, const int32_t* tokens, int32_t B, float* logits) {
    if (!m || !tokens || !logits || B <= 0 || B > m->max_batch) return SNHIP_E_INVAL;
    if (!tokens_ok(m, tokens, B)) return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    snhip_status rc = put_tokens(m, tokens, B, hipMemcpyHostToDevice);
    if (rc == SNHIP_OK) rc = B == 1 ? step_one(m, m->logits) : step_many(m, B, m->logits);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipMemcpyAsync(logits, m->logits, (size_t)B * m->vocab * sizeof(float),
                               hipMemcpyDeviceToHost, m->stream));
    SNHIP_CHECK(hipStreamSynchronize(m->stream));
    return SNHIP_OK;
}

void snhip_step(SnHipModel* m, int token, float* logits) {
    if (!m || !logits) return;
    const int32_t t = token;
    (void)snhip_step_batch(m, &t, 1, logits);
}

snhip_status snhip_prefill_host(SnHipModel* m, const int32_t* tokens, int32_t n, float* logits) {
    if (!m || !tokens || n <= 0 || !logits) return SNHIP_E_INVAL;
    if (!tokens_ok(m, tokens, n)) return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    int32_t* dt = nullptr;
    SNHIP_CHECK(hipMalloc(&dt, (size_t)n * sizeof(int32_t)));
    snhip_status rc = SNHIP_OK;
    if (hipMemcpy(dt, tokens, (size_t)n * sizeof(int32_t), hipMemcpyHostToDevice) != hipSuccess) {
        set_last_error("prefill: token copy failed");
        rc = SNHIP_E_DEVICE;
    } else if (m->gemm_ok && m->D % 64 == 0) {
        rc = run_prefill(m, dt, 1, n, m->logits);
    } else {
        for (int i = 0; i < n && rc == SNHIP_OK; ++i) {   // the reference's step loop (sunnynet.c:347-349)
            rc = put_tokens(m, dt + i, 1, hipMemcpyDeviceToDevice);
            if (rc == SNHIP_OK) rc = run_steps(m, 1, m->logits, false, 1);
        }
    }
    if (rc == SNHIP_OK &&
        hipMemcpyAsync(logits, m->logits, (size_t)m->vocab * sizeof(float), hipMemcpyDeviceToHost,
                       m->stream) != hipSuccess) {
        set_last_error("prefill: logits copy failed");
        rc = SNHIP_E_DEVICE;
    }
    (void)hipStreamSynchronize(m->stream);
    (void)hipFree(dt);
    return rc;
}

void snhip_prefill(SnHipModel* m, const int* tokens, int n, float* logits) {
    (void)snhip_prefill_host(m, tokens, n, logits);
}

snhip_status snhip_prefill_batch_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                     int32_t T, float* logits_dev) {
    if (!m || !tokens_dev || B <= 0 || B > m->max_batch || T <= 0) return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    return run_prefill(m, tokens_dev, B, T, logits_dev);
}

snhip_status snhip_dbg_layer(SnHipModel* m, int32_t token, int32_t layer, float* dbg) {
    if (!m || !dbg || layer < 0 || layer >= m->L || token < 0 || token >= m->vocab) return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    const int D = m->D, I = m->I, R = m->R;
    const size_t hbs = (size_t)m->L * (m->kh ? m->kh : 1) * D;
    hipStream_t st = m->work;
    SNHIP_CHECK(hipEventRecord(m->ev_in, m->stream));
    SNHIP_CHECK(hipStreamWaitEvent(st, m->ev_in, 0));
    SNHIP_CHECK(hipMemcpyAsync(m->tok, &token, sizeof(int32_t), hipMemcpyHostToDevice, st));
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, st, m->tok, m->embed, m->x, D, m->vocab);
    for (int l = 0; l <= layer; ++l) {
        const Layer& A = m->layers[l];
        float* h_l = m->hist + (size_t)l * (m->kh ? m->kh : 1) * D;
        // the layer's input x is needed for the dump's residual: the GEMV
        // step adds it in W_c's epilogue, in place
        launch_ln_conv(1, m->x, A.ni_g, A.ni_c, A.dw, h_l, hbs, m->at, D, m->K, m->eps, st);
        const snhip_status rc = enqueue_layer_gemv(m, 1, l, st);
        if (rc != SNHIP_OK) return rc;
    }
    // sunnynet.c:278-289: raw, at, v, gate, u, s', z (after the wedge), yn, sfb, out.
    // q = U v holds its rows in the qrow_u / qrow_g order: the gates are
    // gathered back to channel order on the host.
    struct Part { const float* src; int n; };
    const float* raw = m->K > 1 ? m->hist + (size_t)layer * m->kh * D : m->at;
    std::vector<float> q(2 * (size_t)D);
    const Part parts[] = {{raw, D}, {m->at, D}, {m->v, R}, {nullptr, D}, {m->u, D},
                          {m->s + (size_t)layer * D, D}, {m->z, I}, {m->yn, I}, {m->sfb, D},
                          {m->x, D}};
    SNHIP_CHECK(hipMemcpyAsync(q.data(), m->q, q.size() * sizeof(float), hipMemcpyDeviceToHost, st));
    float* out = dbg;
    float* gate = nullptr;
    for (const Part& pt : parts) {
        if (pt.src) SNHIP_CHECK(hipMemcpyAsync(out, pt.src, (size_t)pt.n * sizeof(float), hipMemcpyDeviceToHost, st));
        else gate = out;
        out += pt.n;
    }
    SNHIP_CHECK(hipStreamSynchronize(st));
    for (int i = 0; i < D; ++i) gate[i] = q[qrow_g(i)];
    return SNHIP_OK;
}

snhip_status snhip_prefill_all_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                   int32_t T, float* logits_all_dev) {
    if (!m || !tokens_dev || !logits_all_dev || B <= 0 || B > m->max_batch || T <= 0)
        return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    return run_prefill(m, tokens_dev, B, T, nullptr, logits_all_dev);
}

snhip_status snhip_decode_greedy_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                     int32_t n_steps, int32_t* out_tokens_dev,
                                     float* logits_dev) {
    if (!m || !tokens_dev || !out_tokens_dev || B <= 0 || B > m->max_batch || n_steps <= 0)
        return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    if (B == 1 && m->persist_wg) {
        snhip_status rc = put_tokens(m, tokens_dev, 1, hipMemcpyDeviceToDevice);
        if (rc != SNHIP_OK) return rc;
        bool launch_failed = false;
        rc = run_persist(m, 1, n_steps, true, out_tokens_dev, logits_dev, &launch_failed);
        if (!launch_failed) return rc;
        m->persist_wg = 0;
        (void)hipGetLastError();
    }
    if (uses_mi(m, B)) {
        snhip_status rc = put_tokens(m, tokens_dev, B, hipMemcpyDeviceToDevice);
        if (rc != SNHIP_OK) return rc;
        bool launch_failed = false;
        rc = run_persist(m, B, n_steps, true, out_tokens_dev, logits_dev, &launch_failed);
        if (!launch_failed) return rc;
        m->mi_max = 0;
        (void)hipGetLastError();
    }
    if ((long)n_steps * B > (long)m->hist_cap || !m->tok_hist) {
        // Grow the token history; graphs bake its address, so drop them.
        SNHIP_CHECK(hipStreamSynchronize(m->stream));
        SNHIP_CHECK(hipStreamSynchronize(m->work));
        for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
        m->graphs.clear();
        long cap = 256L * m->max_batch;
        while (cap < (long)n_steps * B) cap *= 2;
        if (cap > (1L << 30)) return SNHIP_E_INVAL;
        int32_t* h = nullptr;
        SNHIP_CHECK(hipMalloc(&h, (size_t)cap * sizeof(int32_t)));
        if (m->tok_hist) {
            (void)hipFree(m->tok_hist);
            for (auto it = m->allocs.begin(); it != m->allocs.end(); ++it)
                if (*it == m->tok_hist) { m->allocs.erase(it); break; }
        }
        m->tok_hist = h;
        m->allocs.push_back(h);
        m->hist_cap = (int)cap;
    }
    snhip_status rc = put_tokens(m, tokens_dev, B, hipMemcpyDeviceToDevice);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipMemsetAsync(m->counter, 0, sizeof(int32_t), m->stream));
    float* lg = logits_dev ? logits_dev : m->logits;
    rc = run_steps(m, B, lg, true, n_steps);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipMemcpyAsync(out_tokens_dev, m->tok_hist, (size_t)n_steps * B * sizeof(int32_t),
                               hipMemcpyDeviceToDevice, m->stream));
    return SNHIP_OK;
}

snhip_status snhip_get_state_dev(SnHipModel* m, float* s_dev, float* hist_dev, int32_t B) {
    if (!m || !s_dev || B <= 0 || B > m->max_batch || (m->kh && !hist_dev)) return SNHIP_E_INVAL;
    SNHIP_CHECK(hipMemcpyAsync(s_dev, m->s, (size_t)B * m->L * m->D * sizeof(float),
                               hipMemcpyDeviceToDevice, m->stream));
    if (m->kh)
        SNHIP_CHECK(hipMemcpyAsync(hist_dev, m->hist, (size_t)B * m->L * m->kh * m->D * sizeof(float),
                                   hipMemcpyDeviceToDevice, m->stream));
    return SNHIP_OK;
}

snhip_status snhip_set_state_dev(SnHipModel* m, const float* s_dev, const float* hist_dev,
                                 int32_t B) {
    if (!m || !s_dev || B <= 0 || B > m->max_batch || (m->kh && !hist_dev)) return SNHIP_E_INVAL;
    SNHIP_CHECK(hipMemcpyAsync(m->s, s_dev, (size_t)B * m->L * m->D * sizeof(float),
                               hipMemcpyDeviceToDevice, m->stream));
    if (m->kh)
        SNHIP_CHECK(hipMemcpyAsync(m->hist, hist_dev, (size_t)B * m->L * m->kh * m->D * sizeof(float),
                                   hipMemcpyDeviceToDevice, m->stream));
    if (B >= m->poisoned) m->poisoned = 0;
    return SNHIP_OK;
}

}  // extern "C"
