// RWKV-7 decode step for one sequence (or one per equal slice of the grid) as
// one cooperative launch, rounded in the reference's order
// (sunnynet/runtime/rwkv7.c:127-360), so that a step gives the reference's
// bits. The phases, exchange words, waits and the ordering of the shift
// vectors' rewrites are rkpersist.hip's:
//
//   P1  LN_1 + token-shift mixes (every workgroup), then the rows of W_r,
//       W_k, W_v and the LoRA down-projections W_1 (tanh), A_1, G_1
//       (sigmoid), V_1;
//   P2  workgroup h < n_head: the LoRA up-projections of head h's 64
//       channels, then decay, value residual, in-context rate, the 64 x 64
//       state update, read-out, group norm, bonus and gate -> y of head h;
//   P3  rows of W_o, x_a = x + W_o y;
//   P4  LN_2 + channel-mix input (every workgroup), rows of W_ck, relu^2;
//   P5  rows of W_cv, x_b = x_a + W_cv ck;
//
// then LN_out, the vocabulary rows with per-workgroup argmax keys, and every
// workgroup reduces the keys to the greedy token.
//
// What follows the reference's rounding:
// * Products. Every output is one thread's sequential chain over the inputs
//   from 0, acc = fmaf(x[i], W[i][j], acc), as the reference's GEMV computes
//   it. The layer matrices are read from fp32 copies in (output, input) rows
//   made at load (INT4 rows dequantized to (q - 8) s, the values the
//   reference multiplies), four inputs per global read and per LDS broadcast
//   read of x; outputs past the last multiple of 8 take the reference's
//   scalar tail (acc + x w, two roundings). The vocabulary rows stay INT4
//   and are dequantized in the chain as fma(q, s, -8 s).
// * LayerNorm: one thread's sequential sums (sum, then squared deviations),
//   (x - mean) rstd g + c.
// * The head owners' math is the reference's per head: eight stride-8
//   partial sums folded ((0+4)+(1+5))+((2+6)+(3+7)) for |kk| and the state
//   dots, sequential sums for the group norm and the bonus.
// * expf / tanhf / sigmoid are refmath.h's (glibc's algorithms).
//
// A phase's latency is one chain of K dependent FMAs (K = 768 for the
// model-width products, 3072 for the channel-mix value): rows go one per
// thread, so a workgroup's rows of a product run side by side.
#include <type_traits>

#include "gemv.h"
#include "lanesum.h"
#include "refmath.h"
#include "rkpersist.h"
#include "rkxch.h"

namespace snhip {
namespace {
using namespace rkx;

// One wave per SIMD (four per workgroup): each wave then has the SIMD's 512
// registers, and values that do not fit the 256 VGPRs go to AGPRs instead of
// scratch memory (a scratch reload waits for every vector load in flight,
// the prefetched weights included).
constexpr int NT = 256, NW = NT / 64, HS = 64;
constexpr float kR2 = 0.6065306597126334f;   // 1/sqrt(e), rwkv7.c:38
constexpr float kEpsGroup = 6.4e-4f;          // rwkv7.c:39
constexpr int kPer = kRkPMaxD / NT;           // model-width words per thread
constexpr int kPerF = kRkPMaxF / NT;          // channel-mix key words per thread
constexpr int kSRow = HS + 4;                 // LDS row of a head's state (floats)
constexpr int kSPer = HS * HS / 4 / NT;       // state float4 per thread
static_assert(HS * kSRow <= 6 * kRkPMaxD, "a head's state fits buf");

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> glb(const T* p) { return (gptr<T>)p; }
// A pointer every lane holds alike, as a wave-uniform (scalar) value: read
// once from the LDS layer table, not again for every load it bases.
__device__ __forceinline__ const float* uni(const float* p) {
    const unsigned long long v = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (const float*)(((unsigned long long)hi << 32) | lo);
}
// A weight read that is used once per step: non-temporal, so that the
// step's stream of weights does not push the kernel's code, its exchange
// words and the state out of the L2.
__device__ __forceinline__ f4 stream_ld(gptr<f4> p) { return __builtin_nontemporal_load(p); }
// LDS reads through an LDS-typed pointer: ds_read (counted by lgkmcnt only),
// so waiting for x does not also wait for the weight reads in flight.
typedef __attribute__((address_space(3))) const f4 l_f4;
__device__ __forceinline__ const l_f4* lds4(const float* p) { return (const l_f4*)p; }
// The same pointer with its whole address in a vector register, for loops of
// reads through a pointer every lane holds alike: from a wave-uniform base the
// compiler rebuilds every read's address (two moves, or an add when the base
// is past 64 KB and does not fit the reads' offset field).
__device__ __forceinline__ const l_f4* vaddr(const l_f4* p) {
    uint32_t a = (uint32_t)(size_t)p;
    asm volatile("" : "+v"(a));
    return (const l_f4*)(size_t)a;
}

// One wave runs each chain below, so the wave's instruction issue bounds it:
// a dependent VALU op every ~5.4 clocks, and every ds_read_b128 takes issue
// time of its own (measured on gfx950: a chain fed from LDS ran 25 clocks per
// FMA with a clamped eight-deep window whose reads the compiler regrouped,
// 10 with the ring below). The rings keep a fixed number of windows in
// flight, read without clamps (every LDS buffer a chain reads has kPad
// floats of slack past its end), and scheduling barriers keep the compiler
// from regrouping the reads.
constexpr int kPad = 32;

// sum = sum + v[i] over n4 float4 in element order: windows of 8 float4, one
// in flight ahead of the one in use (reads reach 8 float4 past the last
// multiple of 16).
__device__ __forceinline__ float seq_sum(const l_f4* v, int n4) {
    constexpr int W = 8;
    v = vaddr(v);
    f4 r[2][W];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < W; ++j) r[0][j] = v[j];
    const int n16 = n4 & ~15;
    for (int g = 0; g < n16; g += 2 * W) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < W; ++j) r[h ^ 1][j] = v[g + (h + 1) * W + j];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < W; ++j) {
                s = s + r[h][j].x; s = s + r[h][j].y; s = s + r[h][j].z; s = s + r[h][j].w;
            }
        }
    }
    for (int k = n16; k < n4; ++k) {
        const f4 b = v[k];
        s = s + b.x; s = s + b.y; s = s + b.z; s = s + b.w;
    }
    return s;
}

// acc = fmaf(x[i], w[i], acc) over n4 float4 of w and x, both in LDS, in input
// order: windows of 2 float4 of each, three in flight ahead of the one in use
// (twelve reads outstanding; reads reach 6 float4 past the last multiple of 8).
__device__ __forceinline__ float lds_chain(const l_f4* w, const l_f4* x, int n4, float acc) {
    constexpr int W = 2, AH = 3, NS = AH + 1;
    x = vaddr(x);   // x may be the same for every lane
    f4 wr[NS][W], xr[NS][W];
#pragma unroll
    for (int a = 0; a < AH; ++a)
#pragma unroll
        for (int j = 0; j < W; ++j) {
            wr[a][j] = w[a * W + j];
            xr[a][j] = x[a * W + j];
        }
    const int n8 = n4 & ~(NS * W - 1);
    for (int g = 0; g < n8; g += NS * W) {
#pragma unroll
        for (int h = 0; h < NS; ++h) {
            const int nx = (h + AH) % NS;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < W; ++j) {
                wr[nx][j] = w[g + (h + AH) * W + j];
                xr[nx][j] = x[g + (h + AH) * W + j];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < W; ++j) {
                acc = fmaf(xr[h][j].x, wr[h][j].x, acc);
                acc = fmaf(xr[h][j].y, wr[h][j].y, acc);
                acc = fmaf(xr[h][j].z, wr[h][j].z, acc);
                acc = fmaf(xr[h][j].w, wr[h][j].w, acc);
            }
        }
    }
    for (int k = n8; k < n4; ++k) {
        const f4 wv = w[k], xv = x[k];
        acc = fmaf(xv.x, wv.x, acc);
        acc = fmaf(xv.y, wv.y, acc);
        acc = fmaf(xv.z, wv.z, acc);
        acc = fmaf(xv.w, wv.w, acc);
    }
    return acc;
}

// A LayerNorm's gains and biases for this thread's elements k NT + tid,
// loaded ahead of the values (a phase issues them before its wait).
struct LnP {
    float g[kPer], c[kPer];
};
__device__ __forceinline__ void ln_load(LnP& p, const float* g, const float* c, int n) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = min(k * NT + (int)threadIdx.x, n - 1);
        p.g[k] = g[i];
        p.c[k] = c[i];
    }
}

// LN statistics of n = 256 KL4 values in LDS by wave 0, lane-sliced
// (lanesum.h): the values stay in registers for both sums.
template <int KL4>
__device__ __forceinline__ void ln_stats_lanes(const float* src, int n, float eps, float* stat) {
    const int lane = threadIdx.x & 63;
    float v[4 * KL4];
#pragma unroll
    for (int q = 0; q < KL4; ++q) {
        const f4 x = lds4(src)[lane * KL4 + q];
        v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
    }
    float mean, rstd;
    lane_ln_stats(v, n, eps, mean, rstd);
    if (lane == 0) {
        stat[0] = mean;
        stat[1] = rstd;
    }
}

// dst = LN(src) g + c over n <= kRkPMaxD values in LDS (rwkv7.c:127-140):
// the mean and the variance as sequential sums (by wave 0 lane-sliced when
// n is 256, 512, 768 or 1024, else by thread 0). sq: n floats of LDS scratch.
__device__ __forceinline__ void ln_exact(const float* src, float* dst, float* sq, const LnP& p, int n, float eps,
                                         float* stat) {
    const int t = threadIdx.x;
    const int kl = n % 256 ? 0 : n / 256;
    if (kl >= 1 && kl <= 4) {
        if (t < 64) {
            if (kl == 1) ln_stats_lanes<1>(src, n, eps, stat);
            else if (kl == 2) ln_stats_lanes<2>(src, n, eps, stat);
            else if (kl == 3) ln_stats_lanes<3>(src, n, eps, stat);
            else ln_stats_lanes<4>(src, n, eps, stat);
        }
        __syncthreads();
    } else {
        if (t == 0) stat[0] = seq_sum(lds4(src), n >> 2) / (float)n;
        __syncthreads();
        const float m0 = stat[0];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int i = k * NT + t;
            if (i < n) {
                const float d = src[i] - m0;
                sq[i] = d * d;
            }
        }
        __syncthreads();
        if (t == 0) stat[1] = 1.0f / sqrtf(seq_sum(lds4(sq), n >> 2) / (float)n + eps);
        __syncthreads();
    }
    const float mean = stat[0], rstd = stat[1];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = k * NT + t;
        if (i < n) dst[i] = (src[i] - mean) * rstd * p.g[k] + p.c[k];
    }
    __syncthreads();
}

// ---- products with the weights staged through LDS
//
// A product phase's rows on this workgroup (R of them, K inputs each, fp32
// (output, input) rows) are multiplied as R chains, thread r < R running row
// r in input order, acc = fmaf(x[i], w[i], acc) (rows past the matrix's last
// multiple of 8: acc + x w). The weights reach the chains through LDS. When
// the phase's rows fit the threads' two register slots, the whole phase is
// loaded before the phase waits for its input (the weights do not depend on
// it) and stored with one barrier, rows padded to K + 4 floats; the chains
// then run without barriers. Otherwise they come in chunks of C inputs:
// every thread of the workgroup loads part of a chunk (coalesced four-float
// reads along the rows) into registers, two chunks ahead, and stores it into
// one of two LDS buffers once the chunk before it is in use; rows are padded
// to C + 4 floats so the chains' reads spread over the banks. The first two
// chunks are issued before the wait.
constexpr int kStg = 12288;                    // floats per LDS buffer (two: 96 KB)
constexpr int kPend = 6;                       // float4 per thread per chunk, at most
constexpr int kMaxStageRows = kPend * NT * 4 / 32;   // rows one chunk of 32 inputs can hold

struct Pend {
    f4 v[2][kPend];
};

// Chunk width for R <= kMaxStageRows rows: the widest of 256 / 128 / 64 / 32
// inputs whose chunk fits the threads' registers and whose padded rows fit
// one buffer.
__device__ __forceinline__ int chunk_for(int R) {
    auto fits = [&](int C) { return R * C <= 4 * kPend * NT && R * (C + 4) <= kStg; };
    return fits(256) ? 256 : fits(128) ? 128 : fits(64) ? 64 : 32;
}

// Whole-phase staging: R rows of K inputs fit, padded, the two LDS buffers.
__device__ __forceinline__ bool whole_fits(int R, int K) { return R * (K + 4) <= 2 * kStg; }

// Row and float4 column of float4 element i (i < 2 kStg / 4) of rows of C4
// float4: a float reciprocal, then one correction step (the quotient is off
// by less than 1).
__device__ __forceinline__ void split(int i, int C4, float inv, int& r, int& c4) {
    r = (int)((float)i * inv);
    c4 = i - r * C4;
    const int adj = (int)(c4 >= C4) - (int)(c4 < 0);   // no branch
    r += adj;
    c4 -= adj * C4;
}

// One product phase's staging plan (uniform values). A chunk is C4 float4 of
// each row, stored in LDS at row stride RS floats. Whole phase: one chunk of
// K4 float4, loaded straight into LDS from stg on (whole_issue_lds);
// chunked: register slot s holds chunk ch with ch & 1 == s, stored into
// buffer s.
struct Stager {
    int R, K4, C4, RS, nch;
    float inv;
    bool whole;
};
__device__ __forceinline__ Stager stager(int R, int K) {
    Stager S;
    S.R = R;
    S.K4 = K >> 2;
    S.whole = whole_fits(R, K);
    S.C4 = S.whole ? S.K4 : chunk_for(R) >> 2;
    S.RS = 4 * S.C4 + 4;
    S.nch = (S.K4 + S.C4 - 1) / S.C4;
    S.inv = 1.0f / (float)S.C4;
    return S;
}

// The whole phase straight into LDS: float4 slot q of the padded rows (row q
// / (K4 + 1), column q % (K4 + 1); the pad column loads the row's last float4
// again) by global_load_lds, whose 64 lanes write 64 consecutive slots from a
// wave-uniform base. No registers hold the weights and no pass stores them;
// the data is in LDS once the loads retire (vmcnt). The caller's barrier
// before it: every wave is done with stg.
template <class WR>
__device__ __forceinline__ void whole_issue_lds(float* stg, const Stager& S, WR&& wrow) {
    typedef const __attribute__((address_space(1))) void gvoid;
    typedef __attribute__((address_space(3))) void lvoid;
    const int W4 = S.K4 + 1, n = S.R * W4, tid = threadIdx.x;
    const float inv = 1.0f / (float)W4;
    // unrolled: the loop's back edge made the compiler copy ~20 live
    // registers per trip
#pragma unroll 8
    for (int base = 0; base < n; base += NT) {
        const int q = base + tid;
        if (q < n) {
            int r, c4;
            split(q, W4, inv, r, c4);
            const gptr<f4> src = wrow(r) + min(c4, S.K4 - 1);
            __builtin_amdgcn_global_load_lds((gvoid*)src, (lvoid*)(stg + 4 * (base + (tid & ~63))), 16, 0, 0);
        }
    }
}

// Issues chunk ch into register slot SLOT (row r from wrow(r), a float4
// pointer). The slots are compile-time indices and no branch selects among
// layouts, so no register of a load in flight is copied (a copy waits for
// the load).
template <int SLOT, class WR>
__device__ __forceinline__ void stg_issue(Pend& P, const Stager& S, int ch, WR&& wrow) {
    const int first = 0, n = S.R * S.C4, col0 = ch * S.C4;
#pragma unroll
    for (int p = 0; p < kPend; ++p) {
        const int i = first + (int)threadIdx.x + p * NT;
        if (i < n) {
            int r, c4;
            split(i, S.C4, S.inv, r, c4);
            P.v[SLOT][p] = stream_ld(wrow(r) + min(col0 + c4, S.K4 - 1));
        }
    }
}

// Stores register slot SLOT into LDS from b on (rows at stride S.RS).
template <int SLOT>
__device__ __forceinline__ void stg_commit(const Pend& P, const Stager& S, float* b) {
    const int first = 0, n = S.R * S.C4;
#pragma unroll
    for (int p = 0; p < kPend; ++p) {
        const int i = first + (int)threadIdx.x + p * NT;
        if (i < n) {
            int r, c4;
            split(i, S.C4, S.inv, r, c4);
            const f4 v = P.v[SLOT][p];
            *reinterpret_cast<float4*>(b + r * S.RS + 4 * c4) = make_float4(v.x, v.y, v.z, v.w);
        }
    }
}

// The same with the reference's scalar tail (acc + x w) for rows the caller
// marks: those rows run their chain again from the fp32 rows in global
// memory. (No model shape here has such rows: every output count is a
// multiple of 8; the branch keeps other shapes exact.)
__device__ __forceinline__ float tail_chain(const float* W, int K, int row, const float* x) {
    const gptr<float> w = glb(W) + (size_t)row * K;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) acc = acc + x[k] * w[k];
    return acc;
}

// Issue: the whole phase (into stg), or its first two chunks (before the
// caller's wait).
template <class WR>
__device__ __forceinline__ void stager_issue(Pend& P, float* stg, const Stager& S, WR&& wrow) {
    if (S.whole) {
        __syncthreads();
        whole_issue_lds(stg, S, wrow);
        return;
    }
    stg_issue<0>(P, S, 0, wrow);
    if (S.nch > 1) stg_issue<1>(P, S, 1, wrow);
}

// Run, after the caller's wait: thread r < R ends with row r's sum and calls
// out(r, v); xrow(r): row r's input vector in LDS.
template <class WR, class XR, class OUT>
__device__ __forceinline__ void stager_run(Pend& P, float* stg, const Stager& S, WR&& wrow, XR&& xrow, OUT&& out) {
    const int t = threadIdx.x;
    const bool mine = t < S.R;
    const l_f4* x = lds4(mine ? xrow(t) : xrow(0));
    if (S.whole) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's loads into LDS
        __syncthreads();
        if (mine) out(t, lds_chain(lds4(stg + t * S.RS), x, S.K4, 0.0f));
        return;
    }
    float acc = 0.0f;
    // chunk ch: slot and buffer ch & 1
    auto one = [&](int ch, auto slot) {
        constexpr int SL = decltype(slot)::value;
        float* b = stg + SL * kStg;
        stg_commit<SL>(P, S, b);
        if (ch + 2 < S.nch) stg_issue<SL>(P, S, ch + 2, wrow);
        __syncthreads();
        if (mine) acc = lds_chain(lds4(b + t * S.RS), x + ch * S.C4, min(S.C4, S.K4 - ch * S.C4), acc);
    };
    for (int ch = 0; ch < S.nch; ch += 2) {
        one(ch, std::integral_constant<int, 0>{});
        if (ch + 1 < S.nch) one(ch + 1, std::integral_constant<int, 1>{});
    }
    if (mine) out(t, acc);
}

// ---- lane-sliced chains (a phase with no more rows than waves)
//
// Wave r runs row r; lane j holds inputs [4 KL4 j, 4 KL4 (j + 1)) of the row
// (loaded before the phase's wait) and of x (from LDS) in registers. Every
// lane runs its 4 KL4 FMAs from the running sum of the inputs before, and
// the sum passes from lane j to lane j + 1 as a wave-uniform value: the
// chain keeps input order, acc = fmaf(x[i], w[i], acc), with no LDS read
// between two FMAs (about half the time per FMA of the staged chains).
template <int KL4>
struct LscRow {
    f4 w[KL4 > 0 ? KL4 : 1];
};

// KL4 for a phase of R rows of K inputs: K / 256 when this build has that
// instance, 0 (staged chains) otherwise.
__device__ __forceinline__ int lsc_kl(int R, int K) {
    if (R > NW || K % 256) return 0;
    const int kl = K / 256;
    return kl == 2 || kl == 3 || kl == 4 || kl == 8 || kl == 12 || kl == 16 ? kl : 0;
}

template <int KL4, class WR>
__device__ __forceinline__ void lsc_issue(LscRow<KL4>& W, int R, WR&& wrow) {
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wv < R) {
        const gptr<f4> w = wrow(wv) + lane * KL4;
#pragma unroll
        for (int q = 0; q < KL4; ++q) W.w[q] = stream_ld(w + q);
    }
}

template <int KL4>
__device__ __forceinline__ float lsc_run(const LscRow<KL4>& W, const l_f4* x) {
    const int lane = threadIdx.x & 63;
    f4 xv[KL4];
#pragma unroll
    for (int q = 0; q < KL4; ++q) xv[q] = x[lane * KL4 + q];
    float acc = 0.0f;
    for (int j = 0; j < 64; ++j) {
        float a = acc;
#pragma unroll
        for (int q = 0; q < KL4; ++q) {
            a = fmaf(xv[q].x, W.w[q].x, a);
            a = fmaf(xv[q].y, W.w[q].y, a);
            a = fmaf(xv[q].z, W.w[q].z, a);
            a = fmaf(xv[q].w, W.w[q].w, a);
        }
        acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), j));
    }
    return acc;
}

// One product phase of R rows of K inputs: `issue` (before the caller's
// wait) and `run` pick lane-sliced or staged chains; run calls out(r, v) once
// per row r < R. KL4: lsc_kl(R, K), dispatched by the caller.
template <int KL4>
struct Phase {
    LscRow<KL4> W;
    Stager S;
    template <class WR>
    __device__ __forceinline__ void issue(Pend& P, float* stg, int R, int K, WR&& wrow) {
        if constexpr (KL4 > 0) {
            S.R = R;
            lsc_issue(W, R, wrow);
        } else {
            S = stager(R, K);
            stager_issue(P, stg, S, wrow);
        }
    }
    template <class WR, class OUT>
    __device__ __forceinline__ void run(Pend& P, float* stg, const float* x, WR&& wrow, OUT&& out) {
        if constexpr (KL4 > 0) {
            const int wv = threadIdx.x >> 6;
            if (wv < S.R) {
                const float v = lsc_run(W, lds4(x));
                if ((threadIdx.x & 63) == 0) out(wv, v);
            }
        } else {
            stager_run(P, stg, S, wrow, [&](int) -> const float* { return x; }, out);
        }
    }
};

// Calls f(std::integral_constant<int, kl>) for kl = lsc_kl(R, K).
template <class F>
__device__ __forceinline__ auto with_kl(int kl, F&& f) {
    switch (kl) {
    case 2: return f(std::integral_constant<int, 2>{});
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 12: return f(std::integral_constant<int, 12>{});
    case 16: return f(std::integral_constant<int, 16>{});
    default: return f(std::integral_constant<int, 0>{});
    }
}

// The vocabulary rows, one per thread, read straight from global memory:
// fp32 rows four values per read with eight reads in flight; INT4 rows with
// group BLK (quant.c layout: byte j of a group holds values j and j + BLK/2)
// a group per step with four groups in flight, dequantized in the chain as
// fma(q, s, -8 s). Rows past the last multiple of 8 take acc + x w.
template <bool FUSED>
__device__ __forceinline__ float chain_f32(gptr<f4> w, const l_f4* x, int K4) {
    constexpr int PF = 8;
    x = vaddr(x);
    f4 a[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) a[j] = w[min(j, K4 - 1)];
    float acc = 0.0f;
    for (int q = 0; q < K4; q += PF) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const f4 wv = a[j];
            a[j] = w[min(q + PF + j, K4 - 1)];
            if (q + j < K4) {
                const f4 xv = x[q + j];
                if constexpr (FUSED) {
                    acc = fmaf(xv.x, wv.x, acc);
                    acc = fmaf(xv.y, wv.y, acc);
                    acc = fmaf(xv.z, wv.z, acc);
                    acc = fmaf(xv.w, wv.w, acc);
                } else {
                    acc = acc + xv.x * wv.x;
                    acc = acc + xv.y * wv.y;
                    acc = acc + xv.z * wv.z;
                    acc = acc + xv.w * wv.w;
                }
            }
        }
    }
    return acc;
}

template <int BLK, bool FUSED>
__device__ __forceinline__ float chain_i4(gptr<u4> q, gptr<float> sc, const l_f4* x, int ng) {
    x = vaddr(x);
    constexpr int NQ = BLK / 32;   // 16-byte reads per group
    constexpr int NP = 4;          // groups in flight
    u4 cb[NP][NQ];
    float sb[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int g = min(p, ng - 1);
#pragma unroll
        for (int k = 0; k < NQ; ++k) cb[p][k] = q[(size_t)g * NQ + k];
        sb[p] = sc[g];
    }
    float acc = 0.0f;
    for (int g0 = 0; g0 < ng; g0 += NP) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const int g = g0 + p;
            u4 cur[NQ];
#pragma unroll
            for (int k = 0; k < NQ; ++k) cur[k] = cb[p][k];
            const float s = sb[p];
            const int gn = min(g + NP, ng - 1);
#pragma unroll
            for (int k = 0; k < NQ; ++k) cb[p][k] = q[(size_t)gn * NQ + k];
            sb[p] = sc[gn];
            if (g < ng) {
                const float m8 = -8.0f * s;
                f4 xg[BLK / 4];
#pragma unroll
                for (int e4 = 0; e4 < BLK / 4; ++e4) xg[e4] = x[g * (BLK / 4) + e4];
#pragma unroll
                for (int e4 = 0; e4 < BLK / 4; ++e4) {
                    const f4 xv = xg[e4];
                    float wv[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int e = 4 * e4 + t, b = e % (BLK / 2), hi = e >= BLK / 2;
                        const unsigned word = cur[b >> 4][(b >> 2) & 3];
                        const unsigned nib = (word >> (8 * (b & 3) + 4 * hi)) & 15u;
                        wv[t] = fmaf((float)nib, s, m8);
                    }
                    if constexpr (FUSED) {
                        acc = fmaf(xv.x, wv[0], acc);
                        acc = fmaf(xv.y, wv[1], acc);
                        acc = fmaf(xv.z, wv[2], acc);
                        acc = fmaf(xv.w, wv[3], acc);
                    } else {
                        acc = acc + xv.x * wv[0];
                        acc = acc + xv.y * wv[1];
                        acc = acc + xv.z * wv[2];
                        acc = acc + xv.w * wv[3];
                    }
                }
            }
        }
    }
    return acc;
}

__device__ __forceinline__ float row_any(const RkPMat& W, int row, const float* x) {
    const bool tail = row >= (W.M & ~7);
    if (W.block == 0) {
        const gptr<f4> w = (gptr<f4>)(glb(W.w) + (size_t)row * W.K);
        return tail ? chain_f32<false>(w, lds4(x), W.K >> 2) : chain_f32<true>(w, lds4(x), W.K >> 2);
    }
    const int ng = W.K / W.block;
    const gptr<u4> q = (gptr<u4>)(glb(W.q) + (size_t)row * (W.K >> 1));
    const gptr<float> sc = glb(W.sc) + (size_t)row * ng;
    if (W.block == 32)
        return tail ? chain_i4<32, false>(q, sc, lds4(x), ng) : chain_i4<32, true>(q, sc, lds4(x), ng);
    return tail ? chain_i4<64, false>(q, sc, lds4(x), ng) : chain_i4<64, true>(q, sc, lds4(x), ng);
}

// Before a wait: every wave of the workgroup is past the phase before. Waves
// that finish a phase early then sleep at the barrier instead of polling
// while the phase's chains (one or a few waves) still run.
__device__ __forceinline__ void quiet() { __syncthreads(); }

__device__ __forceinline__ float hsum8(const float* v) {
    const float c0 = v[0] + v[4], c1 = v[1] + v[5], c2 = v[2] + v[6], c3 = v[3] + v[7];
    return (c0 + c1) + (c2 + c3);
}

__device__ __forceinline__ u64 kmax_wave(u64 k) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const u64 other = ((u64)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
                          (uint32_t)__shfl_xor((int)(k & 0xFFFFFFFFull), o, 64);
        k = max(k, other);
    }
    return k;
}

// The P1 products in order: W_r, W_k, W_v, W_1, A_1, G_1, V_1.
__device__ __forceinline__ const RkPMat& p1_mat(const RkPLayer& P, int s) {
    switch (s) {
    case 0: return P.r;
    case 1: return P.k;
    case 2: return P.v;
    case 3: return P.w1;
    case 4: return P.a1;
    case 5: return P.g1;
    default: return P.v1;
    }
}

#ifdef SNHIP_RKE_PROF
// Profiling builds: wall-clock marks of thread 0 of workgroups 0 (a head
// owner) and G - 1 at points of each phase of every layer of the last step.
__device__ unsigned long long g_rke_prof[2][64][12];
#define RKE_MARK(l, k)                                                                         \
    do {                                                                                       \
        if (threadIdx.x == 0 && (wg == 0 || wg == G - 1) && (l) < 64)                          \
            g_rke_prof[wg == 0 ? 0 : 1][l][k] = wall_clock64();                                \
    } while (0)
#else
#define RKE_MARK(l, k) do { } while (0)
#endif

__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_rk_exact(RkPArgs A) {
    // (the buffers chains and sums read carry kPad floats of slack)
    __shared__ __align__(16) float stg[2 * kStg + kPad];   // staged weights (two chunk buffers)
    __shared__ __align__(16) float xs[kRkPMaxD + kPad];    // x entering the phase
    __shared__ __align__(16) float xn[kRkPMaxD];        // LN_1(x) of this layer
    __shared__ __align__(16) float xn2[kRkPMaxD];       // LN_2(x_a)
    __shared__ __align__(16) float sq[kRkPMaxD + kPad];    // LayerNorm scratch
    __shared__ __align__(16) float buf[6 * kRkPMaxD + kPad];   // X6 | y | xk2 | ck | LN_out(x)
    __shared__ __align__(16) float midb[4 * kRkPRank + kPad];  // LoRA middles: tanh(lw), la, sig(lg), lv
    float(*mid)[kRkPRank] = reinterpret_cast<float(*)[kRkPRank]>(midb);
    __shared__ float up[4][HS];                          // dw, da, g, dv of the owned head
    __shared__ float kx[HS], vx[HS], v_[HS], part[8];
    __shared__ __align__(16) float r_[HS], w_[HS], k_[HS], a_[HS], kn_[HS];
    __shared__ __align__(16) float y_[HS + kPad], dt_[HS + kPad], sqh[HS + kPad];
    __shared__ float stat[3];
    __shared__ u64 kred[NW];
    __shared__ int sdead;
    __shared__ uint64_t etab[32];                        // expf's table (refmath::kExp2Tab)
    __shared__ RkPLayer Ls2[2];                          // layer tables of layers l (slot l & 1) and l + 1

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int D0 = A.D, F0 = A.F, L0 = A.L, NH0 = A.NH;
    // Independent sequences run on equal slices of the grid: this workgroup
    // is workgroup wg of sequence sqi's G0 (one sequence: sqi = 0, G0 = the grid).
    const int NI = A.ni > 1 ? A.ni : 1;
    const int G0 = gridDim.x / NI, sqi = blockIdx.x / G0, wg = blockIdx.x - sqi * G0;
    if (NI > 1) {
        A.S += (size_t)sqi * L0 * NH0 * HS * HS;
        A.shift += (size_t)sqi * L0 * 2 * D0;
        A.vfirst += (size_t)sqi * D0;
        A.xch += (size_t)sqi * A.words;
        A.keys += (size_t)sqi * A.words;
        A.tok += sqi;
        A.logits += (size_t)sqi * A.vocab;
    }
    if (tid == 0) sdead = 0;
    if (tid < 32) etab[tid] = refmath::kExp2Tab[tid];
    __syncthreads();
    // Leaves the kernel (in every thread of the workgroup) when any thread's
    // poll failed.
    auto agree = [&](bool ok) -> bool {
        if (!ok) sdead = 1;
        __syncthreads();
        return sdead == 0;
    };
    auto load_table = [&](int l) {
        if (tid < (int)(sizeof(RkPLayer) / 4))
            reinterpret_cast<int*>(&Ls2[l & 1])[tid] = reinterpret_cast<const int*>(A.layers + l)[tid];
    };
    float vfo = 0.0f;   // head owners, thread c < 64: v_first of channel c (layer 0's v)
    int tok = *A.tok;
    const int cnt0 = A.hist0;
    Pend pend;
        // A head owner's P2 operands into LDS: the 64 x 64 state (loaded into
        // sv by the caller, kSPer float4 per thread) into rows of kSRow floats
        // in buf, and the head's up-projection rows into stg (row c of matrix
        // m at uo[m] + c (K_m + 4)).
        auto stage_p2 = [&](const RkPLayer& P, int l, const f4 (&sv)[kSPer]) {
#pragma unroll
            for (int p = 0; p < kSPer; ++p) {
                const int i = tid + p * NT, r = i >> 4, c4 = i & 15;
                *reinterpret_cast<float4*>(buf + r * kSRow + 4 * c4) = make_float4(sv[p].x, sv[p].y, sv[p].z, sv[p].w);
            }
            const int c0 = wg * HS, nm = l > 0 ? 4 : 3;
            const RkPMat* U[4] = {&P.w2, &P.a2, &P.g2, &P.v2};
            int uo[5], n4[5];
            uo[0] = 0;
            n4[0] = 0;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                uo[m + 1] = uo[m] + (m < nm ? HS * (U[m]->K + 4) : 0);
                n4[m + 1] = n4[m] + (m < nm ? HS * (U[m]->K >> 2) : 0);
            }
            for (int base = 0; base < n4[4]; base += 8 * NT) {
                f4 v[8];
                int dst[8];
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    const int i = min(base + p * NT + tid, n4[4] - 1);
                    int m = 0;
#pragma unroll
                    for (int q = 1; q < 4; ++q)
                        if (i >= n4[q]) m = q;
                    const int k4n = U[m]->K >> 2, li = i - n4[m], c = li / k4n, k4 = li - c * k4n;
                    v[p] = *((gptr<f4>)(glb(U[m]->w) + (size_t)(c0 + c) * U[m]->K) + k4);
                    dst[p] = base + p * NT + tid < n4[4] ? uo[m] + c * (U[m]->K + 4) + 4 * k4 : -1;
                }
#pragma unroll
                for (int p = 0; p < 8; ++p)
                    if (dst[p] >= 0)
                        *reinterpret_cast<float4*>(stg + dst[p]) = make_float4(v[p].x, v[p].y, v[p].z, v[p].w);
            }
        };

    for (int st = 0; st < A.nsteps; ++st) {
        int D = D0, F = F0, L = L0, NH = NH0, G = G0;
        asm volatile("" : "+s"(D), "+s"(F), "+s"(L), "+s"(NH), "+s"(G));
        const bool owners_skip = NH * 4 <= G;   // the head owners take no P1 rows
        const size_t slab = rkp_slab(D, F);
        const unsigned ep = A.epoch + (unsigned)st;
        const PollCtl pc{A.err, A.spin_limit, ep + A.stall};
        const bool last = st + 1 == A.nsteps;

        // x = LN_0(E[tok]) (rwkv7.c:351-352); NaN for an out-of-range id.
        // Layer 0's table into slot 0 (every wave is past the previous step's
        // last use of it: the key reduction's barriers).
        {
            load_table(0);
            LnP lp;
            ln_load(lp, A.en_w, A.en_b, D);
            const bool ok = tok >= 0 && tok < A.vocab;
            const float* er = A.embed + (size_t)(ok ? tok : 0) * D;
            for (int i = tid; i < D; i += NT) buf[i] = ok ? er[i] : __builtin_nanf("");
            __syncthreads();
            ln_exact(buf, xs, sq, lp, D, A.eps, stat);
        }

        for (int l = 0; l < L; ++l) {
            u64* sl = A.xch + (size_t)l * slab;
            u64 *s_r = sl, *s_k = sl + D, *s_v = sl + 2 * D, *s_y = sl + 3 * D, *s_xa = sl + 4 * D,
                *s_xb = sl + 5 * D, *s_lw = sl + 6 * D, *s_la = s_lw + kRkPRank, *s_lg = s_la + kRkPRank,
                *s_lv = s_lg + kRkPRank, *s_ck = s_lv + kRkPRank;
            float* sh0 = A.shift + (size_t)l * 2 * D;
            float* sh1 = sh0 + D;
            const RkPLayer& P = Ls2[l & 1];

            // ---- P1: xn = LN_1(x); X6 = xn + lerp (shift_0 - xn); r k v, LoRA downs
            {
                // X6 holds xr | xw | xk | xv | xa | xg (the reference's mix order)
                const int nseg = l > 0 ? 7 : 6;
                int M[7];
#pragma unroll
                for (int sg = 0; sg < 7; ++sg) M[sg] = sg < nseg ? p1_mat(P, sg).M : 0;
                int total = 0;
#pragma unroll
                for (int sg = 0; sg < 7; ++sg) total += M[sg];
                // With the head owners at most a quarter of the grid, the rows
                // go to the workgroups past them, and the owners stage their
                // P2 operands meanwhile; otherwise every workgroup takes rows.
                const bool owner = owners_skip && wg < NH;
                int lo = 0, hi = 0;
                if (owners_skip) {
                    if (!owner) share(total, wg - NH, G - NH, lo, hi);
                } else {
                    share(total, wg, G, lo, hi);
                }
                // segment and row of P1 row `row` (selects, no branches)
                auto locate = [&](int row, int& sg, int& r) {
                    sg = 0;
                    r = row;
#pragma unroll
                    for (int q = 0; q < 6; ++q) {
                        const bool adv = sg == q && r >= M[q];
                        r = adv ? r - M[q] : r;
                        sg = adv ? q + 1 : sg;
                    }
                };
                const int xoff[7] = {0, 2 * D, 3 * D, D, 4 * D, 5 * D, 3 * D};
                // this workgroup's rows from segment sA's row rA on: nA of them
                // there, the rest from the start of the next segment (a share
                // spans two segments at most when no segment is shorter than
                // it; otherwise every row is located on its own)
                // (uniform values: the branch below is a scalar one, so a
                // workgroup whose share is in two segments never runs the
                // general lookup per row)
                int sA, rA;
                locate(lo, sA, rA);
                sA = __builtin_amdgcn_readfirstlane(sA);
                rA = __builtin_amdgcn_readfirstlane(rA);
                int MA = M[0], MB = M[1];   // M[sA], M[sA + 1] (no run-time index)
#pragma unroll
                for (int q = 1; q < 7; ++q) {
                    MA = sA == q ? M[q] : MA;
                    MB = sA + 1 == q ? M[q] : MB;
                }
                const int nA = __builtin_amdgcn_readfirstlane(MA - rA);
                const bool two = __builtin_amdgcn_readfirstlane(
                                     hi - lo <= nA || (sA + 1 < nseg && hi - lo - nA <= MB)) != 0;
                const float* bA = uni(p1_mat(P, sA).w) + (size_t)rA * D;
                const float* bB = uni(p1_mat(P, min(sA + 1, nseg - 1)).w);
                auto wrow = [&](int i) -> gptr<f4> {
                    if (two) return (gptr<f4>)(glb(i < nA ? bA + (size_t)i * D : bB + (size_t)(i - nA) * D));
                    int sg, r;
                    locate(lo + i, sg, r);
                    return (gptr<f4>)(glb(p1_mat(P, sg).w) + (size_t)r * D);
                };
                RKE_MARK(l, 0);
                const Stager S = stager(hi - lo, D);
                LnP lp;
                float shv[kPer], lrp[6][kPer];
                f4 sv[kSPer];
                if (!owner) {
                    stager_issue(pend, stg, S, wrow);   // the first weights, ahead of the wait
                    // the LayerNorm, shift and mix parameters, ahead of the wait too
                    ln_load(lp, P.ln1w, P.ln1b, D);
#pragma unroll
                    for (int k = 0; k < kPer; ++k) {
                        const int ic = min(k * NT + tid, D - 1);
                        shv[k] = ld_ag(sh0 + ic);
#pragma unroll
                        for (int s6 = 0; s6 < 6; ++s6) lrp[s6][k] = P.lerp[(size_t)s6 * D + ic];
                    }
                } else {
                    // the head's 64 x 64 state, kSPer float4 per thread
                    const float* Sh = A.S + ((size_t)l * NH + wg) * HS * HS;
#pragma unroll
                    for (int p = 0; p < kSPer; ++p) sv[p] = ((gptr<f4>)glb(Sh))[tid + p * NT];
                }
                issued();
                // x_b of the layer before (every wave is past its last use of
                // xs and of the other table slot once the poll's barrier is)
                if (l > 0) {
                    quiet();
                    const bool ok = poll_vec<kPer, NT>(A.xch + (size_t)(l - 1) * slab + 5 * D, D, xs, pc);
                    if (!agree(ok)) return;
                }
                if (l + 1 < L) load_table(l + 1);
                RKE_MARK(l, 1);
                if (owner) {
                    // The state and the up-projection rows into LDS: the owners
                    // use neither buf nor stg in this phase, and every wave is
                    // past the layer before's use of them (the poll's barrier).
                    stage_p2(P, l, sv);
                } else {
                    ln_exact(xs, xn, sq, lp, D, A.eps, stat);
#pragma unroll
                    for (int k = 0; k < kPer; ++k) {
                        const int i = k * NT + tid;
                        if (i < D) {
                            const float x = xn[i], d = shv[k] - x;
#pragma unroll
                            for (int s6 = 0; s6 < 6; ++s6) buf[s6 * D + i] = x + lrp[s6][k] * d;
                        }
                    }
                    __syncthreads();
                    u64* outs[7] = {s_r, s_k, s_v, s_lw, s_la, s_lg, s_lv};
                    RKE_MARK(l, 2);
                    stager_run(
                        pend, stg, S, wrow,
                        [&](int i) -> const float* {
                            int sg, r;
                            locate(lo + i, sg, r);
                            return buf + xoff[sg];
                        },
                        [&](int i, float v) {
                            int sg, r;
                            locate(lo + i, sg, r);
                            const RkPMat& W = p1_mat(P, sg);
                            if (r >= (W.M & ~7)) v = tail_chain(W.w, D, r, buf + xoff[sg]);
                            if (sg == 3) v = refmath::tanhf(v);          // the w middle (rwkv7.c:209-214)
                            else if (sg == 5) v = refmath::sigmoid_tab(v, etab);   // the g middle
                            ex_put(outs[sg] + r, v, ep);
                        });
                }
            }

            RKE_MARK(l, 3);
            // ---- P2: head h = wg (rwkv7.c:143-189, 229-299)
            if (wg < NH) {
                const int h = wg, c0 = h * HS;
                const int R[4] = {P.w1.M, P.a1.M, P.g1.M, P.v1.M};
                const int nm = l > 0 ? 4 : 3;
                const RkPMat* U[4] = {&P.w2, &P.a2, &P.g2, &P.v2};
                // the up-projection rows (in stg) and the state (in buf): staged
                // during P1, or here by owners that took P1 rows (once every
                // wave is done with the P1 chunks in stg and X6 in buf)
                if (!owners_skip) {
                    __syncthreads();
                    f4 sv[kSPer];
                    const float* Sh = A.S + ((size_t)l * NH + h) * HS * HS;
#pragma unroll
                    for (int p = 0; p < kSPer; ++p) sv[p] = ((gptr<f4>)glb(Sh))[tid + p * NT];
                    stage_p2(P, l, sv);
                }
                int uo[5];
                uo[0] = 0;
#pragma unroll
                for (int m = 0; m < 4; ++m) uo[m + 1] = uo[m] + (m < nm ? HS * (U[m]->K + 4) : 0);
                float* Sh = A.S + ((size_t)l * NH + h) * HS * HS;
                // the channel vectors of the owned head, ahead of the wait (v0
                // from layer 1 on)
                float cw0, cv0 = 0.0f, ca0, ckk, cka, crk, clnw, clnb;
                {
                    const int c = c0 + (tid & 63);
                    cw0 = P.w0[c];
                    if (l > 0) cv0 = P.v0[c];
                    ca0 = P.a0[c];
                    ckk = P.kk[c];
                    cka = P.ka[c];
                    crk = P.rk[c];
                    clnw = P.lnxw[c];
                    clnb = P.lnxb[c];
                }
                issued();
                quiet();
                {
                    const int i = min(tid, kRkPRank - 1), c = c0 + (tid & 63);
                    const bool lora = tid < kRkPRank, chan = tid < HS;
                    const u64* at[7] = {s_lw + i, s_la + i, s_lg + i, s_lv + i, s_r + c, s_k + c, s_v + c};
                    const bool use[7] = {lora && i < R[0], lora && i < R[1], lora && i < R[2],
                                         lora && l > 0 && i < R[3], chan, chan, chan};
                    u64 w[7];
#pragma unroll
                    for (int k = 0; k < 7; ++k) w[k] = use[k] ? ex_get(at[k]) : ((u64)pc.want << 32);
                    const bool ok = ex_spin(w, at, pc);
                    __syncthreads();
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        if (use[m]) mid[m][i] = ex_f(w[m]);
                    if (chan) {
                        r_[tid] = ex_f(w[4]);
                        kx[tid] = ex_f(w[5]);
                        vx[tid] = ex_f(w[6]);
                    }
                    if (!agree(ok)) return;
                }
                RKE_MARK(l, 4);
                // up-projections of the head's channels: thread 64 m + c runs
                // the chain of matrix m (W_2, A_2, G_2, V_2), output c0 + c
                if (wv < nm) {
                    const RkPMat& W = *U[wv];
                    const int K = W.K, row = c0 + lane;
                    float acc;
                    if (row >= (W.M & ~7)) {
                        acc = tail_chain(W.w, K, row, mid[wv]);
                    } else {
                        acc = lds_chain(lds4(stg + uo[wv] + lane * (K + 4)), lds4(mid[wv]), K >> 2, 0.0f);
                    }
                    up[wv][lane] = acc;
                }
                __syncthreads();
                if (tid < HS) {
                    // channel terms (rwkv7.c:236-260)
                    const int t = tid, c = c0 + t;
                    const float ww = refmath::expf_tab(-refmath::sigmoid_tab(up[0][t] + cw0, etab) * kR2, etab);
                    float vv = vx[t];
                    if (l == 0) {
                        vfo = vv;
                        A.vfirst[c] = vv;
                    } else {
                        const float mix = refmath::sigmoid_tab(up[3][t] + cv0, etab);
                        vv = vv + (vfo - vv) * mix;
                    }
                    const float av = refmath::sigmoid_tab(up[1][t] + ca0, etab);
                    const float kv = kx[t];
                    const float kkv = kv * ckk;
                    const float k2 = kv + kv * (av - 1.0f) * cka;
                    const float rv = r_[t];
                    w_[t] = ww; k_[t] = k2; v_[t] = vv; a_[t] = av; kn_[t] = kkv;
                    dt_[t] = rv * k2 * crk;
                }
                __syncthreads();
                // |kk|: eight stride-8 partial sums of squares (rwkv7.c:156-162)
                if (tid < 8) {
                    float ss = 0.0f;
#pragma unroll
                    for (int m = 0; m < 8; ++m) {
                        const float e = kn_[8 * m + tid];
                        ss = fmaf(e, e, ss);
                    }
                    part[tid] = ss;
                }
                __syncthreads();
                if (tid == 0) {
                    float nrm = sqrtf(hsum8(part));
                    if (!(nrm > 1e-12f)) nrm = 1e-12f;
                    stat[0] = 1.0f / nrm;
                }
                __syncthreads();
                float kn = 0.0f;
                if (tid < HS) kn = kn_[tid] * stat[0];
                __syncthreads();
                if (tid < HS) kn_[tid] = kn;
                __syncthreads();
                if (tid < HS) {
                    // state row t (rwkv7.c:165-187), four columns at a time
                    // from the LDS copy; column j's terms go to partial j mod 8
                    const l_f4* srow = lds4(buf + tid * kSRow);
                    const l_f4 *kn4p = vaddr(lds4(kn_)), *a4p = vaddr(lds4(a_)), *k4p = vaddr(lds4(k_)),
                               *w4p = vaddr(lds4(w_)), *r4p = vaddr(lds4(r_));
                    const float vv = v_[tid];
                    float proj[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < HS / 4; ++c) {
                        const f4 s4 = srow[c], kn4 = kn4p[c];
                        const int q = 4 * (c & 1);
                        proj[q] = fmaf(s4.x, kn4.x, proj[q]);
                        proj[q + 1] = fmaf(s4.y, kn4.y, proj[q + 1]);
                        proj[q + 2] = fmaf(s4.z, kn4.z, proj[q + 2]);
                        proj[q + 3] = fmaf(s4.w, kn4.w, proj[q + 3]);
                    }
                    const float pv = hsum8(proj);
                    float yacc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                    float* Srow = Sh + (size_t)tid * HS;
#pragma unroll
                    for (int c = 0; c < HS / 4; ++c) {
                        const f4 s4 = srow[c], kn4 = kn4p[c], a4 = a4p[c], k4 = k4p[c], w4 = w4p[c], r4 = r4p[c];
                        const int q = 4 * (c & 1);
                        f4 ns;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float kka = kn4[e] * a4[e];
                            const float vk = vv * k4[e];
                            ns[e] = fmaf(s4[e], w4[e], vk - pv * kka);
                            yacc[q + e] = fmaf(ns[e], r4[e], yacc[q + e]);
                        }
                        *reinterpret_cast<float4*>(Srow + 4 * c) = make_float4(ns.x, ns.y, ns.z, ns.w);
                    }
                    y_[tid] = hsum8(yacc);
                }
                __syncthreads();
                // group norm, bonus, gate (rwkv7.c:266-288): the mean and the
                // bonus dot as sequential sums, then the variance
                if (tid < 2) stat[1 + tid] = seq_sum(lds4(tid == 0 ? y_ : dt_), HS / 4);
                __syncthreads();
                const float mean = stat[1] / (float)HS, dot = stat[2];
                float yy = 0.0f;
                if (tid < HS) {
                    yy = y_[tid];
                    const float dd = yy - mean;
                    sqh[tid] = dd * dd;
                }
                __syncthreads();
                if (tid == 0) stat[0] = 1.0f / sqrtf(seq_sum(lds4(sqh), HS / 4) / (float)HS + kEpsGroup);
                __syncthreads();
                if (tid < HS) {
                    const int c = c0 + tid;
                    const float n = (yy - mean) * stat[0] * clnw + clnb;
                    ex_put(s_y + c, (n + dot * v_[tid]) * up[2][tid], ep);
                }
            }

            // ---- P3: x_a = x + W_o y (rwkv7.c:290-292)
            {
                int lo, hi;
                share(D, wg, G, lo, hi);
                const float* wb = uni(P.o.w) + (size_t)lo * D;
                auto wrow = [&](int i) -> gptr<f4> { return (gptr<f4>)(glb(wb) + (size_t)i * D); };
                const bool ok = with_kl(lsc_kl(hi - lo, D), [&](auto kl) -> bool {
                    Phase<decltype(kl)::value> ph;
                    ph.issue(pend, stg, hi - lo, D, wrow);
                    issued();
                    RKE_MARK(l, 5);
                    quiet();
                    if (!agree(poll_vec<kPer, NT>(s_y, D, buf, pc))) return false;
                    RKE_MARK(l, 6);
                    // shift_0 <- xn (rwkv7.c:229), by a workgroup past the head
                    // owners (it has xn). Every workgroup that reads shift_0 has
                    // by now: the owners have all of r, k, v and the LoRA
                    // middles, and every workgroup that takes P1 rows has some.
                    if (wg == G - 1)
                        for (int i = tid; i < D; i += NT) st_ag(sh0 + i, xn[i]);
                    ph.run(pend, stg, buf, wrow, [&](int i, float v) {
                        const int row = lo + i;
                        if (row >= (P.o.M & ~7)) v = tail_chain(P.o.w, D, row, buf);
                        ex_put(s_xa + row, xs[row] + v, ep);
                    });
                    return true;
                });
                if (!ok) return;
            }

            // ---- P4: xn2 = LN_2(x_a); xk2 = xn2 + cmk_lerp (shift_1 - xn2); ck = relu(W_ck xk2)^2
            {
                int lo, hi;
                share(F, wg, G, lo, hi);
                const float* wb = uni(P.cmk.w) + (size_t)lo * D;
                auto wrow = [&](int i) -> gptr<f4> { return (gptr<f4>)(glb(wb) + (size_t)i * D); };
                const Stager S = stager(hi - lo, D);
                stager_issue(pend, stg, S, wrow);
                LnP lp;
                ln_load(lp, P.ln2w, P.ln2b, D);
                float shv[kPer], lrp[kPer];
#pragma unroll
                for (int k = 0; k < kPer; ++k) {
                    const int ic = min(k * NT + tid, D - 1);
                    shv[k] = ld_ag(sh1 + ic);
                    lrp[k] = P.cmk_lerp[ic];
                }
                issued();
                RKE_MARK(l, 7);
                quiet();
                if (!agree(poll_vec<kPer, NT>(s_xa, D, xs, pc))) return;
                RKE_MARK(l, 8);
                ln_exact(xs, xn2, sq, lp, D, A.eps, stat);
#pragma unroll
                for (int k = 0; k < kPer; ++k) {
                    const int i = k * NT + tid;
                    if (i < D) {
                        const float x = xn2[i];
                        buf[i] = x + lrp[k] * (shv[k] - x);
                    }
                }
                __syncthreads();
                stager_run(
                    pend, stg, S, wrow, [&](int) -> const float* { return buf; },
                    [&](int i, float v) {
                        const int row = lo + i;
                        if (row >= (P.cmk.M & ~7)) v = tail_chain(P.cmk.w, D, row, buf);
                        const float r = v > 0.0f ? v : 0.0f;
                        ex_put(s_ck + row, r * r, ep);
                    });
            }

            // ---- P5: x_b = x_a + W_cv ck; shift_1 <- xn2 (rwkv7.c:305-315)
            {
                int lo, hi;
                share(D, wg, G, lo, hi);
                const float* wb = uni(P.cmv.w) + (size_t)lo * F;
                auto wrow = [&](int i) -> gptr<f4> { return (gptr<f4>)(glb(wb) + (size_t)i * F); };
                const bool ok = with_kl(lsc_kl(hi - lo, F), [&](auto kl) -> bool {
                    Phase<decltype(kl)::value> ph;
                    ph.issue(pend, stg, hi - lo, F, wrow);
                    issued();
                    RKE_MARK(l, 9);
                    quiet();
                    if (!agree(poll_vec<kPerF, NT>(s_ck, F, buf, pc))) return false;
                    RKE_MARK(l, 10);
                    // Every workgroup has read shift_1 by now: each has rows of ck.
                    if (wg == 0)
                        for (int i = tid; i < D; i += NT) st_ag(sh1 + i, xn2[i]);
                    ph.run(pend, stg, buf, wrow, [&](int i, float v) {
                        const int row = lo + i;
                        if (row >= (P.cmv.M & ~7)) v = tail_chain(P.cmv.w, F, row, buf);
                        ex_put(s_xb + row, xs[row] + v, ep);
                    });
                    return true;
                });
                if (!ok) return;
                RKE_MARK(l, 11);
            }
        }

        // ---- head: logits = W_head LN_out(x) (rwkv7.c:358-359), argmax keys
        {
            LnP lp;
            ln_load(lp, A.on_w, A.on_b, D);
            quiet();
            if (!agree(poll_vec<kPer, NT>(A.xch + (size_t)(L - 1) * slab + 5 * D, D, xs, pc))) return;
            ln_exact(xs, buf, sq, lp, D, A.eps, stat);
            int lo, hi;
            share(A.vocab, wg, G, lo, hi);
            u64 best = 0ull;
            for (int row = lo + tid; row < hi; row += NT) {
                const float d = row_any(A.head, row, buf);
                if (last) A.logits[row] = d;
                best = max(best, argmax_key(d, row));
            }
            best = kmax_wave(best);
            if (lane == 0) kred[wv] = best;
            __syncthreads();
            if (tid < 2) {
                u64 b = kred[0];
                for (int w = 1; w < NW; ++w) b = max(b, kred[w]);
                ex_put_bits(A.keys + 2 * wg + tid, tid == 0 ? (uint32_t)(b >> 32) : (uint32_t)b, ep);
            }
        }
        if (!A.greedy) return;   // (one step)
        // ---- every workgroup reduces the keys to the greedy token
        {
            constexpr int KW = 2 * kRkPMaxGrid / NT;
            u64 w[KW];
            const u64* at[KW];
#pragma unroll
            for (int k = 0; k < KW; ++k) {
                const int i = k * NT + tid;
                at[k] = A.keys + min(i, 2 * G - 1);
                w[k] = i < 2 * G ? ex_get(at[k]) : ((u64)pc.want << 32);
            }
            if (!agree(ex_spin(w, at, pc))) return;
            // word 2 j + 1 of a pair sits in the next lane (NT is even)
            u64 b = 0ull;
#pragma unroll
            for (int k = 0; k < KW; ++k) {
                const uint32_t hi = (uint32_t)w[k], lo = (uint32_t)__shfl_down((int)(uint32_t)w[k], 1, 64);
                if (k * NT + tid < 2 * G && (tid & 1) == 0) b = max(b, ((u64)hi << 32) | lo);
            }
            b = kmax_wave(b);
            if (lane == 0) kred[wv] = b;
            __syncthreads();
            u64 m = kred[0];
            for (int w2 = 1; w2 < NW; ++w2) m = max(m, kred[w2]);
            tok = (int)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull));
            const long hrow = (long)(cnt0 + st) * NI + sqi;
            if (wg == 0 && tid == 0 && hrow < A.hist_cap) A.tok_hist[hrow] = tok;
            __syncthreads();   // every wave has read kred (and the tables) before the next step writes them
        }
    }   // steps
    if (wg == 0 && tid == 0) {
        *A.tok = tok;
        if (sqi == 0) *A.counter = cnt0 + A.nsteps;
    }
}

}  // namespace

bool rke_shape_ok(int D, int F, int HS_, int NH, const int (*ranks)[4], int L) {
    if (!rkp_shape_ok(D, F, HS_, NH, ranks, L)) return false;
    // a head owner's up-projection rows (64 per matrix, padded by 4) fit the
    // two stage buffers
    for (int l = 0; l < L; ++l) {
        int n = 0;
        for (int j = 0; j < 4; ++j) n += HS * (ranks[l][j] + 4);
        if (n > 2 * kStg) return false;
    }
    return D % 4 == 0 && F % 4 == 0;
}

// Grids the kernel accepts: every product's rows on a workgroup fit a
// staged chunk (at most kMaxStageRows).
bool rke_grid_ok(int G, int D, int F, int p1rows) {
    // The P1 rows go to the G - NH workgroups past the head owners when the
    // owners are at most a quarter of the grid, else to all G; at least one
    // each (the shift_0 rewrite relies on it: there are 3 D rows at least).
    const int NH = D / HS, G1 = NH * 4 <= G ? G - NH : G;
    return G >= NH + 1 && G1 <= 3 * D && (p1rows + G1 - 1) / G1 <= kMaxStageRows && (F + G - 1) / G <= kMaxStageRows &&
           (D + G - 1) / G <= kMaxStageRows;
}

int rke_grid(int NH) {
    int dev = 0, coop = 0, ncu = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(k_rk_exact), NT, 0) !=
            hipSuccess || occ < 1)
        return 0;
    const int G = (ncu / 8) * 8;
    return G >= 8 && G >= NH ? G : 0;
}

#ifdef SNHIP_RKE_PROF
extern "C" int snhip_rke_prof(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_rke_prof), sizeof(g_rke_prof)) == hipSuccess ? 0 : 1;
}
#endif

snhip_status launch_rk_exact(const RkPArgs& a, int G, hipStream_t st) {
    const int ni = a.ni > 1 ? a.ni : 1;
    if (G % ni || G / ni < 8 || (G / ni) % 8 || G / ni < a.NH || G > kRkPMaxGrid ||
        (ni > 1 && a.words < (size_t)a.L * rkp_slab(a.D, a.F) + 2 * (size_t)(G / ni))) {
        set_last_error("RWKV-7 exact persistent step: bad grid");
        return SNHIP_E_INVAL;
    }
    RkPArgs args = a;
    void* kargs[] = {&args};
    SNHIP_CHECK(launch_persistent(reinterpret_cast<const void*>(k_rk_exact), dim3(G), dim3(NT), kargs, st));
    return SNHIP_OK;
}

}  // namespace snhip
