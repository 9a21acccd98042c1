// RWKV-7 decode step for one sequence as one cooperative launch
// (sunnynet/runtime/rwkv7.c:143-360; the math is the one listed at the top of
// rwkv.hip).
//
// At one sequence the step is a chain of small matrix-vector products; run as
// separate kernels (even replayed from a graph) each costs about 4.6 us of
// launch and drain on gfx950 whatever its size, about 100 of them per step.
// Here one launch runs the whole step: one 512-thread workgroup per CU, the
// products' rows spread over every wave of the grid. Five phases per layer:
//
//   P1  LN_1 + token-shift mixes (every workgroup, into LDS), then the rows of
//       W_r, W_k, W_v and the LoRA down-projections W_1, A_1, G_1, V_1;
//   P2  workgroup h < n_head: the LoRA up-projections of head h's 64
//       channels, decay / value residual / in-context rate, the 64 x 64 state
//       update (the head's state lives in LDS and registers for the phase),
//       read-out, group norm, bonus and gate -> y of head h;
//   P3  rows of W_o, x_a = x + W_o y;
//   P4  LN_2 + channel-mix input (every workgroup), rows of W_ck, relu^2;
//   P5  rows of W_cv, x_b = x_a + W_cv ck.
//
// then LN_out and the head rows with a per-workgroup argmax key, and every
// workgroup reduces the keys to the greedy token, the next step's input: a
// greedy launch runs many steps (and a step that returns logits, one).
//
// Exchange without grid barriers. Every value a phase produces has its own
// word in a per-layer slab: the launch's epoch in the high half, the value's
// bits in the low half, written once per launch with one agent-scope store.
// A phase's readers poll the words they need until each carries the epoch,
// so a phase waits for exactly its inputs, in one store-to-load round trip
// across XCDs. Step st of a launch uses the epoch A.epoch + st, and a word's
// first write in a step follows every workgroup's argmax keys of the step
// before, so every read of the word in that step. The recurrent state (S,
// v_first) is read and written only by the threads that own it. The shift
// vectors, read by every workgroup in P1 / P4 and rewritten by workgroup 0,
// are rewritten only once workgroup 0 has seen outputs of every workgroup
// that follow those reads; they are stored and loaded at agent scope, and a
// rewrite completes before workgroup 0's next exchange wait, so before its
// keys, which every reader of the next step has seen.
#include <type_traits>

#include "gemv.h"
#include "rkpersist.h"
#include "rkxch.h"

namespace snhip {
namespace {
using namespace rkx;

constexpr int NT = 512, NW = NT / 64, HS = 64;
constexpr float kR2 = 0.6065306597126334f;   // 1/sqrt(e), rwkv7.c:38
constexpr float kEpsGroup = 6.4e-4f;          // rwkv7.c:39
constexpr int kPer = kRkPMaxD / NT;           // LayerNorm values per thread
constexpr int kPerF = kRkPMaxF / NT;          // channel-mix key values per thread
typedef unsigned long long u64;

template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> glb(const T* p) { return (gptr<T>)p; }

__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }


// Cross-lane sums through DPP moves (VALU, no LDS round trips): within
// aligned groups of 2, 4, 8 and 16 lanes (quad permutations, then the half
// row and row mirrors, each pairing every lane with one whose partial covers
// the other half of its group), and over the wave (the four row sums read
// from lanes 0, 16, 32, 48). Every lane of a group gets its group's sum.
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float grp_sum(float v, int n) {
    if (n >= 2) v += dppf<0xB1>(v);    // quad_perm [1, 0, 3, 2]
    if (n >= 4) v += dppf<0x4E>(v);    // quad_perm [2, 3, 0, 1]
    if (n >= 8) v += dppf<0x141>(v);   // row_half_mirror
    if (n >= 16) v += dppf<0x140>(v);  // row_mirror
    return v;
}
__device__ __forceinline__ float lane_val(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wsum(float v) {
    v = grp_sum(v, 16);
    return (lane_val(v, 0) + lane_val(v, 16)) + (lane_val(v, 32) + lane_val(v, 48));
}

__device__ __forceinline__ float bsum(float v, float* red) {
    v = wsum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) s += red[w];
    return s;
}

// This thread's gains and biases of a LayerNorm over n <= kRkPMaxD values
// (element k NT + tid in slot k).
__device__ __forceinline__ void ln_params(const float* g, const float* c, int n, float (&gv)[kPer],
                                          float (&cv)[kPer]) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int ic = min(k * NT + (int)threadIdx.x, n - 1);
        gv[k] = g[ic];
        cv[k] = c[ic];
    }
}

// y[i] = LN(x)[i] * g[i] + c[i] over n <= kRkPMaxD values in LDS
// (rwkv7.c:127-140 form, two passes), with the gains and biases loaded by
// ln_params (a phase issues them ahead of its exchange wait).
__device__ void layer_norm(const float* x, float* y, const float (&gv)[kPer], const float (&cv)[kPer], int n,
                           float eps, float* red) {
    float v[kPer];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = k * NT + threadIdx.x;
        v[k] = i < n ? x[i] : 0.0f;
        s += v[k];
    }
    const float mean = bsum(s, red) / (float)n;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k)
        if (k * NT + (int)threadIdx.x < n) {
            const float d = v[k] - mean;
            q += d * d;
        }
    const float rstd = 1.0f / sqrtf(bsum(q, red) / (float)n + eps);
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = k * NT + threadIdx.x;
        if (i < n) y[i] = (v[k] - mean) * rstd * gv[k] + cv[k];
    }
    __syncthreads();
}

__device__ void layer_norm(const float* x, float* y, const float* g, const float* c, int n, float eps,
                           float* red) {
    float gv[kPer], cv[kPer];
    ln_params(g, c, n, gv, cv);
    layer_norm(x, y, gv, cv, n, eps, red);
}

// Partial dot of one 16-value unit u of row `row` with X (LDS): fp32, or INT4
// with the quant.c layout (byte j of a group holds values j and j + block/2;
// w = fma(q, s, -8 s), quant.c:82-83).
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));
struct Unit {
    f4 f[4];
    u2 c;
    float s;
};

// Loads and products of one unit, the weight format a template argument
// (INT4: block 32 or 64 read from W). Callers issue every load of a row (or
// of four rows) unconditionally from clamped, valid addresses and select the
// contributions afterwards: a load under a branch gets a full wait at the
// branch's join, which would serialize them.
template <bool Q>
__device__ __forceinline__ void unit_load(Unit& U, const RkPMat& W, int row, int u) {
    if constexpr (!Q) {
        const gptr<f4> p = (gptr<f4>)(glb(W.w) + (size_t)row * W.K + u * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j) U.f[j] = p[j];
    } else {
        const int upg = W.block >> 4;
        U.c = *(gptr<u2>)(glb(W.q) + (size_t)row * (W.K >> 1) + (size_t)u * 8);
        U.s = glb(W.sc)[(size_t)row * (W.K / W.block) + u / upg];
    }
}

template <bool Q>
__device__ __forceinline__ float unit_dot(const Unit& U, const RkPMat& W, int u, const float* X, float acc) {
    if constexpr (!Q) {
        const float* x = X + u * 16;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = fmaf(U.f[j].x, x[4 * j], acc);
            acc = fmaf(U.f[j].y, x[4 * j + 1], acc);
            acc = fmaf(U.f[j].z, x[4 * j + 2], acc);
            acc = fmaf(U.f[j].w, x[4 * j + 3], acc);
        }
        return acc;
    } else {
        const int upg = W.block >> 4, g = u / upg, qd = u - g * upg;
        const float* xl = X + g * W.block + qd * 8;
        const float* xh = xl + (W.block >> 1);
        const float m8 = -8.0f * U.s;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned b = ((i < 4 ? U.c.x : U.c.y) >> (8 * (i & 3))) & 0xFFu;
            acc = fmaf(fmaf((float)(b & 15u), U.s, m8), xl[i], acc);
            acc = fmaf(fmaf((float)(b >> 4), U.s, m8), xh[i], acc);
        }
        return acc;
    }
}

template <bool Q, int NU>
__device__ __forceinline__ float row_dot_t(const RkPMat& W, int row, const float* X, int lane) {
    const int nu = W.K >> 4;
    Unit U[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j) unit_load<Q>(U[j], W, row, min(lane + 64 * j, nu - 1));
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int u = min(lane + 64 * j, nu - 1);
        const float a = unit_dot<Q>(U[j], W, u, X, 0.0f);
        acc += lane + 64 * j < nu ? a : 0.0f;
    }
    return wsum(acc);
}

template <bool Q>
__device__ __forceinline__ float row_dot_q(const RkPMat& W, int row, const float* X, int lane) {
    const int n = ((W.K >> 4) + 63) >> 6;
    if (n <= 1) return row_dot_t<Q, 1>(W, row, X, lane);
    if (n == 2) return row_dot_t<Q, 2>(W, row, X, lane);
    return row_dot_t<Q, 4>(W, row, X, lane);
}

// W[row] . X over the wave (every lane gets the sum); K <= 4096.
__device__ float row_dot(const RkPMat& W, int row, const float* X, int lane) {
    return W.block == 0 ? row_dot_q<false>(W, row, X, lane) : row_dot_q<true>(W, row, X, lane);
}

// N rows row0 + k * stride at once (rows past `end` read row end - 1 and
// are dropped), K <= 1024 (one unit per lane): every load issued before the
// first product.
template <bool Q, int N>
__device__ void row_dotn(const RkPMat& W, int row0, int stride, int end, const float* X, int lane,
                         float (&out)[N]) {
    const int nu = W.K >> 4;
    const int u = min(lane, nu - 1);
    Unit U[N];
#pragma unroll
    for (int k = 0; k < N; ++k) unit_load<Q>(U[k], W, min(row0 + k * stride, end - 1), u);
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const float a = unit_dot<Q>(U[k], W, u, X, 0.0f);
        out[k] = wsum(lane < nu ? a : 0.0f);
    }
}

// NR rows of W (row0 + k stride, clamped to the matrix) with NU units per
// lane each, loaded before the vector they multiply has arrived: a phase
// issues them ahead of its exchange wait, so the weights' memory latency
// overlaps the wait instead of following it.
template <bool Q, int NU, int NR>
struct PreRows {
    Unit u[NR][NU];
};

template <bool Q, int NU, int NR>
__device__ __forceinline__ void pre_load(PreRows<Q, NU, NR>& R, const RkPMat& W, int row0, int stride, int lane) {
    const int nu = W.K >> 4;
#pragma unroll
    for (int k = 0; k < NR; ++k)
#pragma unroll
        for (int j = 0; j < NU; ++j)
            unit_load<Q>(R.u[k][j], W, min(row0 + k * stride, W.M - 1), min(lane + 64 * j, nu - 1));
}

// out[k] = (row k of R) . X over the wave, in row_dot's order.
template <bool Q, int NU, int NR>
__device__ __forceinline__ void pre_dot(const PreRows<Q, NU, NR>& R, const RkPMat& W, const float* X, int lane,
                                        float (&out)[NR]) {
    const int nu = W.K >> 4;
#pragma unroll
    for (int k = 0; k < NR; ++k) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = min(lane + 64 * j, nu - 1);
            const float v = unit_dot<Q>(R.u[k][j], W, u, X, 0.0f);
            acc += lane + 64 * j < nu ? v : 0.0f;
        }
        out[k] = wsum(acc);
    }
}

// f(format, units per lane) for the instantiation that fits W: INT4 or fp32,
// NU = 1, 2 or 4 units of 16 values per lane (K <= 4096; K <= 1024 when
// ONE, the matrices whose input is a model-width vector).
template <bool ONE = false, class Fn>
__device__ __forceinline__ bool with_format(const RkPMat& W, Fn&& f) {
    if constexpr (ONE) {
        if (W.block != 0) return f(std::true_type{}, std::integral_constant<int, 1>{});
        return f(std::false_type{}, std::integral_constant<int, 1>{});
    }
    const int n = ((W.K >> 4) + 63) >> 6;
    if (W.block != 0) {
        if (n <= 1) return f(std::true_type{}, std::integral_constant<int, 1>{});
        if (n == 2) return f(std::true_type{}, std::integral_constant<int, 2>{});
        return f(std::true_type{}, std::integral_constant<int, 4>{});
    }
    if (n <= 1) return f(std::false_type{}, std::integral_constant<int, 1>{});
    if (n == 2) return f(std::false_type{}, std::integral_constant<int, 2>{});
    return f(std::false_type{}, std::integral_constant<int, 4>{});
}

// Two rows of two matrices with K <= 1024 at once (both loads first).
template <bool QA, bool QB>
__device__ __forceinline__ void pair_t(const RkPMat& WA, int rA, const float* XA, const RkPMat& WB, int rB,
                                       const float* XB, int lane, float& dA, float& dB) {
    const int nA = WA.K >> 4, nB = WB.K >> 4;
    const int uA = min(lane, nA - 1), uB = min(lane, nB - 1);
    Unit UA, UB;
    unit_load<QA>(UA, WA, rA, uA);
    unit_load<QB>(UB, WB, rB, uB);
    const float a = unit_dot<QA>(UA, WA, uA, XA, 0.0f);
    const float b = unit_dot<QB>(UB, WB, uB, XB, 0.0f);
    dA = wsum(lane < nA ? a : 0.0f);
    dB = wsum(lane < nB ? b : 0.0f);
}

__device__ void row_pair(const RkPMat& WA, int rA, const float* XA, const RkPMat& WB, int rB, const float* XB,
                         int lane, float& dA, float& dB) {
    if (WA.block == 0) {
        if (WB.block == 0) pair_t<false, false>(WA, rA, XA, WB, rB, XB, lane, dA, dB);
        else pair_t<false, true>(WA, rA, XA, WB, rB, XB, lane, dA, dB);
    } else {
        if (WB.block == 0) pair_t<true, false>(WA, rA, XA, WB, rB, XB, lane, dA, dB);
        else pair_t<true, true>(WA, rA, XA, WB, rB, XB, lane, dA, dB);
    }
}

// Rows [r0, r0 + n) of a matrix with K = 16 * nu, nu a power of two <= 16:
// 64 / nu rows per wave pass, lanes (row, unit); out[i] = dot of row r0 + i.
__device__ void small_rows(const RkPMat& W, int r0, int n, const float* X, float* out, int wv, int lane) {
    const int nu = W.K >> 4;
    const int per = 64 / nu;
    const int sub = lane / nu, u = lane - sub * nu;
    for (int base = wv * per; base < n; base += NW * per) {
        const int i = base + sub;
        float acc = 0.0f;
        Unit U;
        const int row = r0 + min(i, n - 1);
        if (W.block == 0) {
            unit_load<false>(U, W, row, u);
            acc = unit_dot<false>(U, W, u, X, 0.0f);
        } else {
            unit_load<true>(U, W, row, u);
            acc = unit_dot<true>(U, W, u, X, 0.0f);
        }
        acc = i < n ? acc : 0.0f;
        acc = grp_sum(acc, nu);
        if (i < n && u == 0) out[i] = acc;
    }
}

// The LoRA up-projections of head rows [c0, c0 + HS): W_2, A_2, G_2 and, when
// nm = 4, V_2 (matrix m multiplies X0 + m kRkPRank into out(m)), in
// small_rows' lanes and order, but in batches whose weight loads are all
// issued before the first product: item i of the T = sum over m of K_m / 16
// row passes goes to wave i mod NW, kUpI items per wave and batch (four
// separate calls paid four memory latencies one after another).
constexpr int kUpI = 4;
struct UpPlan {
    int lg[4];   // log2 of the units per row of matrix m
    int nm, T;
};
template <bool Q>
struct UpBatch {
    Unit U[kUpI];
    int mm[kUpI], ps[kUpI];
};

template <class Mat>
__device__ __forceinline__ UpPlan up_plan(Mat&& mat, int nm) {
    UpPlan pl;
    pl.nm = nm;
    pl.T = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        pl.lg[m] = m < nm ? 31 - __builtin_clz(mat(m).K >> 4) : 0;
        pl.T += m < nm ? 1 << pl.lg[m] : 0;
    }
    return pl;
}

// Loads the batch of items i0, i0 + NW, ... (wave-uniform i0).
template <bool Q, class Mat>
__device__ __forceinline__ void up_load(UpBatch<Q>& B, Mat&& mat, const UpPlan& pl, int i0, int c0, int lane) {
#pragma unroll
    for (int j = 0; j < kUpI; ++j) {
        int m = 0, pass = min(i0 + NW * j, pl.T - 1);
#pragma unroll
        for (int q = 0; q < 3; ++q)
            if (m == q && q + 1 < pl.nm && pass >= 1 << pl.lg[q]) {
                pass -= 1 << pl.lg[q];
                m = q + 1;
            }
        const int sub = lane >> pl.lg[m], u = lane - (sub << pl.lg[m]);
        unit_load<Q>(B.U[j], mat(m), c0 + min((pass << (6 - pl.lg[m])) + sub, HS - 1), u);
        B.mm[j] = m;
        B.ps[j] = pass;
    }
}

template <bool Q, class Mat, class Out>
__device__ __forceinline__ void up_dot(const UpBatch<Q>& B, Mat&& mat, Out&& out, const UpPlan& pl, int i0,
                                       const float* X0, int lane) {
#pragma unroll
    for (int j = 0; j < kUpI; ++j) {
        if (i0 + NW * j >= pl.T) break;
        const int m = B.mm[j], sub = lane >> pl.lg[m], u = lane - (sub << pl.lg[m]);
        const int i = (B.ps[j] << (6 - pl.lg[m])) + sub;
        float acc = unit_dot<Q>(B.U[j], mat(m), u, X0 + m * kRkPRank, 0.0f);
        acc = grp_sum(i < HS ? acc : 0.0f, 1 << pl.lg[m]);
        if (i < HS && u == 0) out(m)[i] = acc;
    }
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

#ifdef SNHIP_RKP_PROF
// Profiling builds: wall-clock marks of thread 0 of workgroups 0 (a head
// owner) and G - 1 at every phase entry and barrier entry of every launch.
__device__ unsigned long long g_rkp_prof[2][64 * 6 + 2][2];
#define RKP_MARK(ph, k)                                                                        \
    do {                                                                                       \
        if (threadIdx.x == 0 && (wg == 0 || wg == G - 1) && (ph) < 64 * 6 + 2)                 \
            g_rkp_prof[wg == 0 ? 0 : 1][ph][k] = wall_clock64();                               \
    } while (0)
#else
#define RKP_MARK(ph, k) do { } while (0)
#endif

__global__ __launch_bounds__(NT) void k_rk_persist(RkPArgs A) {
    __shared__ float xs[kRkPMaxD];            // x entering the phase
    __shared__ float xn[kRkPMaxD];            // LN_1(x) of this layer
    __shared__ float xn2[kRkPMaxD];           // LN_2(x_a)
    __shared__ float buf[6 * kRkPMaxD];       // X6 | ck | head inputs
    __shared__ float hv[12][HS];              // per-channel values of the owned head
    __shared__ float red[NW];
    __shared__ u64 kred[NW];
    __shared__ int sdead;
    __shared__ RkPLayer Ls2[2];                  // layer tables of layers l (l & 1) and l + 1

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int D0 = A.D, F0 = A.F, L0 = A.L, NH0 = A.NH;
    // Independent sequences run on equal slices of the grid: this workgroup
    // is workgroup wg of sequence sq's G0 (one sequence: sq = 0, G0 = the grid).
    const int NI = A.ni > 1 ? A.ni : 1;
    const int G0 = gridDim.x / NI, sq = blockIdx.x / G0, wg = blockIdx.x - sq * G0;
    if (NI > 1) {
        A.S += (size_t)sq * L0 * NH0 * HS * HS;
        A.shift += (size_t)sq * L0 * 2 * D0;
        A.vfirst += (size_t)sq * D0;
        A.xch += (size_t)sq * A.words;
        A.keys += (size_t)sq * A.words;
        A.tok += sq;
        A.logits += (size_t)sq * A.vocab;
    }
    if (tid == 0) sdead = 0;
    if (tid < (int)(sizeof(RkPLayer) / 4))
        reinterpret_cast<int*>(&Ls2[0])[tid] = reinterpret_cast<const int*>(A.layers)[tid];
    __syncthreads();
    // Leaves the kernel (in every thread of the workgroup) when any thread's
    // poll failed.
    auto agree = [&](bool ok) -> bool {
        if (!ok) sdead = 1;
        __syncthreads();
        return sdead == 0;
    };
    float vfo = 0.0f;   // head owners, thread c < 64: v_first of channel c (layer 0's v)
    int tok = *A.tok;
    const int cnt0 = A.hist0;

    // Greedy launches run nsteps steps, step st with epoch A.epoch + st; every
    // workgroup reduces the argmax keys to the next step's token itself.
    for (int st = 0; st < A.nsteps; ++st) {
        // The shape, opaque to the compiler in every step, so that what it
        // derives is not hoisted out of the step loop and held in registers.
        int D = D0, F = F0, L = L0, NH = NH0, G = G0;
        asm volatile("" : "+s"(D), "+s"(F), "+s"(L), "+s"(NH), "+s"(G));
        const size_t slab = rkp_slab(D, F);
        const unsigned ep = A.epoch + (unsigned)st;
        const PollCtl pc{A.err, A.spin_limit, ep + A.stall};
        const bool last = st + 1 == A.nsteps;

        // x = LN_0(E[tok]) (rwkv7.c:351-352); NaN for an out-of-range id. From
        // the second step on, layer 0's table goes back into slot 0 (every wave is
        // past the previous step's last use of it: the key reduction's barrier).
        {
            const bool ok = tok >= 0 && tok < A.vocab;
            const float* er = A.embed + (size_t)(ok ? tok : 0) * D;
            if (st > 0 && tid < (int)(sizeof(RkPLayer) / 4))
                reinterpret_cast<int*>(&Ls2[0])[tid] = reinterpret_cast<const int*>(A.layers)[tid];
            for (int i = tid; i < D; i += NT) buf[i] = ok ? er[i] : __builtin_nanf("");
            __syncthreads();
            layer_norm(buf, xs, A.en_w, A.en_b, D, A.eps, red);
        }

        for (int l = 0; l < L; ++l) {
            u64* sl = A.xch + (size_t)l * slab;
            u64 *s_r = sl, *s_k = sl + D, *s_v = sl + 2 * D, *s_y = sl + 3 * D, *s_xa = sl + 4 * D,
                *s_xb = sl + 5 * D, *s_lw = sl + 6 * D, *s_la = s_lw + kRkPRank, *s_lg = s_la + kRkPRank,
                *s_lv = s_lg + kRkPRank, *s_ck = s_lv + kRkPRank;
            float* sh0 = A.shift + (size_t)l * 2 * D;
            float* sh1 = sh0 + D;

            // ---- P1: xn = LN_1(x); X6 = xn + lerp (shift_0 - xn); r k v, LoRA down
            {
                // The layer's table (staged a layer ahead) gives the shift,
                // mix and LayerNorm parameters, issued ahead of the wait for
                // x_b of the layer before: the wait outlasts their latency.
                const RkPLayer& P = Ls2[l & 1];
                float shv[kPer], lrp[6][kPer], lg[kPer], lc[kPer];
#pragma unroll
                for (int k = 0; k < kPer; ++k) {
                    const int ic = min(k * NT + tid, D - 1);
                    shv[k] = ld_ag(sh0 + ic);
#pragma unroll
                    for (int s6 = 0; s6 < 6; ++s6) lrp[s6][k] = P.lerp[(size_t)s6 * D + ic];
                }
                ln_params(P.ln1w, P.ln1b, D, lg, lc);
                issued();
                // x_b of the layer before (every wave is past its last use of xs
                // and of the other layer-table slot once the poll's barrier is)
                if (l > 0) {
                    __syncthreads();   // waves done early sleep here instead of polling
                    const bool ok = poll_vec<kPer, NT>(A.xch + (size_t)(l - 1) * slab + 5 * D, D, xs, pc);
                    if (!agree(ok)) return;
                }
                // the next layer's table into the other slot
                if (l + 1 < L && tid < (int)(sizeof(RkPLayer) / 4))
                    reinterpret_cast<int*>(&Ls2[(l + 1) & 1])[tid] =
                        reinterpret_cast<const int*>(A.layers + l + 1)[tid];
                __syncthreads();
                RKP_MARK(l * 6 + 0, 0);
                // The workgroup's rows (r, k, v, then the LoRA down-projections,
                // with V_1 from layer 1 on), from the segment sizes read at once.
                const int nseg = l > 0 ? 7 : 6;
                int M[7];
#pragma unroll
                for (int sg = 0; sg < 7; ++sg) M[sg] = sg < nseg ? p1_mat(P, sg).M : 0;
                int total = 0;
#pragma unroll
                for (int sg = 0; sg < 7; ++sg) total += M[sg];
                int lo, hi;
                share(total, wg, G, lo, hi);
                auto locate = [&](int row, int& sg, int& r) {
                    sg = 0;
                    r = row;
#pragma unroll
                    for (int q = 0; q < 6; ++q)
                        if (sg == q && r >= M[q]) {
                            r -= M[q];
                            sg = q + 1;
                        }
                };
                bool uni = true;
#pragma unroll
                for (int sg = 1; sg < 7; ++sg)
                    uni = uni && (sg >= nseg || (p1_mat(P, sg).block == 0) == (P.r.block == 0));
                auto body = [&](auto q, bool pre) {
                    constexpr bool Q = decltype(q)::value;
                    const int xoff[7] = {0, 2 * D, 3 * D, D, 4 * D, 5 * D, 3 * D};
                    u64* outs[7] = {s_r, s_k, s_v, s_lw, s_la, s_lg, s_lv};
                    // the wave's first two rows, issued after x arrived and
                    // before the LayerNorm, which they overlap
                    const int row0 = lo + wv;
                    int sA0, rA0, sB0, rB0;
                    locate(min(row0, total - 1), sA0, rA0);
                    locate(min(row0 + NW, hi - 1) < 0 ? 0 : min(row0 + NW, hi - 1), sB0, rB0);
                    Unit UA, UB;
                    if (pre && row0 < hi) {
                        unit_load<Q>(UA, p1_mat(P, sA0), rA0, min(lane, (p1_mat(P, sA0).K >> 4) - 1));
                        unit_load<Q>(UB, p1_mat(P, sB0), rB0, min(lane, (p1_mat(P, sB0).K >> 4) - 1));
                    }
                    layer_norm(xs, xn, lg, lc, D, A.eps, red);
#pragma unroll
                    for (int k = 0; k < kPer; ++k) {
                        const int i = k * NT + tid;
                        if (i < D) {
                            const float d = shv[k] - xn[i];
#pragma unroll
                            for (int s6 = 0; s6 < 6; ++s6) buf[s6 * D + i] = xn[i] + lrp[s6][k] * d;
                        }
                    }
                    __syncthreads();
                    for (int row = row0; row < hi; row += 2 * NW) {
                        const int rowB = min(row + NW, hi - 1);
                        int sA, rA, sB, rB;
                        locate(row, sA, rA);
                        locate(rowB, sB, rB);
                        float dA, dB;
                        if (pre && row == row0) {
                            const RkPMat& WA = p1_mat(P, sA);
                            const RkPMat& WB = p1_mat(P, sB);
                            const int nA = WA.K >> 4, nB = WB.K >> 4;
                            const float a = unit_dot<Q>(UA, WA, min(lane, nA - 1), buf + xoff[sA], 0.0f);
                            const float b = unit_dot<Q>(UB, WB, min(lane, nB - 1), buf + xoff[sB], 0.0f);
                            dA = wsum(lane < nA ? a : 0.0f);
                            dB = wsum(lane < nB ? b : 0.0f);
                        } else {
                            row_pair(p1_mat(P, sA), rA, buf + xoff[sA], p1_mat(P, sB), rB, buf + xoff[sB], lane, dA,
                                     dB);
                        }
                        if (lane == 0) {
                            ex_put(outs[sA] + rA, dA, ep);
                            if (row + NW < hi) ex_put(outs[sB] + rB, dB, ep);
                        }
                    }
                };
                if (!uni) body(std::false_type{}, false);
                else if (P.r.block != 0) body(std::true_type{}, true);
                else body(std::false_type{}, true);
            }
            const RkPLayer& P = Ls2[l & 1];
            RKP_MARK(l * 6 + 0, 1);

            // ---- P2: head h = wg (rwkv7.c:143-189, 229-299)
            if (wg >= NH) RKP_MARK(l * 6 + 1, 0);
            if (wg < NH) {
                const int h = wg, c0 = h * HS;
                const int Rw = P.w1.M, Ra = P.a1.M, Rg = P.g1.M, Rv = P.v1.M;
                float* in_w = buf;                  // tanh(lw)
                float* in_a = buf + kRkPRank;       // la
                float* in_g = buf + 2 * kRkPRank;   // sig(lg)
                float* in_v = buf + 3 * kRkPRank;   // lv
                float* r_ = hv[9];
                float* kx = hv[11];                 // k of the channel (before k2)
                float* vx = hv[3];                  // v (dv goes to hv[10] below)
                // up-projections: dw, da, g and (from layer 1 on) dv
                const int nm = l > 0 ? 4 : 3;
                auto upm = [&](int m) -> const RkPMat& { return m == 0 ? P.w2 : m == 1 ? P.a2 : m == 2 ? P.g2 : P.v2; };
                auto upo = [&](int m) -> float* { return hv[m == 3 ? 10 : m]; };
                const UpPlan pl = up_plan(upm, nm);
                const bool q4 = P.w2.block != 0;
                const bool uni = (P.a2.block != 0) == q4 && (P.g2.block != 0) == q4 &&
                                 (nm < 4 || (P.v2.block != 0) == q4);
                auto owner = [&](auto q, bool batched) -> bool {
                    constexpr bool Q = decltype(q)::value;
                    // The head's state rows, its channel parameters and the first
                    // batch of up-projection weights are issued ahead of the wait
                    // for the phase's inputs, which (every workgroup's P1 rows and
                    // a round trip) outlasts their memory latency.
                    const gptr<f4> Sp = (gptr<f4>)(glb(A.S) + ((size_t)l * NH + wg) * HS * HS +
                                                   (size_t)(tid >> 3) * HS + (tid & 7) * 8);
                    const f4 pS0 = Sp[0], pS1 = Sp[1];
                    const int cc = c0 + (tid & 63);
                    const float pw0 = glb(P.w0)[cc], pv0 = glb(P.v0)[cc], pa0 = glb(P.a0)[cc], pkk = glb(P.kk)[cc];
                    const float pka = glb(P.ka)[cc], prk = glb(P.rk)[cc], plw = glb(P.lnxw)[cc], plb = glb(P.lnxb)[cc];
                    UpBatch<Q> ub;
                    if (batched) up_load<Q>(ub, upm, pl, wv, c0, lane);
                    issued();
                    {
                        const int i = min(tid, kRkPRank - 1), c = c0 + (tid & 63);
                        const bool lora = tid < kRkPRank, chan = tid < HS;
                        const u64* at[7] = {s_lw + i, s_la + i, s_lg + i, s_lv + i, s_r + c, s_k + c, s_v + c};
                        const bool use[7] = {lora && i < Rw, lora && i < Ra, lora && i < Rg, lora && l > 0 && i < Rv,
                                             chan, chan, chan};
                        u64 w[7];
#pragma unroll
                        for (int k = 0; k < 7; ++k) w[k] = use[k] ? ex_get(at[k]) : ((u64)pc.want << 32);
                        const bool ok = ex_spin(w, at, pc);
                        __syncthreads();   // every wave is done with X6 in buf
                        if (use[0]) in_w[i] = tanhf(ex_f(w[0]));
                        if (use[1]) in_a[i] = ex_f(w[1]);
                        if (use[2]) in_g[i] = sgm(ex_f(w[2]));
                        if (use[3]) in_v[i] = ex_f(w[3]);
                        if (chan) {
                            r_[tid] = ex_f(w[4]);
                            kx[tid] = ex_f(w[5]);
                            vx[tid] = ex_f(w[6]);
                        }
                        if (!agree(ok)) return false;
                    }
                    RKP_MARK(l * 6 + 1, 0);
                    if (batched) {
                        up_dot<Q>(ub, upm, upo, pl, wv, buf, lane);
                        for (int i0 = wv + NW * kUpI; i0 < pl.T; i0 += NW * kUpI) {
                            up_load<Q>(ub, upm, pl, i0, c0, lane);
                            up_dot<Q>(ub, upm, upo, pl, i0, buf, lane);
                        }
                    } else {
                        small_rows(P.w2, c0, HS, in_w, hv[0], wv, lane);
                        small_rows(P.a2, c0, HS, in_a, hv[1], wv, lane);
                        small_rows(P.g2, c0, HS, in_g, hv[2], wv, lane);
                        if (l > 0) small_rows(P.v2, c0, HS, in_v, hv[10], wv, lane);
                    }
                    __syncthreads();
                    float* w_ = hv[4]; float* k_ = hv[5]; float* v_ = hv[6]; float* a_ = hv[7];
                    float* kn_ = hv[8]; float* y_ = hv[10];
                    if (tid < HS) {
                        const int c = c0 + tid;
                        const float ww = expf(-sgm(hv[0][tid] + pw0) * kR2);            // :236-237
                        float vv = vx[tid];
                        if (l == 0) {
                            vfo = vv;
                            A.vfirst[c] = vv;                                            // :240
                        } else {
                            const float mix = sgm(hv[10][tid] + pv0);                    // :244-246
                            vv = vv + (vfo - vv) * mix;
                        }
                        const float av = sgm(hv[1][tid] + pa0);                         // :251-252
                        const float kv = kx[tid];
                        const float kkv = kv * pkk;                                      // :259
                        const float k2 = kv + kv * (av - 1.0f) * pka;                   // :260
                        float nrm = sqrtf(wsum(kkv * kkv));                              // :158-162
                        if (!(nrm > 1e-12f)) nrm = 1e-12f;
                        w_[tid] = ww; k_[tid] = k2; v_[tid] = vv; a_[tid] = av; kn_[tid] = kkv * (1.0f / nrm);
                    }
                    __syncthreads();   // (y_ reuses dv's row: dv was read above)
                    // S = S diag(w) - (S kk^)(kk^ a)^T + v k^T; y = S r. Thread t owns
                    // row i = t / 8, columns 8 (t % 8) .. 8 (t % 8) + 7.
                    const int i = tid >> 3, j0 = (tid & 7) * 8;
                    float* Sr = A.S + ((size_t)l * NH + h) * HS * HS + (size_t)i * HS + j0;
                    float s[8] = {pS0.x, pS0.y, pS0.z, pS0.w, pS1.x, pS1.y, pS1.z, pS1.w};
                    float pv = 0.0f;
#pragma unroll
                    for (int q = 0; q < 8; ++q) pv = fmaf(s[q], kn_[j0 + q], pv);
                    pv = grp_sum(pv, 8);
                    const float vi = v_[i];
                    float yacc = 0.0f;
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const int j = j0 + q;
                        const float ns = fmaf(s[q], w_[j], vi * k_[j] - pv * (kn_[j] * a_[j]));   // :180-181
                        s[q] = ns;
                        yacc = fmaf(ns, r_[j], yacc);
                    }
                    *reinterpret_cast<float4*>(Sr) = make_float4(s[0], s[1], s[2], s[3]);
                    *reinterpret_cast<float4*>(Sr + 4) = make_float4(s[4], s[5], s[6], s[7]);
                    yacc = grp_sum(yacc, 8);
                    if ((tid & 7) == 0) y_[i] = yacc;
                    __syncthreads();
                    if (tid < HS) {
                        // group norm, bonus, gate (:266-288)
                        const int c = c0 + tid;
                        const float yy = y_[tid];
                        const float mean = wsum(yy) / (float)HS;
                        const float d = yy - mean;
                        const float rstd = 1.0f / sqrtf(wsum(d * d) / (float)HS + kEpsGroup);
                        const float dot = wsum(r_[tid] * k_[tid] * prk);
                        const float n = d * rstd * plw + plb;
                        ex_put(s_y + c, (n + dot * v_[tid]) * hv[2][tid], ep);
                    }
                    return true;
                };
                bool ok;
                if (!uni) ok = owner(std::false_type{}, false);
                else if (q4) ok = owner(std::true_type{}, true);
                else ok = owner(std::false_type{}, true);
                if (!ok) return;
            }
            RKP_MARK(l * 6 + 1, 1);

            // ---- P3: x_a = x + W_o y (:290-292)
            {
                int lo, hi;
                share(D, wg, G, lo, hi);
                const bool ok = with_format<true>(P.o, [&](auto q, auto nu) -> bool {
                    constexpr bool Q = decltype(q)::value;
                    constexpr int NU = decltype(nu)::value;
                    PreRows<Q, NU, 1> pr;
                    pre_load(pr, P.o, lo + wv, NW, lane);
                    issued();
                    __syncthreads();
                    if (!agree(poll_vec<kPer, NT>(s_y, D, buf, pc))) return false;
                    RKP_MARK(l * 6 + 2, 0);
                    // shift_0 <- xn (:229). Every workgroup has read shift_0 by
                    // now: the owners have all of r, k, v and the LoRA middles,
                    // and every workgroup has rows among them (at most as many
                    // workgroups as those rows).
                    if (wg == 0)
                        for (int i = tid; i < D; i += NT) st_ag(sh0 + i, xn[i]);
                    for (int row = lo + wv; row < hi; row += NW) {
                        float d[1];
                        if (row == lo + wv) pre_dot(pr, P.o, buf, lane, d);
                        else d[0] = row_dot(P.o, row, buf, lane);
                        if (lane == 0) ex_put(s_xa + row, xs[row] + d[0], ep);
                    }
                    return true;
                });
                if (!ok) return;
            }
            RKP_MARK(l * 6 + 2, 1);

            // ---- P4: xn2 = LN_2(x_a); xk2 = xn2 + cmk_lerp (shift_1 - xn2); ck = relu(W_ck xk2)^2
            {
                int lo, hi;
                share(F, wg, G, lo, hi);
                const bool ok = with_format<true>(P.cmk, [&](auto q, auto nu) -> bool {
                    constexpr bool Q = decltype(q)::value;
                    constexpr int NU = decltype(nu)::value;
                    // The shift, mix and LayerNorm parameters ahead of the wait
                    // for x_a (they come back within it); the wave's first two
                    // rows after it, overlapped by the LayerNorm (weights ahead
                    // of the wait would hold its first check back).
                    float shv[kPer], lrp[kPer], lg[kPer], lc[kPer];
#pragma unroll
                    for (int k = 0; k < kPer; ++k) {
                        const int ic = min(k * NT + tid, D - 1);
                        shv[k] = ld_ag(sh1 + ic);
                        lrp[k] = P.cmk_lerp[ic];
                    }
                    ln_params(P.ln2w, P.ln2b, D, lg, lc);
                    issued();
                    __syncthreads();
                    if (!agree(poll_vec<kPer, NT>(s_xa, D, xs, pc))) return false;
                    RKP_MARK(l * 6 + 3, 0);
                    PreRows<Q, NU, 2> pr;                   // rows lo + wv and lo + wv + NW
                    pre_load(pr, P.cmk, lo + wv, NW, lane);
                    issued();
                    layer_norm(xs, xn2, lg, lc, D, A.eps, red);
#pragma unroll
                    for (int k = 0; k < kPer; ++k) {
                        const int i = k * NT + tid;
                        if (i < D) buf[i] = xn2[i] + lrp[k] * (shv[k] - xn2[i]);
                    }
                    __syncthreads();
                    for (int row = lo + wv; row < hi; row += 2 * NW) {
                        const int rowB = min(row + NW, hi - 1);
                        float d[2];
                        if (row == lo + wv) pre_dot(pr, P.cmk, buf, lane, d);
                        else row_pair(P.cmk, row, buf, P.cmk, rowB, buf, lane, d[0], d[1]);
                        const float tA = d[0] > 0.0f ? d[0] : 0.0f, tB = d[1] > 0.0f ? d[1] : 0.0f;
                        if (lane == 0) {
                            ex_put(s_ck + row, tA * tA, ep);
                            if (row + NW < hi) ex_put(s_ck + rowB, tB * tB, ep);
                        }
                    }
                    return true;
                });
                if (!ok) return;
            }
            RKP_MARK(l * 6 + 3, 1);

            // ---- P5: x_b = x_a + W_cv ck; shift_1 <- xn2 (:305-315)
            {
                int lo, hi;
                share(D, wg, G, lo, hi);
                const bool ok = with_format(P.cmv, [&](auto q, auto nu) -> bool {
                    constexpr bool Q = decltype(q)::value;
                    constexpr int NU = decltype(nu)::value;
                    PreRows<Q, NU, 1> pr;
                    pre_load(pr, P.cmv, lo + wv, NW, lane);
                    issued();
                    __syncthreads();
                    if (!agree(poll_vec<kPerF, NT>(s_ck, F, buf, pc))) return false;
                    RKP_MARK(l * 6 + 4, 0);
                    // Every workgroup has read shift_1 by now: each has rows of
                    // ck (at most F workgroups).
                    if (wg == 0)
                        for (int i = tid; i < D; i += NT) st_ag(sh1 + i, xn2[i]);
                    for (int row = lo + wv; row < hi; row += NW) {
                        float d[1];
                        if (row == lo + wv) pre_dot(pr, P.cmv, buf, lane, d);
                        else d[0] = row_dot(P.cmv, row, buf, lane);
                        if (lane == 0) ex_put(s_xb + row, xs[row] + d[0], ep);
                    }
                    return true;
                });
                if (!ok) return;
            }
            RKP_MARK(l * 6 + 4, 1);
        }
        RKP_MARK(64 * 6, 0);

        // ---- head: logits = W_head LN_out(x) (:358-359), argmax keys. Passes of
        // N rows per wave alternate between two register sets: the next pass is
        // issued before the current one is multiplied, and the first before x
        // arrives.
        {
            int lo, hi;
            share(A.vocab, wg, G, lo, hi);
            u64 best = 0ull;
            auto head_rows = [&](auto q, auto nrows) -> bool {
                constexpr bool Q = decltype(q)::value;
                constexpr int N = decltype(nrows)::value;
                constexpr int STEP = N * NW;
                PreRows<Q, 1, N> ra, rb;
                float lg[kPer], lc[kPer];
                ln_params(A.on_w, A.on_b, D, lg, lc);
                pre_load(ra, A.head, lo + wv, NW, lane);
                issued();
                __syncthreads();
                if (!agree(poll_vec<kPer, NT>(A.xch + (size_t)(L - 1) * slab + 5 * D, D, xs, pc))) return false;
                layer_norm(xs, buf, lg, lc, D, A.eps, red);
                auto finish = [&](const float (&d)[N], int row) {
#pragma unroll
                    for (int k = 0; k < N; ++k) {
                        const int rk = row + k * NW;
                        if (rk < hi) {
                            if (lane == 0 && last) A.logits[rk] = d[k];
                            best = max(best, argmax_key(d[k], rk));
                        }
                    }
                };
                // A pass is prefetched only when the wave has it (uniform
                // branches): a prefetch past hi would read the next
                // workgroup's rows for nothing and hold the key poll that
                // follows behind its loads.
                for (int row = __builtin_amdgcn_readfirstlane(lo + wv); row < hi; row += 2 * STEP) {
                    if (row + STEP < hi) pre_load(rb, A.head, row + STEP, NW, lane);
                    {
                        float d[N];
                        pre_dot(ra, A.head, buf, lane, d);
                        finish(d, row);
                    }
                    if (row + 2 * STEP < hi) pre_load(ra, A.head, row + 2 * STEP, NW, lane);
                    if (row + STEP < hi) {
                        float d[N];
                        pre_dot(rb, A.head, buf, lane, d);
                        finish(d, row + STEP);
                    }
                }
                return true;
            };
            const bool ok = A.head.block == 0 ? head_rows(std::false_type{}, std::integral_constant<int, 2>{})
                                              : head_rows(std::true_type{}, std::integral_constant<int, 16>{});
            if (!ok) return;
            if (lane == 0) kred[wv] = best;
            __syncthreads();
            if (tid < 2) {
                u64 b = kred[0];
                for (int w = 1; w < NW; ++w) b = max(b, kred[w]);
                ex_put_bits(A.keys + 2 * wg + tid, tid == 0 ? (uint32_t)(b >> 32) : (uint32_t)b, ep);
            }
        }
        RKP_MARK(64 * 6, 1);
        if (!A.greedy) return;   // (one step)
        // ---- every workgroup reduces the keys to the greedy token
        RKP_MARK(64 * 6 + 1, 0);
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
            for (int o = 32; o > 0; o >>= 1) {
                const u64 v = __shfl_xor(b, o, 64);
                b = max(b, v);
            }
            if (lane == 0) kred[wv] = b;
            __syncthreads();
            u64 m = kred[0];
            for (int w2 = 1; w2 < NW; ++w2) m = max(m, kred[w2]);
            tok = (int)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull));
            const long hrow = (long)(cnt0 + st) * NI + sq;
            if (wg == 0 && tid == 0 && hrow < A.hist_cap) A.tok_hist[hrow] = tok;
        }
    }   // steps
    if (wg == 0 && tid == 0) {
        *A.tok = tok;
        if (sq == 0) *A.counter = cnt0 + A.nsteps;
    }
}

}  // namespace

bool rkp_shape_ok(int D, int F, int HS_, int NH, const int (*ranks)[4], int L) {
    if (HS_ != HS || D % HS || NH != D / HS || D > kRkPMaxD || D % 16 || F > kRkPMaxF || F % 16 || L < 1)
        return false;
    for (int l = 0; l < L; ++l)
        for (int j = 0; j < 4; ++j) {
            const int r = ranks[l][j];
            if (r < 16 || r > kRkPRank || (r & (r - 1))) return false;
        }
    return true;
}

#ifdef SNHIP_RKP_PROF
extern "C" int snhip_rkp_prof(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_rkp_prof), sizeof(g_rkp_prof)) == hipSuccess ? 0 : 1;
}
#endif

int rkp_grid(int NH) {
    int dev = 0, coop = 0, ncu = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(k_rk_persist), NT, 0) !=
            hipSuccess || occ < 1)
        return 0;
    const int G = (ncu / 8) * 8;
    return G >= 8 && G >= NH ? G : 0;
}

snhip_status launch_rk_persist(const RkPArgs& a, int G, hipStream_t st) {
    const int ni = a.ni > 1 ? a.ni : 1;
    if (G % ni || G / ni < 8 || (G / ni) % 8 || G / ni < a.NH || G > kRkPMaxGrid ||
        (ni > 1 && a.words < (size_t)a.L * rkp_slab(a.D, a.F) + 2 * (size_t)(G / ni))) {
        set_last_error("RWKV-7 persistent step: bad grid");
        return SNHIP_E_INVAL;
    }
    RkPArgs args = a;
    void* kargs[] = {&args};
    SNHIP_CHECK(launch_persistent(reinterpret_cast<const void*>(k_rk_persist), dim3(G), dim3(NT), kargs, st));
    return SNHIP_OK;
}

}  // namespace snhip
