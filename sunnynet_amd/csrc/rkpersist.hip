// RWKV-7 decode step for one sequence as one cooperative launch
// (sunnynet/runtime/rwkv7.c:143-360; the math is the one listed at the top of
// rwkv.hip).
//
// At one sequence the step is a chain of small matrix-vector products; run as
// separate kernels (even replayed from a graph) each costs about 4.6 us of
// launch and drain on gfx950 whatever its size, about 100 of them per step.
// Here one launch runs the whole step: one 512-thread workgroup per CU, the
// products' rows spread over every wave of the grid, and a grid barrier
// between the phases that depend on a whole vector. Five phases per layer:
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
// then LN_out and the head rows with a per-workgroup argmax key, and workgroup
// 0 reduces the keys to the greedy token. Every vector a phase produces has
// its own slot in a per-layer slab and is written once per launch with
// agent-scope stores, so after the barrier (each wave's stores complete
// before it arrives) plain loads read it from any XCD; the kernel boundary
// orders one step's writes before the next step's reads. The recurrent state
// (S, the two shift vectors, v_first) is read and written only by the
// workgroup that owns it.
#include <type_traits>

#include "gemv.h"
#include "rkpersist.h"

namespace snhip {
namespace {

constexpr int NT = 512, NW = NT / 64, HS = 64;
constexpr float kR2 = 0.6065306597126334f;   // 1/sqrt(e), rwkv7.c:38
constexpr float kEpsGroup = 6.4e-4f;          // rwkv7.c:39
constexpr int kPer = kRkPMaxD / NT;           // LayerNorm values per thread
typedef unsigned long long u64;

template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> glb(const T* p) { return (gptr<T>)p; }

__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ void st_ag(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
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

// y[i] = LN(x)[i] * g[i] + c[i] over n <= kRkPMaxD values in LDS
// (rwkv7.c:127-140 form, two passes).
__device__ void layer_norm(const float* x, float* y, const float* g, const float* c, int n, float eps,
                           float* red) {
    float v[kPer], gv[kPer], cv[kPer];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = k * NT + threadIdx.x, ic = min(i, n - 1);
        gv[k] = g[ic];
        cv[k] = c[ic];
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
        for (int o = nu >> 1; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (i < n && u == 0) out[i] = acc;
    }
}

// Grid barrier in two halves (two levels: eight group counters, then one top
// counter and a flag). Arrival waits for this wave's stores (and loads: the
// wait count covers both), so loads that do not depend on the barrier are
// issued between arrival and the wait. The wait is true when it timed out
// and the launch is abandoned.
__device__ __forceinline__ void bar_arrive(u64* bar, unsigned& gen, int wg, int G, int* slast) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    ++gen;
    if (threadIdx.x == 0) {
        u64* grp = bar + 32 * (1 + (wg & 7));
        const int ng = G >> 3;
        int last = 0;
        const u64 old = __hip_atomic_fetch_add(grp, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == (u64)gen * ng - 1) {
            const u64 o2 = __hip_atomic_fetch_add(bar, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = o2 == (u64)gen * 8 - 1;
        }
        if (last) __hip_atomic_store(bar + 32 * 9, (u64)gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *slast = last;
    }
}

__device__ __forceinline__ bool bar_wait(u64* bar, unsigned* err, unsigned limit, unsigned stall, unsigned gen,
                                         int* slast, int* sdead) {
    if (threadIdx.x == 0) {
        int dead = 0;
        if (!*slast) {
            unsigned n = 0;
            while (__hip_atomic_load(bar + 32 * 9, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
                   (u64)gen + stall) {
                if (++n > limit) {
                    __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    dead = 1;
                    break;
                }
                if ((n & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    dead = 1;
                    break;
                }
            }
        }
        *sdead = dead;
    }
    __syncthreads();
    return *sdead != 0;
}

// Keeps loads issued so far where they are (the optimizer would sink them to
// their use, past the barrier wait).
__device__ __forceinline__ void issued() { asm volatile("" ::: "memory"); }

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

// This workgroup's share [lo, hi) of n rows.
__device__ __forceinline__ void share(int n, int wg, int G, int& lo, int& hi) {
    lo = (int)((long)n * wg / G);
    hi = (int)((long)n * (wg + 1) / G);
}

__global__ __launch_bounds__(NT) void k_rk_persist(RkPArgs A) {
    __shared__ float xs[kRkPMaxD];            // x entering the phase
    __shared__ float xn[kRkPMaxD];            // LN_1(x) of this layer
    __shared__ float xn2[kRkPMaxD];           // LN_2(x_a)
    __shared__ float buf[6 * kRkPMaxD];       // X6 | ck | head inputs
    __shared__ float hv[12][HS];              // per-channel values of the owned head
    __shared__ float red[NW];
    __shared__ u64 kred[NW];
    __shared__ int sdead, slast;
    __shared__ RkPLayer Ls;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wg = blockIdx.x, G = gridDim.x;
    const int D = A.D, F = A.F, L = A.L, NH = A.NH;
    const size_t slab = rkp_slab(D, F);
    unsigned gen = A.gen0;

    // x = LN_0(E[tok]) (rwkv7.c:351-352); NaN for an out-of-range id.
    {
        const int t = *A.tok;
        const bool ok = t >= 0 && t < A.vocab;
        const float* er = A.embed + (size_t)(ok ? t : 0) * D;
        for (int i = tid; i < D; i += NT) buf[i] = ok ? er[i] : __builtin_nanf("");
        __syncthreads();
        layer_norm(buf, xs, A.en_w, A.en_b, D, A.eps, red);
    }

    for (int l = 0; l < L; ++l) {
        if (tid < (int)(sizeof(RkPLayer) / 4))
            reinterpret_cast<int*>(&Ls)[tid] = reinterpret_cast<const int*>(A.layers + l)[tid];
        float* sl = A.xch + (size_t)l * slab;
        float *s_r = sl, *s_k = sl + D, *s_v = sl + 2 * D, *s_y = sl + 3 * D, *s_xa = sl + 4 * D,
              *s_xb = sl + 5 * D, *s_lw = sl + 6 * D, *s_la = s_lw + kRkPRank, *s_lg = s_la + kRkPRank,
              *s_lv = s_lg + kRkPRank, *s_ck = s_lv + kRkPRank;
        float* sh0 = A.shift + (size_t)l * 2 * D;
        float* sh1 = sh0 + D;
        if (l > 0) {
            const float* xb = A.xch + (size_t)(l - 1) * slab + 5 * D;
            for (int i = tid; i < D; i += NT) xs[i] = xb[i];
        }
        __syncthreads();
        const RkPLayer& P = Ls;

        // ---- P1: xn = LN_1(x); X6 = xn + lerp (shift_0 - xn); r k v, LoRA down
        RKP_MARK(l * 6 + 0, 0);
        {
            float shv[kPer], lrp[6][kPer];      // loaded before the LayerNorm
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int ic = min(k * NT + tid, D - 1);
                shv[k] = sh0[ic];
#pragma unroll
                for (int s6 = 0; s6 < 6; ++s6) lrp[s6][k] = P.lerp[(size_t)s6 * D + ic];
            }
            layer_norm(xs, xn, P.ln1w, P.ln1b, D, A.eps, red);
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int i = k * NT + tid;
                if (i < D) {
                    const float d = shv[k] - xn[i];
#pragma unroll
                    for (int s6 = 0; s6 < 6; ++s6) buf[s6 * D + i] = xn[i] + lrp[s6][k] * d;
                }
            }
        }
        __syncthreads();
        {
            const int xoff[7] = {0, 2 * D, 3 * D, D, 4 * D, 5 * D, 3 * D};
            float* outs[7] = {s_r, s_k, s_v, s_lw, s_la, s_lg, s_lv};
            const int nseg = l > 0 ? 7 : 6;
            int total = 0;
            for (int s = 0; s < nseg; ++s) total += p1_mat(P, s).M;
            int lo, hi;
            share(total, wg, G, lo, hi);
            for (int row = lo + wv; row < hi; row += 2 * NW) {
                const int rowB = min(row + NW, hi - 1);
                int sA = 0, rA = row, sB = 0, rB = rowB;
                while (rA >= p1_mat(P, sA).M) rA -= p1_mat(P, sA++).M;
                while (rB >= p1_mat(P, sB).M) rB -= p1_mat(P, sB++).M;
                float dA, dB;
                row_pair(p1_mat(P, sA), rA, buf + xoff[sA], p1_mat(P, sB), rB, buf + xoff[sB], lane, dA, dB);
                if (lane == 0) {
                    st_ag(outs[sA] + rA, dA);
                    if (row + NW < hi) st_ag(outs[sB] + rB, dB);
                }
            }
        }
        RKP_MARK(l * 6 + 0, 1);
        // Head owners load their state rows and channel parameters while the
        // barrier completes (none depends on it).
        f4 pS0 = {0, 0, 0, 0}, pS1 = {0, 0, 0, 0};
        float pw0 = 0, pv0 = 0, pa0 = 0, pkk = 0, pka = 0, prk = 0, plw = 0, plb = 0, pvf = 0;
        bar_arrive(A.bar, gen, wg, G, &slast);
        if (wg < NH) {
            const gptr<f4> Sp = (gptr<f4>)(glb(A.S) + ((size_t)l * NH + wg) * HS * HS + (size_t)(tid >> 3) * HS +
                                           (tid & 7) * 8);
            pS0 = Sp[0];
            pS1 = Sp[1];
            const int c = wg * HS + (tid & 63);
            pw0 = glb(P.w0)[c]; pv0 = glb(P.v0)[c]; pa0 = glb(P.a0)[c]; pkk = glb(P.kk)[c];
            pka = glb(P.ka)[c]; prk = glb(P.rk)[c]; plw = glb(P.lnxw)[c]; plb = glb(P.lnxb)[c];
            // v_first is rewritten by this workgroup in layer 0 of every launch:
            // read it past the caches.
            pvf = __hip_atomic_load(A.vfirst + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        issued();
        if (bar_wait(A.bar, A.err, A.spin_limit, A.stall, gen, &slast, &sdead)) return;
        RKP_MARK(l * 6 + 1, 0);

        // ---- P2: head h = wg (rwkv7.c:143-189, 229-299)
        if (wg == 0)
            for (int i = tid; i < D; i += NT) sh0[i] = xn[i];        // shift_0 <- xn (:229)
        if (wg < NH) {
            const int h = wg, c0 = h * HS;
            const int Rw = P.w1.M, Ra = P.a1.M, Rg = P.g1.M, Rv = P.v1.M;
            float* in_w = buf;                  // tanh(lw)
            float* in_a = buf + kRkPRank;       // la
            float* in_g = buf + 2 * kRkPRank;   // sig(lg)
            float* in_v = buf + 3 * kRkPRank;   // lv
            for (int i = tid; i < kRkPRank; i += NT) {
                if (i < Rw) in_w[i] = tanhf(s_lw[i]);
                if (i < Ra) in_a[i] = s_la[i];
                if (i < Rg) in_g[i] = sgm(s_lg[i]);
                if (l > 0 && i < Rv) in_v[i] = s_lv[i];
            }
            __syncthreads();
            small_rows(P.w2, c0, HS, in_w, hv[0], wv, lane);     // dw
            small_rows(P.a2, c0, HS, in_a, hv[1], wv, lane);     // da
            small_rows(P.g2, c0, HS, in_g, hv[2], wv, lane);     // g
            if (l > 0) small_rows(P.v2, c0, HS, in_v, hv[3], wv, lane);   // dv
            __syncthreads();
            float* w_ = hv[4]; float* k_ = hv[5]; float* v_ = hv[6]; float* a_ = hv[7];
            float* kn_ = hv[8]; float* r_ = hv[9]; float* y_ = hv[10];
            if (tid < HS) {
                const int c = c0 + tid;
                const float ww = expf(-sgm(hv[0][tid] + pw0) * kR2);            // :236-237
                float vv = s_v[c];
                if (l == 0) {
                    st_ag(A.vfirst + c, vv);                                     // :240
                } else {
                    const float mix = sgm(hv[3][tid] + pv0);                     // :244-246
                    vv = vv + (pvf - vv) * mix;
                }
                const float av = sgm(hv[1][tid] + pa0);                         // :251-252
                const float kv = s_k[c];
                const float kkv = kv * pkk;                                      // :259
                const float k2 = kv + kv * (av - 1.0f) * pka;                   // :260
                float nrm = sqrtf(wsum(kkv * kkv));                              // :158-162
                if (!(nrm > 1e-12f)) nrm = 1e-12f;
                w_[tid] = ww; k_[tid] = k2; v_[tid] = vv; a_[tid] = av; kn_[tid] = kkv * (1.0f / nrm);
                r_[tid] = s_r[c];
            }
            __syncthreads();
            // S = S diag(w) - (S kk^)(kk^ a)^T + v k^T; y = S r. Thread t owns
            // row i = t / 8, columns 8 (t % 8) .. 8 (t % 8) + 7.
            const int i = tid >> 3, j0 = (tid & 7) * 8;
            float* Sr = A.S + ((size_t)l * NH + h) * HS * HS + (size_t)i * HS + j0;
            float s[8] = {pS0.x, pS0.y, pS0.z, pS0.w, pS1.x, pS1.y, pS1.z, pS1.w};
            float pv = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) pv = fmaf(s[q], kn_[j0 + q], pv);
            pv += __shfl_xor(pv, 1, 64);
            pv += __shfl_xor(pv, 2, 64);
            pv += __shfl_xor(pv, 4, 64);
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
            yacc += __shfl_xor(yacc, 1, 64);
            yacc += __shfl_xor(yacc, 2, 64);
            yacc += __shfl_xor(yacc, 4, 64);
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
                st_ag(s_y + c, (n + dot * v_[tid]) * hv[2][tid]);
            }
        }
        RKP_MARK(l * 6 + 1, 1);
        bar_arrive(A.bar, gen, wg, G, &slast);
        if (bar_wait(A.bar, A.err, A.spin_limit, A.stall, gen, &slast, &sdead)) return;
        RKP_MARK(l * 6 + 2, 0);

        // ---- P3: x_a = x + W_o y (:290-292)
        for (int i = tid; i < D; i += NT) buf[i] = s_y[i];
        __syncthreads();
        {
            int lo, hi;
            share(D, wg, G, lo, hi);
            for (int row = lo + wv; row < hi; row += NW) {
                const float d = row_dot(P.o, row, buf, lane);
                if (lane == 0) st_ag(s_xa + row, xs[row] + d);
            }
        }
        RKP_MARK(l * 6 + 2, 1);
        bar_arrive(A.bar, gen, wg, G, &slast);
        if (bar_wait(A.bar, A.err, A.spin_limit, A.stall, gen, &slast, &sdead)) return;
        RKP_MARK(l * 6 + 3, 0);

        // ---- P4: xn2 = LN_2(x_a); xk2 = xn2 + cmk_lerp (shift_1 - xn2); ck = relu(W_ck xk2)^2
        for (int i = tid; i < D; i += NT) xs[i] = s_xa[i];
        __syncthreads();
        {
            float shv[kPer], lrp[kPer];
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int ic = min(k * NT + tid, D - 1);
                shv[k] = sh1[ic];
                lrp[k] = P.cmk_lerp[ic];
            }
            layer_norm(xs, xn2, P.ln2w, P.ln2b, D, A.eps, red);
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int i = k * NT + tid;
                if (i < D) buf[i] = xn2[i] + lrp[k] * (shv[k] - xn2[i]);
            }
        }
        __syncthreads();
        {
            int lo, hi;
            share(F, wg, G, lo, hi);
            for (int row = lo + wv; row < hi; row += 2 * NW) {
                const int rowB = min(row + NW, hi - 1);
                float dA, dB;
                row_pair(P.cmk, row, buf, P.cmk, rowB, buf, lane, dA, dB);
                const float tA = dA > 0.0f ? dA : 0.0f, tB = dB > 0.0f ? dB : 0.0f;
                if (lane == 0) {
                    st_ag(s_ck + row, tA * tA);
                    if (row + NW < hi) st_ag(s_ck + rowB, tB * tB);
                }
            }
        }
        RKP_MARK(l * 6 + 3, 1);
        bar_arrive(A.bar, gen, wg, G, &slast);
        if (bar_wait(A.bar, A.err, A.spin_limit, A.stall, gen, &slast, &sdead)) return;
        RKP_MARK(l * 6 + 4, 0);

        // ---- P5: x_b = x_a + W_cv ck; shift_1 <- xn2 (:305-315)
        if (wg == 0)
            for (int i = tid; i < D; i += NT) sh1[i] = xn2[i];
        for (int i = tid; i < F; i += NT) buf[i] = s_ck[i];
        __syncthreads();
        {
            int lo, hi;
            share(D, wg, G, lo, hi);
            for (int row = lo + wv; row < hi; row += NW) {
                const float d = row_dot(P.cmv, row, buf, lane);
                if (lane == 0) st_ag(s_xb + row, xs[row] + d);
            }
        }
        RKP_MARK(l * 6 + 4, 1);
        bar_arrive(A.bar, gen, wg, G, &slast);
        if (bar_wait(A.bar, A.err, A.spin_limit, A.stall, gen, &slast, &sdead)) return;
    }
    RKP_MARK(64 * 6, 0);

    // ---- head: logits = W_head LN_out(x) (:358-359), argmax keys
    {
        const float* xb = A.xch + (size_t)(L - 1) * slab + 5 * D;
        for (int i = tid; i < D; i += NT) xs[i] = xb[i];
        __syncthreads();
        layer_norm(xs, buf, A.on_w, A.on_b, D, A.eps, red);
        int lo, hi;
        share(A.vocab, wg, G, lo, hi);
        u64 best = 0ull;
        auto head_rows = [&](auto q, auto nrows) {
            constexpr bool Q = decltype(q)::value;
            constexpr int N = decltype(nrows)::value;
            for (int row = lo + wv; row < hi; row += N * NW) {
                float d[N];
                row_dotn<Q, N>(A.head, row, NW, hi, buf, lane, d);
#pragma unroll
                for (int k = 0; k < N; ++k) {
                    const int rk = row + k * NW;
                    if (rk < hi) {
                        if (lane == 0) A.logits[rk] = d[k];
                        best = max(best, argmax_key(d[k], rk));
                    }
                }
            }
        };
        if (A.head.block == 0) head_rows(std::false_type{}, std::integral_constant<int, 4>{});
        else head_rows(std::true_type{}, std::integral_constant<int, 16>{});
        if (lane == 0) kred[wv] = best;
        __syncthreads();
        if (tid == 0) {
            u64 b = kred[0];
            for (int w = 1; w < NW; ++w) b = max(b, kred[w]);
            __hip_atomic_store(A.keys + wg, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    RKP_MARK(64 * 6, 1);
    if (!A.greedy) return;
    bar_arrive(A.bar, gen, wg, G, &slast);
        if (bar_wait(A.bar, A.err, A.spin_limit, A.stall, gen, &slast, &sdead)) return;
    RKP_MARK(64 * 6 + 1, 0);
    if (wg == 0) {
        u64 b = 0ull;
        for (int i = tid; i < G; i += NT) b = max(b, A.keys[i]);
        for (int o = 32; o > 0; o >>= 1) {
            const u64 v = __shfl_xor(b, o, 64);
            b = max(b, v);
        }
        if (lane == 0) kred[wv] = b;
        __syncthreads();
        if (tid == 0) {
            u64 m = kred[0];
            for (int w = 1; w < NW; ++w) m = max(m, kred[w]);
            const int32_t tk = (int32_t)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull));
            const int step = *A.counter;
            *A.tok = tk;
            if (step < A.hist_cap) A.tok_hist[step] = tk;
            *A.counter = step + 1;
        }
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
    if (G < 8 || G % 8 || G < a.NH) {
        set_last_error("RWKV-7 persistent step: bad grid");
        return SNHIP_E_INVAL;
    }
    RkPArgs args = a;
    void* kargs[] = {&args};
    SNHIP_CHECK(launch_persistent(reinterpret_cast<const void*>(k_rk_persist), dim3(G), dim3(NT), kargs, st));
    return SNHIP_OK;
}

}  // namespace snhip
