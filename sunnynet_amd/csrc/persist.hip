// Persistent decode of one sequence: every layer of every step in one
// cooperative launch (the B = 1 path of snhip_step / snhip_decode_greedy_dev).
//
// The math is the decode step of sunnynet/runtime/sunnynet.c:212-334, in the
// same operation order as the per-kernel path (model.hip). A step is a chain
// of small matrix-vector products, each too short to fill the chip as its own
// launch; here the whole grid (one workgroup per CU) walks through the step in
// phases separated by grid barriers:
//
//   A  LN_in(x), depthwise conv -> at;  v = V at,  sfb = W_eff s      (all WGs)
//   B  q = U v for one group of 8 channels per WG (16 contiguous rows of U:
//      8 value, 8 gate),
//      competitive + decay gate, s' = p s + (1 - p) u, conv history shift
//   C  z = wedge(W_z u)
//   D  y = LN_I(z);  x = W_c y + b s' + sfb + x
//   H  logits = E LN_out(x), per-WG argmax key;  then every WG reduces the
//      keys to the same greedy token, the next step's input.
//
// 4 L + 1 barriers per step. A barrier is split into arrive and wait; between
// the two, the loads that do not depend on the phase that just ended are
// issued: the dot waves load the weights of their first two batches of rows
// of the next phase (and b s' + sfb + x for phase D), the staging wave the
// inputs produced two or more phases earlier (the state s and conv-history
// products for phase A, the old state and history for phase B) and the next
// LayerNorm's gain and bias. After the wait only the previous phase's output
// is fetched. Conv history: the phase-B owner of a channel also stores
// hd[k] = hist'[k] * dw[K-2-k] for the next step, so phase A forms
// acc = raw * dw[K-1] + hd[0] + hd[1] + ... in the reference's order
// (sunnynet.c:227-233) with the products already rounded, bit-identical.
//
// Values exchanged between workgroups (x, v, sfb, u, z, s, hist, hd, the
// argmax keys) are written and read with agent-scope atomic accesses
// (global_load / global_store with sc1 on gfx950): the per-XCD L2 caches are
// not coherent with each other, and plain loads would see stale lines. Each
// wave drains its stores (s_waitcnt 0) before the workgroup arrives at a
// barrier. Weights and other read-only data use ordinary cached loads.
//
// The barrier is two-level: workgroup g counts on group counter g & 7 (128
// bytes apart, one per XCD under round-robin dispatch); the last arrival of a
// group bumps the top counter that every workgroup polls. Counters only grow
// (targets are epoch multiples), so no reset is needed inside the launch. Every
// poll loop is bounded: on time-out the flag word is set and every workgroup
// leaves the kernel at its next barrier.
#include "decode.h"

namespace snhip {
namespace {

constexpr int NT = 256;                      // threads per workgroup (4 waves)
constexpr int kMaxD = kPersistMaxD;          // dim
constexpr int kMaxK = kPersistMaxK;          // inner, rank
constexpr int PD = kMaxD / NT;               // values per thread of a dim-wide vector
constexpr int PI = kMaxK / NT;               // of an inner- or rank-wide vector
constexpr int PH = 8;                        // fp32: float4 per lane in one batch
constexpr int MUH_MAX = 8;                   // INT4: units in one batch (32-wide groups;
template <int BLK> constexpr int muh() { return BLK == 64 ? 4 : MUH_MAX; }   // half for 64)

// Read-only data through global-address-space pointers: global_load (counted
// by vmcnt only). Through a generic pointer the compiler emits flat loads,
// which also count against lgkmcnt, so the first LDS wait after a prefetch
// would stall until every prefetched weight had arrived.
// (Native vector types: HIP's float4 / uint4 are classes whose copy goes
// through a generic reference and would lose the address space.)
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const float g_f32;
typedef __attribute__((address_space(1))) const f32x4v g_f32x4;
typedef __attribute__((address_space(1))) const u32x4v g_u32x4;
__device__ __forceinline__ float ldg(const float* p) { return *(g_f32*)p; }
__device__ __forceinline__ float4 ldg4(const float* p) {
    const f32x4v v = *(g_f32x4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldgq(const uint8_t* p) {
    const u32x4v v = *(g_u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
// The layer table never changes during a launch: read through the constant
// address space it becomes scalar loads (counted by lgkmcnt), so fetching a
// layer's pointers does not wait for the vector loads in flight.
#if defined(__HIP_DEVICE_COMPILE__)
typedef __attribute__((address_space(4))) const PLayer c_layer;
#else
typedef const PLayer c_layer;   // host pass of the kernel source
#endif
// LDS activations are addressed the same way (ds_read, not flat).
typedef __attribute__((address_space(3))) const float l_f32;
typedef __attribute__((address_space(3))) const f32x4v l_f32x4;
__device__ __forceinline__ float4 lds4(l_f32x4* p) {
    const f32x4v v = *p;
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float ldc(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }

// The same value, opaque to the optimizer. Applied to the thread index at
// every phase boundary so per-lane addresses are formed inside each phase
// instead of being hoisted out of the step loop (where hundreds of them
// would stay live and spill).
__device__ __forceinline__ int opq(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Sum over the lane's 16-lane row, in every lane of the row: a rotation
// butterfly with DPP row_ror 8, 4, 2, 1 (pairs are symmetric and the adds
// commutative, so every lane ends with the same value).
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_sum(float v) {
    v += dppf<0x128>(v);   // row_ror:8
    v += dppf<0x124>(v);   // row_ror:4
    v += dppf<0x122>(v);   // row_ror:2
    v += dppf<0x121>(v);   // row_ror:1
    return v;
}
__device__ __forceinline__ float lane_val(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Whole-wave sum (wave-uniform result).
__device__ __forceinline__ float wsum(float v) {
    v = row_sum(v);
    return (lane_val(v, 0) + lane_val(v, 16)) + (lane_val(v, 32) + lane_val(v, 48));
}

__device__ __forceinline__ unsigned long long kmax_wave(unsigned long long k) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long other =
            ((unsigned long long)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
            (uint32_t)__shfl_xor((int)(k & 0xFFFFFFFFull), o, 64);
        k = max(k, other);
    }
    return k;
}

// Orderable key of (value, index): larger value wins, then smaller index
// (torch.argmax's first maximal index, sunnynet/cli.py:41).
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

__device__ __forceinline__ float bsum(float v, float* red) {
    v = wsum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Two-pass LayerNorm statistics (sunnynet.c:198-210 form) over n values,
// element k * NT + tid held in xv[k].
template <int N>
__device__ __forceinline__ void ln_stats(const float (&xv)[N], int n, float eps, int tid, float* red,
                                         float& mean, float& rstd) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (k * NT + tid < n) sum += xv[k];
    mean = bsum(sum, red) / (float)n;
    float vs = 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (k * NT + tid < n) {
            const float d = xv[k] - mean;
            vs += d * d;
        }
    rstd = 1.0f / sqrtf(bsum(vs, red) / (float)n + eps);
}

// Issue agent-scope loads of n values (element k * NT + tid in v[k]); the
// caller consumes them later.
template <int N>
__device__ __forceinline__ void issue_ldc(float (&v)[N], const float* src, int n, int tid) {
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (k * NT < n) v[k] = ldc(src + min(k * NT + tid, n - 1));
}
template <int N>
__device__ __forceinline__ void issue_ldg(float (&v)[N], const float* src, int n, int tid) {
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (k * NT < n) v[k] = ldg(src + min(k * NT + tid, n - 1));
}

// Keeps the scheduler from moving instructions across this point, so loads
// stay in the issue order the kernel relies on (vmcnt drains in order).
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

// One phase's matrix-vector work: rows of one matrix W with contraction
// length Kd, split in units; rows below `split` multiply x0, the others x1.
// fp32: a unit is one row; a lane holds float4 i of a row at k = i * 256 +
// 4 * lane (nk4 of them, rounded up to a power of two), a batch holds
// PH / nk4 rows. INT4: a unit is rpp rows, one per segment of seg lanes, each
// lane one group of BLK inputs; a batch holds MUH units. This wave takes units
// u0, u0 + ustride, ... in batches; two batches are in registers at a time.
struct PhaseDesc {
    PMat W;
    int nu, split;
    int Kd, nk4, lg4, ng, seg, rpp, rpb;
    l_f32* x0;              // LDS activation of rows < split (staged layout)
    l_f32* x1;              // of rows >= split
    int u0, ustride, nb;    // first unit, stride, batches
};

// A row's epilogue pre-loads (phase D: s', sfb, x).
struct Pre3 {
    float s, f, x;
};

// Epilogue inputs read with the weights (phase D): s', sfb and x per row.
struct EpiPre {
    const float* s;         // s' (new state) of the layer, or NULL: no pre-loads
    const float* sfb;
    const float* x;         // residual input
};

constexpr int EPS = 2;                       // slots per batch with epilogue pre-loads

template <int BLK>
struct Pool {
    static constexpr int MUH = muh<BLK>();
    static constexpr int QW = BLK ? BLK / 32 : 1;    // uint4 per INT4 group
    static constexpr int MS = BLK ? MUH : PH;        // slots (rows / units) per batch
    float4 wf[2][BLK ? 1 : PH];
    uint4 wq[2][BLK ? MUH : 1][QW];
    float wsc[2][BLK ? MUH : 1];
    float ep[2][EPS][3];
    bool ep_on[2];
    int unit[2][MS];                                 // -1: empty slot

    // Batch b of P into half h. Straight-line code with the same loads on
    // every path (empty slots and lanes read element 0 of the matrix), so the
    // compiler's wait counts for earlier loads stay exact. EP: also s', sfb,
    // x of the batch's first EPS rows.
    template <bool EP>
    __device__ __forceinline__ void load(const PhaseDesc& P, int h, int b, int lane, const EpiPre& E) {
        const bool bok = b < P.nb;
        ep_on[h] = EP;
        if constexpr (BLK == 0) {
            const int sh = P.lg4;
#pragma unroll
            for (int j = 0; j < PH; ++j) {
                const int r = j >> sh, i = j & ((1 << sh) - 1);
                const int u = P.u0 + (b * P.rpb + r) * P.ustride;
                const bool ok = bok && r < P.rpb && u < P.nu;
                const int k = i * 256 + lane * 4;
                wf[h][j] = ldg4(P.W.w + ((ok && k < P.Kd) ? (size_t)u * P.Kd + k : 0));
            }
#pragma unroll
            for (int r = 0; r < PH; ++r) {
                const int u = P.u0 + (b * P.rpb + r) * P.ustride;
                unit[h][r] = (bok && r < P.rpb && u < P.nu) ? u : -1;
            }
            if constexpr (EP) {
#pragma unroll
                for (int r = 0; r < EPS; ++r) {
                    const int u = unit[h][r] < 0 ? 0 : unit[h][r];
                    ep[h][r][0] = ldc(E.s + u);
                    ep[h][r][1] = ldc(E.sfb + u);
                    ep[h][r][2] = ldc(E.x + u);
                }
            }
        } else {
            const int lrow = lane / P.seg, lg = lane - lrow * P.seg;
#pragma unroll
            for (int s = 0; s < MUH; ++s) {
                const int u = P.u0 + (b * MUH + s) * P.ustride;
                const bool uok = bok && u < P.nu;
                unit[h][s] = uok ? u : -1;
                const int r = u * P.rpp + lrow;
                const bool ok = uok && r < P.W.M && lg < P.ng;
                const uint8_t* qr = P.W.q + (ok ? (size_t)r * (P.Kd / 2) + lg * (BLK / 2) : 0);
#pragma unroll
                for (int q = 0; q < QW; ++q) wq[h][s][q] = ldgq(qr + 16 * q);
                wsc[h][s] = ldg(P.W.sc + (ok ? (size_t)r * P.ng + lg : 0));
                if constexpr (EP) {
                    if (s < EPS) {
                        const int rr = (uok && r < P.W.M) ? r : 0;
                        ep[h][s][0] = ldc(E.s + rr);
                        ep[h][s][1] = ldc(E.sfb + rr);
                        ep[h][s][2] = ldc(E.x + rr);
                    }
                }
            }
        }
    }

    // epi(row, value, writer, pre, has_pre): the row's dot product; `writer`
    // is true on exactly one lane per row; pre = the row's epilogue pre-loads
    // when has_pre.
    template <int NK4, class Epi>
    __device__ __forceinline__ void compute_f32(const PhaseDesc& P, int h, int lane, Epi&& epi) {
        constexpr int RPB = PH / NK4;
        float acc[RPB];
#pragma unroll
        for (int r = 0; r < RPB; ++r) {
            acc[r] = 0.0f;
            if (unit[h][r] < 0) continue;
            l_f32* xs = unit[h][r] < P.split ? P.x0 : P.x1;
#pragma unroll
            for (int i = 0; i < NK4; ++i) {
                const int k = i * 256 + lane * 4;
                if (k < P.Kd) {
                    const float4 x4 = lds4((l_f32x4*)(xs + k));
                    const float4 w4 = wf[h][r * NK4 + i];
                    acc[r] = fmaf(w4.x, x4.x, acc[r]);
                    acc[r] = fmaf(w4.y, x4.y, acc[r]);
                    acc[r] = fmaf(w4.z, x4.z, acc[r]);
                    acc[r] = fmaf(w4.w, x4.w, acc[r]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPB; ++r) acc[r] = row_sum(acc[r]);
#pragma unroll
        for (int r = 0; r < RPB; ++r)
            acc[r] = (lane_val(acc[r], 0) + lane_val(acc[r], 16)) + (lane_val(acc[r], 32) + lane_val(acc[r], 48));
#pragma unroll
        for (int r = 0; r < RPB; ++r)
            if (unit[h][r] >= 0) {
                const bool hp = ep_on[h] && r < EPS;
                const int re = r < EPS ? r : 0;
                epi(unit[h][r], acc[r], lane == 0, Pre3{ep[h][re][0], ep[h][re][1], ep[h][re][2]}, hp);
            }
    }

    template <class Epi>
    __device__ __forceinline__ void compute_i4(const PhaseDesc& P, int h, int lane, Epi&& epi) {
        const int lrow = lane / P.seg, lg = lane - lrow * P.seg;
        constexpr int NW = BLK / 8;                  // 32-bit words of codes per group
        float acc[MUH];
#pragma unroll
        for (int s = 0; s < MUH; ++s) {
            acc[s] = 0.0f;
            const int r = unit[h][s] * P.rpp + lrow;
            if (unit[h][s] < 0 || r >= P.W.M || lg >= P.ng) continue;
            l_f32x4* x4 = (l_f32x4*)(r < P.split ? P.x0 : P.x1);
            const float sc = wsc[h][s];
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const uint4& qq = wq[h][s][w >> 2];
                const int wi = w & 3;
                const uint32_t word = wi == 0 ? qq.x : wi == 1 ? qq.y : wi == 2 ? qq.z : qq.w;
                // Byte 4w + e holds element 4w + e (low nibble) and
                // 4w + e + BLK/2 (high nibble); quant.c:82-83 dequantization.
                const float4 xl = lds4(x4 + w * P.ng + lg);
                const float4 xh = lds4(x4 + (w + NW) * P.ng + lg);
                const float xlo[4] = {xl.x, xl.y, xl.z, xl.w};
                const float xhi[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t byte = (word >> (8 * e)) & 0xFFu;
                    const float wl = (float)((int)(byte & 0x0Fu) - 8) * sc;
                    const float wh = (float)((int)(byte >> 4) - 8) * sc;
                    acc[s] = fmaf(wl, xlo[e], acc[s]);
                    acc[s] = fmaf(wh, xhi[e], acc[s]);
                }
            }
        }
        if (P.seg >= 16) {
            // rows of 16 lanes by DPP, then the rows of each segment
#pragma unroll
            for (int s = 0; s < MUH; ++s) acc[s] = row_sum(acc[s]);
#pragma unroll
            for (int s = 0; s < MUH; ++s) {
                const float r0 = lane_val(acc[s], 0), r1 = lane_val(acc[s], 16);
                const float r2 = lane_val(acc[s], 32), r3 = lane_val(acc[s], 48);
                acc[s] = P.seg == 64 ? (r0 + r1) + (r2 + r3)
                       : P.seg == 32 ? (lane < 32 ? r0 + r1 : r2 + r3)
                                     : acc[s];
            }
        } else {
            for (int o = P.seg >> 1; o > 0; o >>= 1)
#pragma unroll
                for (int s = 0; s < MUH; ++s) acc[s] += __shfl_xor(acc[s], o, 64);
        }
#pragma unroll
        for (int s = 0; s < MUH; ++s) {
            if (unit[h][s] < 0) continue;
            const int r = unit[h][s] * P.rpp + lrow;
            const bool hp = ep_on[h] && s < EPS;
            const int se = s < EPS ? s : 0;
            epi(r, acc[s], r < P.W.M && lg < P.ng && lg == 0,
                Pre3{ep[h][se][0], ep[h][se][1], ep[h][se][2]}, hp);
        }
    }

    template <class Epi>
    __device__ __forceinline__ void compute(const PhaseDesc& P, int h, int lane, Epi&& epi) {
        if constexpr (BLK == 0) {
            switch (P.nk4) {
                case 1: compute_f32<1>(P, h, lane, epi); break;
                case 2: compute_f32<2>(P, h, lane, epi); break;
                case 4: compute_f32<4>(P, h, lane, epi); break;
                default: compute_f32<8>(P, h, lane, epi); break;
            }
        } else {
            compute_i4(P, h, lane, epi);
        }
    }
};

struct GridBar {
    unsigned* sub;
    unsigned* top;
    unsigned* err;
    unsigned cnt, ngrp, epoch, stall, limit;
};

// All of this workgroup's global stores have completed; count it in.
__device__ __forceinline__ void bar_arrive(GridBar& g) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    ++g.epoch;
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(g.sub, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1 == g.cnt * g.epoch)
            __hip_atomic_fetch_add(g.top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Waits until every workgroup has arrived; false on time-out (or another
// workgroup's time-out), after which the caller leaves the kernel.
__device__ __forceinline__ bool bar_wait(GridBar& g, int* flag) {
    if (threadIdx.x == 0) {
        const unsigned want = g.ngrp * g.epoch + g.stall;
        int ok = 1;
        unsigned spins = 0;
        while ((int)(__hip_atomic_load(g.top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - want) < 0) {
            if ((++spins & 255) == 0) {
                if (__hip_atomic_load(g.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) { ok = 0; break; }
                if (spins > g.limit) {
                    __hip_atomic_store(g.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                    break;
                }
            }
            __builtin_amdgcn_s_sleep(1);
        }
        *flag = ok;
    }
    __syncthreads();
    return *flag != 0;
}

// Order of loads. vmcnt drains in issue order per wave, so a value can only
// be consumed once everything issued before it has arrived, and the compiler
// computes exact waits only across straight-line code that issues the same
// loads on every path. Each phase therefore issues, in this order and without
// branches: its own inputs (the previous phase's output, LayerNorm
// parameters), then the next phase's inputs produced earlier (state, history
// products), then the next phase's weights into the register half the current
// phase does not use. Phases alternate halves: A and C use half 0, B and D
// half 1; the LM head streams through both. A phase's weights are issued a
// full phase ahead and are in registers when it starts (arriving at a barrier
// drains every outstanding access: gfx9 counts stores and loads together).
// KHT: conv-history entries (taps - 1), a compile-time count so the history
// loads are straight-line too.
template <int BLK, int KHT>
__global__ __launch_bounds__(NT) void k_decode_persist(PersistArgs a) {
    __shared__ __align__(16) float xs[kMaxK];     // activation of the current products
    __shared__ __align__(16) float xs2[kMaxD];    // old state s (phase A, W_eff's rows)
    __shared__ float raw[kMaxD];                  // LN_in(x) of the layer: history input
    __shared__ float hdl[KHT * kMaxD];            // conv-history products of the layer
    __shared__ float q16[16];
    __shared__ float red[4];
    __shared__ unsigned long long kred[4];
    __shared__ int flag;

    int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    auto fresh = [&]() {
        tid = opq(tid);
        lane = tid & 63;
    };
    const int nwg = gridDim.x, wg = blockIdx.x;
    const int NW = nwg * 4, gw = wg * 4 + wv;
    const int D = a.D, I = a.I, R = a.R, K = KHT + 1, L = a.L;
    constexpr int kh = KHT;

    GridBar bar;
    {
        const int g = wg & 7;
        bar.sub = a.bar + g * 32;
        bar.top = a.bar + 256;
        bar.err = a.bar + kPersistBarErr;
        bar.cnt = (unsigned)((nwg - g + 7) / 8);
        bar.ngrp = (unsigned)min(nwg, 8);
        bar.epoch = 0;
        bar.stall = a.stall;
        bar.limit = a.spin_limit;
    }

    auto sidx = [&](int i, int Kd) -> int {
        if constexpr (BLK == 0) return i;
        else return ((((i % BLK) >> 2) * (Kd / BLK) + i / BLK) << 2) + (i & 3);
    };
    auto geom = [&](PhaseDesc& P, int Kd) {
        P.Kd = Kd;
        if constexpr (BLK == 0) {
            const int n = (Kd + 255) / 256;
            P.lg4 = n <= 1 ? 0 : n <= 2 ? 1 : n <= 4 ? 2 : 3;
            P.nk4 = 1 << P.lg4;
            P.ng = 0; P.seg = 64; P.rpp = 1;
            P.rpb = PH / P.nk4;
        } else {
            P.nk4 = 0; P.lg4 = 0;
            P.ng = Kd / BLK;
            P.seg = (P.ng < 64 && 64 % P.ng == 0) ? P.ng : 64;
            P.rpp = 64 / P.seg;
            P.rpb = muh<BLK>();
        }
    };
    auto finish = [&](PhaseDesc& P, int u0, int stride) {
        P.u0 = u0;
        P.ustride = stride;
        const int cnt = u0 < P.nu ? (P.nu - u0 + stride - 1) / stride : 0;
        P.nb = (cnt + P.rpb - 1) / P.rpb;
    };
    auto desc = [&](const PMat& W, int Kd, const float* x0, const float* x1, int split) {
        // x0 / x1 are this workgroup's LDS arrays
        PhaseDesc P;
        geom(P, Kd);
        P.W = W;
        P.nu = (W.M + P.rpp - 1) / P.rpp;
        P.split = split;
        P.x0 = (l_f32*)x0; P.x1 = (l_f32*)x1;
        finish(P, gw, NW);
        return P;
    };
    // V's rows multiply at, W_eff's rows (from row R on) the old state.
    auto layer = [&](int l) -> PLayer { return ((c_layer*)a.layers)[l]; };
    auto descA = [&](int l) { return desc(layer(l).VW, D, xs, xs2, R); };
    const int ngroups = D / 8;
    // Group c: the 16 contiguous rows 16c.. of U (8 values, 8 gates), split
    // over the workgroup's four waves. (A workgroup without a group loads
    // the last group's rows and leaves them unused.)
    auto descB = [&](int l, int c) {
        const PMat U = layer(l).U;
        PhaseDesc P;
        geom(P, R);
        const size_t r0 = (size_t)16 * min(c, ngroups - 1);
        if constexpr (BLK == 0) P.W = PMat{U.w + r0 * R, nullptr, nullptr, 16};
        else P.W = PMat{nullptr, U.q + r0 * (R / 2), U.sc + r0 * P.ng, 16};
        P.nu = (16 + P.rpp - 1) / P.rpp;
        P.split = 16;
        P.x0 = (l_f32*)xs; P.x1 = (l_f32*)xs;
        finish(P, wv, 4);
        return P;
    };
    auto descC = [&](int l) {
        const PMat W = layer(l).Wz;
        return desc(W, D, xs, xs, W.M);
    };
    auto descD = [&](int l) {
        const PMat W = layer(l).Wc;
        return desc(W, I, xs, xs, W.M);
    };
    auto descH = [&]() { return desc(a.head, D, xs, xs, a.head.M); };
    const EpiPre none{nullptr, nullptr, nullptr};

    Pool<BLK> pool;
    // All batches of a phase from one half (batch 0 loaded a phase earlier).
    auto run0 = [&](const PhaseDesc& P, const EpiPre& E, auto&& epi) {
        for (int b = 0; b < P.nb; ++b) {
            if (b > 0) pool.template load<false>(P, 0, b, lane, E);
            pool.compute(P, 0, lane, epi);
        }
    };
    auto run1 = [&](const PhaseDesc& P, const EpiPre& E, auto&& epi) {
        for (int b = 0; b < P.nb; ++b) {
            if (b > 0) pool.template load<false>(P, 1, b, lane, E);
            pool.compute(P, 1, lane, epi);
        }
    };
    // Double-buffered through both halves (batches 0 and 1 loaded before).
    auto run_stream = [&](const PhaseDesc& P, const EpiPre& E, auto&& epi) {
        for (int b = 0; b < P.nb; b += 2) {
            pool.compute(P, 0, lane, epi);
            pool.template load<false>(P, 0, b + 2, lane, E);
            if (b + 1 < P.nb) {
                pool.compute(P, 1, lane, epi);
                pool.template load<false>(P, 1, b + 3, lane, E);
            }
        }
    };

    // Phase A inputs produced earlier: s -> xs2, conv-history products -> hdl.
    float sv[PD], hv[PD][KHT > 0 ? KHT : 1];
    auto prestage_issue = [&](int l) {
        const float* s_l = a.s + (size_t)l * D;
        const float* hd_l = a.hd + (size_t)l * (kh ? kh : 1) * D;
#pragma unroll
        for (int k = 0; k < PD; ++k) {
            const int i = min(k * NT + tid, D - 1);
            sv[k] = ldc(s_l + i);
#pragma unroll
            for (int t = 0; t < KHT; ++t) hv[k][t] = ldc(hd_l + (size_t)t * D + i);
        }
    };
    auto prestage_store = [&]() {
#pragma unroll
        for (int k = 0; k < PD; ++k) {
            const int i = k * NT + tid;
            if (i >= D) continue;
            xs2[sidx(i, D)] = sv[k];
#pragma unroll
            for (int t = 0; t < KHT; ++t) hdl[t * D + i] = hv[k][t];
        }
    };
    // Phase B inputs for channel group c: old s and history of channel
    // 8 c + (tid & 7) (used by tid < 8).
    float pb_s = 0.0f, pb_h[KHT > 1 ? KHT - 1 : 1];
    auto preload_B = [&](int l, int c) {
        const int i = min(c, ngroups - 1) * 8 + (tid & 7);
        pb_s = ldc(a.s + (size_t)l * D + i);
        const float* h_l = a.hist + (size_t)l * (kh ? kh : 1) * D;
#pragma unroll
        for (int t = 0; t + 1 < KHT; ++t) pb_h[t] = ldc(h_l + (size_t)t * D + i);
    };

    // ---- phases (A of layer 0 differs: it also issues its own weights)
    auto phaseA = [&](int l, bool tok_ok, const float* erow) {
        const PLayer Ly = layer(l);
        float xv[PD], gv[PD], cv[PD], dv[PD];
        if (l == 0) issue_ldg(xv, erow, D, tid);
        else issue_ldc(xv, a.x, D, tid);
        issue_ldg(gv, Ly.ni_g, D, tid);
        issue_ldg(cv, Ly.ni_c, D, tid);
        issue_ldg(dv, Ly.dw + (size_t)(K - 1) * D, D, tid);
        issue_fence();
        if (l == 0) {
            prestage_issue(0);
            issue_fence();
            pool.template load<false>(descA(0), 0, 0, lane, none);
            issue_fence();
        }
        preload_B(l, wg);
        issue_fence();
        pool.template load<false>(descB(l, wg), 1, 0, lane, none);
        issue_fence();
        if (l == 0) prestage_store();
#pragma unroll
        for (int k = 0; k < PD; ++k)
            if (k * NT + tid >= D) xv[k] = 0.0f;
            else if (l == 0 && !tok_ok) xv[k] = __builtin_nanf("");
        float mean, rstd;
        ln_stats(xv, D, a.eps, tid, red, mean, rstd);
#pragma unroll
        for (int k = 0; k < PD; ++k) {
            const int i = k * NT + tid;
            if (i >= D) continue;
            const float r = (xv[k] - mean) * rstd * gv[k] + cv[k];
            raw[i] = r;
            float acc = r * dv[k];
#pragma unroll
            for (int t = 0; t < KHT; ++t) acc = acc + hdl[t * D + i];
            xs[sidx(i, D)] = KHT > 0 ? r + acc : r;
        }
        __syncthreads();
        run0(descA(l), none, [&](int r, float v, bool w, Pre3, bool) {
            if (w) stc(r < R ? a.v + r : a.sfb + (r - R), v);
        });
    };
    auto phaseB = [&](int l) {
        const PLayer Ly = layer(l);
        float* s_l = a.s + (size_t)l * D;
        float* h_l = a.hist + (size_t)l * (kh ? kh : 1) * D;
        float* hd_l = a.hd + (size_t)l * (kh ? kh : 1) * D;
        float vv[PI];
        issue_ldc(vv, a.v, R, tid);
        issue_fence();
        pool.template load<false>(descC(l), 0, 0, lane, none);
        issue_fence();
#pragma unroll
        for (int k = 0; k < PI; ++k)
            if (k * NT + tid < R) xs[sidx(k * NT + tid, R)] = vv[k];
        __syncthreads();
        for (int c = wg; c < ngroups; c += nwg) {
            const PhaseDesc P = descB(l, c);
            if (c != wg) {
                preload_B(l, c);
                pool.template load<false>(P, 1, 0, lane, none);
            }
            run1(P, none, [&](int r, float v, bool w, Pre3, bool) {
                if (w) q16[r] = v;
            });
            __syncthreads();
            if (tid < 8) {
                const int i = c * 8 + tid;
                const float gi = q16[8 + tid];
                const float uu = q16[tid] * (sgm(gi - q16[8 + ((tid + 1) & 7)]) *
                                             sgm(gi - q16[8 + ((tid + 2) & 7)]));
                float p = 1.0f - ldg(Ly.delta + i) * (1.0f - sgm(gi));
                if (a.clamp && p < a.p_floor) p = a.p_floor;
                stc(s_l + i, p * pb_s + (1.0f - p) * uu);
                stc(a.u + i, uu);
                if (KHT > 0) {
                    // hist' = [raw, hist[0], ..., hist[kh-2]]; hd' = hist' * dw
                    const float r = raw[i];
                    stc(h_l + i, r);
                    stc(hd_l + i, r * ldg(Ly.dw + (size_t)(K - 2) * D + i));
#pragma unroll
                    for (int t = 1; t < KHT; ++t) {
                        stc(h_l + (size_t)t * D + i, pb_h[t - 1]);
                        stc(hd_l + (size_t)t * D + i, pb_h[t - 1] * ldg(Ly.dw + (size_t)(K - 2 - t) * D + i));
                    }
                }
            }
            __syncthreads();
        }
    };
    auto phaseC = [&](int l, const EpiPre& preD) {
        const PLayer Ly = layer(l);
        float uv[PD];
        issue_ldc(uv, a.u, D, tid);
        issue_fence();
        pool.template load<true>(descD(l), 1, 0, lane, preD);
        issue_fence();
#pragma unroll
        for (int k = 0; k < PD; ++k)
            if (k * NT + tid < D) xs[sidx(k * NT + tid, D)] = uv[k];
        __syncthreads();
        const float at = Ly.a_tanh;
        run0(descC(l), none, [&](int r, float v, bool w, Pre3, bool) {
            if (w) stc(a.z + r, v * (1.0f + 0.5f * at / (1.0f + fabsf(v))));
        });
    };
    auto phaseD = [&](int l, bool bad_tok, const EpiPre& preD) {
        const PLayer Ly = layer(l);
        float zv[PI], gv[PI], cv[PI];
        issue_ldc(zv, a.z, I, tid);
        issue_ldg(gv, Ly.nm_g, I, tid);
        issue_ldg(cv, Ly.nm_c, I, tid);
        issue_fence();
        const bool more = l + 1 < L;
        prestage_issue(more ? l + 1 : l);
        issue_fence();
        pool.template load<false>(more ? descA(l + 1) : descH(), 0, 0, lane, none);
        issue_fence();
#pragma unroll
        for (int k = 0; k < PI; ++k)
            if (k * NT + tid >= I) zv[k] = 0.0f;
        float mean, rstd;
        ln_stats(zv, I, a.eps, tid, red, mean, rstd);
#pragma unroll
        for (int k = 0; k < PI; ++k) {
            const int i = k * NT + tid;
            if (i < I) xs[sidx(i, I)] = (zv[k] - mean) * rstd * gv[k] + cv[k];
        }
        __syncthreads();
        const float bg = Ly.b_gain;
        run1(descD(l), preD, [&](int r, float v, bool w, Pre3 pre, bool hp) {
            if (w) {
                if (!hp) pre = Pre3{ldc(preD.s + r), ldc(preD.sfb + r), ldc(preD.x + r)};
                const float xr = bad_tok ? __builtin_nanf("") : pre.x;
                stc(a.x + r, v + (bg * pre.s + pre.f + xr));
            }
        });
        if (more) prestage_store();
        else pool.template load<false>(descH(), 1, 1, lane, none);
    };
    auto barrier = [&]() -> bool {
        bar_arrive(bar);
        fresh();
        const bool ok = bar_wait(bar, &flag);
        fresh();
        return ok;
    };

    // Conv-history products of the stored history, for the first step: each
    // channel group's owner (the phase-B assignment) writes its channels.
    if (KHT > 0)
        for (int c = wg; c < ngroups; c += nwg)
            for (int idx = tid; idx < L * kh * 8; idx += NT) {
                const int l = idx / (kh * 8), t = (idx / 8) % kh, i = c * 8 + (idx & 7);
                const size_t off = ((size_t)l * kh + t) * D + i;
                stc(a.hd + off, ldc(a.hist + off) * ldg(layer(l).dw + (size_t)(K - 2 - t) * D + i));
            }
    if (!barrier()) return;

    int tok = a.tok_in[0];
    for (int step = 0; step < a.n_steps; ++step) {
        const bool last = step + 1 == a.n_steps;
        const bool tok_ok = tok >= 0 && tok < a.vocab;
        const float* erow = a.embed + (size_t)(tok_ok ? tok : 0) * D;
        // Layer 0 (peeled: its phase A issues its own weights), then the rest.
        for (int l = 0; l < L; ++l) {
            const EpiPre preD{a.s + (size_t)l * D, a.sfb, l == 0 ? erow : a.x};
            if (l == 0) phaseA(0, tok_ok, erow);
            else phaseA(l, true, erow);
            if (!barrier()) return;
            phaseB(l);
            if (!barrier()) return;
            phaseC(l, preD);
            if (!barrier()) return;
            phaseD(l, l == 0 && !tok_ok, preD);
            if (!barrier()) return;
        }

        // ---- H: logits = E LN_out(x) (sunnynet.c:280-333), argmax key per workgroup
        {
            float xv[PD], gv[PD], cv[PD];
            issue_ldc(xv, a.x, D, tid);
            issue_ldg(gv, a.no_g, D, tid);
            issue_ldg(cv, a.no_c, D, tid);
#pragma unroll
            for (int k = 0; k < PD; ++k)
                if (k * NT + tid >= D) xv[k] = 0.0f;
            float mean, rstd;
            ln_stats(xv, D, a.eps, tid, red, mean, rstd);
#pragma unroll
            for (int k = 0; k < PD; ++k) {
                const int i = k * NT + tid;
                if (i < D) xs[sidx(i, D)] = (xv[k] - mean) * rstd * gv[k] + cv[k];
            }
            __syncthreads();
            unsigned long long best = 0ull;
            float* lg = last ? a.logits : nullptr;
            const bool greedy = a.greedy != 0;
            run_stream(descH(), none, [&](int r, float v, bool w, Pre3, bool) {
                if (w) {
                    if (lg) lg[r] = v;
                    if (greedy) best = max(best, argmax_key(v, r));
                }
            });
            if (greedy) {
                best = kmax_wave(best);
                if (lane == 0) kred[wv] = best;
                __syncthreads();
                if (tid == 0)
                    __hip_atomic_store(a.part + wg, max(max(kred[0], kred[1]), max(kred[2], kred[3])),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (!a.greedy) break;
        if (!barrier()) return;
        // Every workgroup reduces the same keys to the same token.
        {
            unsigned long long k = 0ull;
#pragma unroll
            for (int j = 0; j < kPersistMaxGrid / NT; ++j)
                k = max(k, __hip_atomic_load(a.part + min(j * NT + tid, nwg - 1), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
            k = kmax_wave(k);
            if (lane == 0) kred[wv] = k;
            __syncthreads();
            k = max(max(kred[0], kred[1]), max(kred[2], kred[3]));
            tok = (int)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
            if (wg == 0 && tid == 0) a.out_tok[step] = tok;
            __syncthreads();
        }
    }
}

const void* kernel_for(int blk) {
    return blk == 0 ? (const void*)k_decode_persist<0, kPersistTaps - 1>
         : blk == 32 ? (const void*)k_decode_persist<32, kPersistTaps - 1>
                     : (const void*)k_decode_persist<64, kPersistTaps - 1>;
}

}  // namespace

int persist_occupancy(int blk) {
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel_for(blk), NT, 0);
    return e == hipSuccess ? nb : 0;
}

snhip_status launch_decode_persist(const PersistArgs& a, int nwg, int blk, hipStream_t st) {
    if (a.D > kMaxD || a.I > kMaxK || a.R > kMaxK || a.K != kPersistTaps || a.D % 8 || nwg < 1 ||
        nwg > kPersistMaxGrid || a.n_steps < 1 || (a.greedy && !a.out_tok) ||
        (!a.greedy && a.n_steps != 1)) {
        set_last_error("persistent decode: unsupported shape or arguments");
        return SNHIP_E_INVAL;
    }
    PersistArgs args = a;
    void* kargs[] = {&args};
    SNHIP_CHECK(hipLaunchCooperativeKernel(kernel_for(blk), dim3(nwg), dim3(NT), kargs, 0, st));
    return SNHIP_OK;
}

}  // namespace snhip
