// Persistent decode of one sequence: every layer of every step in one
// cooperative launch (the B = 1 path of snhip_step / snhip_decode_greedy_dev).
//
// The math is the decode step of sunnynet/runtime/sunnynet.c:212-334, in the
// same operation order as the per-kernel path (model.hip). A step is a chain
// of small matrix-vector products, each too short to fill the chip as its own
// launch; here the whole grid (one or two workgroups per CU) walks through the
// step in phases separated by grid barriers:
//
//   A  LN_in(x), depthwise conv -> at;  v = V at,  sfb = W_eff s      (all WGs)
//   B  q = U v for one group of 8 channels per WG (16 rows: 8 value, 8 gate),
//      competitive + decay gate, s' = p s + (1 - p) u, conv history shift
//   C  z = wedge(W_z u)
//   D  y = LN_I(z);  x = W_c y + b s' + sfb + x
//   H  logits = E LN_out(x), per-WG argmax key;  then every WG reduces the
//      keys to the same greedy token, the next step's input.
//
// 4 L + 1 barriers per step. Before waiting at a barrier each wave issues the
// weight loads of its first batch of rows of the next phase (they do not depend
// on the activations), so weight streaming overlaps the barrier.
//
// Values exchanged between workgroups (x, v, sfb, u, z, s, the conv history,
// the argmax keys) are written and read with agent-scope atomic accesses
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
constexpr int kMaxK = kPersistMaxDim;
constexpr int PER = kMaxK / NT;              // values per thread in the LayerNorms
constexpr int MR = 2;                        // fp32: rows per wave batch
constexpr int NK = kMaxK / 256;              // fp32: float4 per lane per row
constexpr int MU = 8;                        // INT4: units per wave batch

__device__ __forceinline__ float ldc(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float ssum(float v, int seg) {
    for (int o = seg >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
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
__device__ __forceinline__ void ln_stats(const float (&xv)[PER], int n, float eps, float* red,
                                         float& mean, float& rstd) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (k * NT + (int)threadIdx.x < n) sum += xv[k];
    mean = bsum(sum, red) / (float)n;
    float vs = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (k * NT + (int)threadIdx.x < n) {
            const float d = xv[k] - mean;
            vs += d * d;
        }
    rstd = 1.0f / sqrtf(bsum(vs, red) / (float)n + eps);
}

// One phase's matrix-vector work: up to two matrices with the same
// contraction length Kd, split in units (fp32: one row; INT4: rpp rows, one
// per segment of seg lanes, each lane one group of BLK inputs). This wave
// takes units u0, u0 + ustride, ...
struct PhaseDesc {
    PMat j0, j1;
    int nu0, nu1;
    int Kd, ng, seg, rpp;
    const float* x0;        // LDS activation of job 0 (staged layout)
    const float* x1;        // of job 1
    int u0, ustride, nb;    // first unit, stride, batches
};

template <int BLK>
struct Batch {
    static constexpr int MB = BLK ? MU : MR;
    static constexpr int QW = BLK ? BLK / 32 : 1;    // uint4 per INT4 group
    float4 wf[BLK ? 1 : MR][NK];
    uint4 wq[BLK ? MU : 1][QW];
    float wsc[BLK ? MU : 1];
    int job[MB], unit[MB];

    __device__ __forceinline__ void load(const PhaseDesc& P, int b, int lane) {
        const int lrow = lane / P.seg, lg = lane - lrow * P.seg;
#pragma unroll
        for (int s = 0; s < MB; ++s) {
            const int u = P.u0 + (b * MB + s) * P.ustride;
            int j = -1, ul = 0;
            if (u < P.nu0) { j = 0; ul = u; }
            else if (u < P.nu0 + P.nu1) { j = 1; ul = u - P.nu0; }
            job[s] = j;
            unit[s] = ul;
            if (j < 0) continue;
            if constexpr (BLK == 0) {
                const float* row = (j ? P.j1.w : P.j0.w) + (size_t)ul * P.Kd;
#pragma unroll
                for (int i = 0; i < NK; ++i) {
                    const int k = i * 256 + lane * 4;
                    if (k < P.Kd) wf[s][i] = *reinterpret_cast<const float4*>(row + k);
                }
            } else {
                const int r = ul * P.rpp + lrow;
                if (r < (j ? P.j1.M : P.j0.M) && lg < P.ng) {
                    const uint8_t* qr = (j ? P.j1.q : P.j0.q) + (size_t)r * (P.Kd / 2) + lg * (BLK / 2);
#pragma unroll
                    for (int h = 0; h < QW; ++h) wq[s][h] = *reinterpret_cast<const uint4*>(qr + 16 * h);
                    wsc[s] = (j ? P.j1.sc : P.j0.sc)[(size_t)r * P.ng + lg];
                }
            }
        }
    }

    // epi(job, row, value, writer): the row's dot product; `writer` is true
    // on exactly one lane per row.
    template <class Epi>
    __device__ __forceinline__ void compute(const PhaseDesc& P, int lane, Epi&& epi) {
        const int lrow = lane / P.seg, lg = lane - lrow * P.seg;
#pragma unroll
        for (int s = 0; s < MB; ++s) {
            if (job[s] < 0) continue;
            const float* xs = job[s] ? P.x1 : P.x0;
            if constexpr (BLK == 0) {
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < NK; ++i) {
                    const int k = i * 256 + lane * 4;
                    if (k < P.Kd) {
                        const float4 x4 = *reinterpret_cast<const float4*>(xs + k);
                        acc = fmaf(wf[s][i].x, x4.x, acc);
                        acc = fmaf(wf[s][i].y, x4.y, acc);
                        acc = fmaf(wf[s][i].z, x4.z, acc);
                        acc = fmaf(wf[s][i].w, x4.w, acc);
                    }
                }
                acc = wsum(acc);
                epi(job[s], unit[s], acc, lane == 0);
            } else {
                const int M = job[s] ? P.j1.M : P.j0.M;
                const int r = unit[s] * P.rpp + lrow;
                const bool live = r < M && lg < P.ng;
                float acc = 0.0f;
                if (live) {
                    const float sc = wsc[s];
#pragma unroll
                    for (int j = 0; j < BLK / 2; ++j) {
                        const uint4& qq = wq[s][j >> 4];
                        const int wi = (j >> 2) & 3;
                        const uint32_t word = wi == 0 ? qq.x : wi == 1 ? qq.y : wi == 2 ? qq.z : qq.w;
                        const uint32_t byte = (word >> ((j & 3) * 8)) & 0xFFu;
                        // quant.c:82-83, bit-identical dequantization
                        const float wl = (float)((int)(byte & 0x0Fu) - 8) * sc;
                        const float wh = (float)((int)(byte >> 4) - 8) * sc;
                        acc = fmaf(wl, xs[j * P.ng + lg], acc);
                        acc = fmaf(wh, xs[(j + BLK / 2) * P.ng + lg], acc);
                    }
                }
                acc = ssum(acc, P.seg);
                epi(job[s], r, acc, live && lg == 0);
            }
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

template <int BLK>
__global__ __launch_bounds__(NT) void k_decode_persist(PersistArgs a) {
    __shared__ __align__(16) float xs[kMaxK];
    __shared__ __align__(16) float xs2[kMaxK];
    __shared__ float raw[kMaxK];
    __shared__ float q16[16];
    __shared__ float red[4];
    __shared__ unsigned long long kred[4];
    __shared__ int flag;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int nwg = gridDim.x, wg = blockIdx.x;
    const int NW = nwg * 4, gw = wg * 4 + wv;
    const int D = a.D, I = a.I, R = a.R, K = a.K, kh = a.kh;
    constexpr int MB = Batch<BLK>::MB;

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
        else return (i % BLK) * (Kd / BLK) + i / BLK;
    };
    auto geom = [&](PhaseDesc& P, int Kd) {
        P.Kd = Kd;
        if constexpr (BLK == 0) {
            P.ng = 0; P.seg = 64; P.rpp = 1;
        } else {
            P.ng = Kd / BLK;
            P.seg = (P.ng < 64 && 64 % P.ng == 0) ? P.ng : 64;
            P.rpp = 64 / P.seg;
        }
    };
    auto finish = [&](PhaseDesc& P, int u0, int stride) {
        P.u0 = u0;
        P.ustride = stride;
        const int total = P.nu0 + P.nu1;
        const int cnt = u0 < total ? (total - u0 + stride - 1) / stride : 0;
        P.nb = (cnt + MB - 1) / MB;
    };
    auto one = [&](const PMat& W, int Kd, const float* x) {
        PhaseDesc P;
        geom(P, Kd);
        P.j0 = W; P.j1 = W;
        P.nu0 = (W.M + P.rpp - 1) / P.rpp; P.nu1 = 0;
        P.x0 = x; P.x1 = x;
        finish(P, gw, NW);
        return P;
    };
    auto descA = [&](int l) {
        const PLayer& Ly = a.layers[l];
        PhaseDesc P;
        geom(P, D);
        P.j0 = Ly.V; P.j1 = Ly.Ws;
        P.nu0 = (Ly.V.M + P.rpp - 1) / P.rpp;
        P.nu1 = (Ly.Ws.M + P.rpp - 1) / P.rpp;
        P.x0 = xs; P.x1 = xs2;
        finish(P, gw, NW);
        return P;
    };
    // Group c: rows 8c.. (values) and D + 8c.. (gates) of U, split over the
    // workgroup's four waves.
    auto descB = [&](int l, int c) {
        const PMat& U = a.layers[l].U;
        PhaseDesc P;
        geom(P, R);
        const size_t r0 = (size_t)8 * c, r1 = (size_t)D + 8 * c;
        if constexpr (BLK == 0) {
            P.j0 = PMat{U.w + r0 * R, nullptr, nullptr, 8};
            P.j1 = PMat{U.w + r1 * R, nullptr, nullptr, 8};
        } else {
            P.j0 = PMat{nullptr, U.q + r0 * (R / 2), U.sc + r0 * P.ng, 8};
            P.j1 = PMat{nullptr, U.q + r1 * (R / 2), U.sc + r1 * P.ng, 8};
        }
        P.nu0 = P.nu1 = (8 + P.rpp - 1) / P.rpp;
        P.x0 = xs; P.x1 = xs;
        finish(P, wv, 4);
        return P;
    };
    auto descC = [&](int l) { return one(a.layers[l].Wz, D, xs); };
    auto descD = [&](int l) { return one(a.layers[l].Wc, I, xs); };
    auto descH = [&]() { return one(a.head, D, xs); };

    Batch<BLK> bt;
    auto run = [&](const PhaseDesc& P, auto&& epi) {
        for (int b = 0; b < P.nb; ++b) {
            if (b > 0) bt.load(P, b, lane);   // batch 0 was loaded before the barrier
            bt.compute(P, lane, epi);
        }
    };

    const int ngroups = D / 8;
    int tok = a.tok_in[0];
    bt.load(descA(0), 0, lane);
    for (int step = 0; step < a.n_steps; ++step) {
        const bool last = step + 1 == a.n_steps;
        const bool tok_ok = tok >= 0 && tok < a.vocab;
        const float* erow = a.embed + (size_t)(tok_ok ? tok : 0) * D;
        for (int l = 0; l < a.L; ++l) {
            const PLayer& Ly = a.layers[l];
            float* s_l = a.s + (size_t)l * D;
            float* h_l = a.hist + (size_t)l * (kh ? kh : 1) * D;

            // ---- A: raw = LN_in(x), at = raw + conv(raw, hist) (sunnynet.c:221-237);
            //         v = V at, sfb = W_eff s (old state)
            {
                float xv[PER];
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int i = k * NT + tid;
                    float v = 0.0f;
                    if (i < D) v = l == 0 ? (tok_ok ? erow[i] : __builtin_nanf("")) : ldc(a.x + i);
                    xv[k] = v;
                }
                float mean, rstd;
                ln_stats(xv, D, a.eps, red, mean, rstd);
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int i = k * NT + tid;
                    if (i >= D) continue;
                    const float r = (xv[k] - mean) * rstd * Ly.ni_g[i] + Ly.ni_c[i];
                    raw[i] = r;
                    float at = r;
                    if (K > 1) {
                        float acc = r * Ly.dw[(size_t)(K - 1) * D + i];
#pragma unroll
                        for (int k2 = 0; k2 < kPersistMaxTaps - 1; ++k2)
                            if (k2 < kh) acc = acc + ldc(h_l + (size_t)k2 * D + i) * Ly.dw[(size_t)(K - 2 - k2) * D + i];
                        at = r + acc;
                    }
                    const int si = sidx(i, D);
                    xs[si] = at;
                    xs2[si] = ldc(s_l + i);
                }
                __syncthreads();
                run(descA(l), [&](int j, int r, float v, bool w) {
                    if (w) stc((j ? a.sfb : a.v) + r, v);
                });
            }
            bar_arrive(bar);
            if (wg < ngroups) bt.load(descB(l, wg), 0, lane);
            if (!bar_wait(bar, &flag)) return;

            // ---- B: q = U v for this workgroup's channel groups; gates, state
            //         update and conv history shift (sunnynet.c:238-266)
            if (wg < ngroups) {
                for (int i = tid; i < R; i += NT) xs[sidx(i, R)] = ldc(a.v + i);
                __syncthreads();
                for (int c = wg; c < ngroups; c += nwg) {
                    const PhaseDesc P = descB(l, c);
                    for (int b = 0; b < P.nb; ++b) {
                        if (b > 0 || c != wg) bt.load(P, b, lane);
                        bt.compute(P, lane, [&](int j, int r, float v, bool w) {
                            if (w) q16[j * 8 + r] = v;
                        });
                    }
                    __syncthreads();
                    if (tid < 8) {
                        const int i = c * 8 + tid;
                        const float gi = q16[8 + tid];
                        const float uu = q16[tid] * (sgm(gi - q16[8 + ((tid + 1) & 7)]) *
                                                     sgm(gi - q16[8 + ((tid + 2) & 7)]));
                        float p = 1.0f - Ly.delta[i] * (1.0f - sgm(gi));
                        if (a.clamp && p < a.p_floor) p = a.p_floor;
                        const float so = ldc(s_l + i);
                        stc(s_l + i, p * so + (1.0f - p) * uu);
                        stc(a.u + i, uu);
                        if (kh) {
                            float h[kPersistMaxTaps - 1];
#pragma unroll
                            for (int k2 = 0; k2 < kPersistMaxTaps - 1; ++k2)
                                h[k2] = k2 + 1 < kh ? ldc(h_l + (size_t)k2 * D + i) : 0.0f;
#pragma unroll
                            for (int k2 = kPersistMaxTaps - 2; k2 >= 1; --k2)
                                if (k2 < kh) stc(h_l + (size_t)k2 * D + i, h[k2 - 1]);
                            stc(h_l + i, raw[i]);
                        }
                    }
                    __syncthreads();
                }
            }
            bar_arrive(bar);
            bt.load(descC(l), 0, lane);
            if (!bar_wait(bar, &flag)) return;

            // ---- C: z = wedge(W_z u) (sunnynet.c:268-271)
            for (int i = tid; i < D; i += NT) xs[sidx(i, D)] = ldc(a.u + i);
            __syncthreads();
            run(descC(l), [&](int, int r, float v, bool w) {
                if (w) stc(a.z + r, v * (1.0f + 0.5f * Ly.a_tanh / (1.0f + fabsf(v))));
            });
            bar_arrive(bar);
            bt.load(descD(l), 0, lane);
            if (!bar_wait(bar, &flag)) return;

            // ---- D: y = LN_I(z); x = W_c y + b s' + sfb + x (sunnynet.c:272-277)
            {
                float zv[PER];
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int i = k * NT + tid;
                    zv[k] = i < I ? ldc(a.z + i) : 0.0f;
                }
                float mean, rstd;
                ln_stats(zv, I, a.eps, red, mean, rstd);
#pragma unroll
                for (int k = 0; k < PER; ++k) {
                    const int i = k * NT + tid;
                    if (i < I) xs[sidx(i, I)] = (zv[k] - mean) * rstd * Ly.nm_g[i] + Ly.nm_c[i];
                }
                __syncthreads();
                run(descD(l), [&](int, int r, float v, bool w) {
                    if (w) {
                        const float xr = l == 0 ? (tok_ok ? erow[r] : __builtin_nanf("")) : ldc(a.x + r);
                        stc(a.x + r, v + (Ly.b_gain * ldc(s_l + r) + ldc(a.sfb + r) + xr));
                    }
                });
            }
            bar_arrive(bar);
            if (l + 1 < a.L) bt.load(descA(l + 1), 0, lane);
            else bt.load(descH(), 0, lane);
            if (!bar_wait(bar, &flag)) return;
        }

        // ---- H: logits = E LN_out(x) (sunnynet.c:280-333), argmax key per workgroup
        {
            float xv[PER];
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int i = k * NT + tid;
                xv[k] = i < D ? ldc(a.x + i) : 0.0f;
            }
            float mean, rstd;
            ln_stats(xv, D, a.eps, red, mean, rstd);
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int i = k * NT + tid;
                if (i < D) xs[sidx(i, D)] = (xv[k] - mean) * rstd * a.no_g[i] + a.no_c[i];
            }
            __syncthreads();
            unsigned long long best = 0ull;
            float* lg = last ? a.logits : nullptr;
            const bool greedy = a.greedy != 0;
            run(descH(), [&](int, int r, float v, bool w) {
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
        bar_arrive(bar);
        if (!last) bt.load(descA(0), 0, lane);
        if (!bar_wait(bar, &flag)) return;
        // Every workgroup reduces the same keys to the same token.
        {
            unsigned long long k = 0ull;
            for (int i = tid; i < nwg; i += NT)
                k = max(k, __hip_atomic_load(a.part + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            k = kmax_wave(k);
            if (lane == 0) kred[wv] = k;
            __syncthreads();
            k = max(max(kred[0], kred[1]), max(kred[2], kred[3]));
            tok = (int)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
            if (wg == 0 && tid == 0) a.out_tok[step] = tok;
        }
    }
}

}  // namespace

int persist_occupancy(int blk) {
    int nb = 0;
    hipError_t e;
    if (blk == 0) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_decode_persist<0>, NT, 0);
    else if (blk == 32) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_decode_persist<32>, NT, 0);
    else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_decode_persist<64>, NT, 0);
    return e == hipSuccess ? nb : 0;
}

snhip_status launch_decode_persist(const PersistArgs& a, int nwg, int blk, hipStream_t st) {
    if (a.D > kMaxK || a.I > kMaxK || a.R > kMaxK || a.K > kPersistMaxTaps || a.D % 8 || nwg < 1 ||
        a.n_steps < 1 || (a.greedy && !a.out_tok) || (!a.greedy && a.n_steps != 1)) {
        set_last_error("persistent decode: unsupported shape or arguments");
        return SNHIP_E_INVAL;
    }
    PersistArgs args = a;
    void* kargs[] = {&args};
    const void* fn = blk == 0 ? (const void*)k_decode_persist<0>
                   : blk == 32 ? (const void*)k_decode_persist<32>
                               : (const void*)k_decode_persist<64>;
    SNHIP_CHECK(hipLaunchCooperativeKernel(fn, dim3(nwg), dim3(NT), kargs, 0, st));
    return SNHIP_OK;
}

}  // namespace snhip
