// Fused compete gate + decay gate + gated scan of a SunnyNet block, forward
// and backward (sunnynet/kernels/core_avx2.c:34-149), on gfx950.
//
// Inputs q (B,T,2D) = [u_raw | gate] per step, delta (D), s0 (B,D). Channels
// form groups of 8; inside a group, with e = expf(0 - gate),
//   sigma = 1 / (1 + e_i)
//   s1 = 1 / (1 + e_i / e_{i+1}),  s2 = 1 / (1 + e_i / e_{i+2})   (mod 8)
//   u = u_raw (s1 s2),  p = fma(delta, sigma, 1 - delta)
//   s_t = fma(p, s_{t-1}, (1 - p) u)
// with outputs states, u, p (B,T,D). The backward walks time in reverse with
// the reference's operation order (ds, dp, du, then the gate derivatives,
// whose group neighbours i-1 and i-2 are read back the same way). Every
// operation is the reference's IEEE fp32 operation in its order, except expf,
// which is the device's (within 1 ulp of glibc's): results agree to a few ulp.
//
// Design. Each step reads 8 B of q per channel and the forward writes 12 B
// (states, u, p); the backward reads 28 B (q, u, p, the previous state,
// dstate, du_in) and writes 8 B (dq). Both are HBM-bound streams around a
// cheap sequential chain (one FMA per step forward, four operations
// backward) and a heavy independent part (one exp, three divisions and the
// gate algebra per channel and step). A workgroup owns 128 channels of one
// batch row (two per lane, so a group of 8 channels is one lane quad and the
// neighbour reads are DPP quad permutes) and W waves. Time is cut into tiles
// of W TC steps; wave w owns steps [w TC, (w+1) TC) of each tile. The carried
// state is handed from wave to wave through LDS with a sequence flag (no
// workgroup barrier), so the heavy part of every wave runs concurrently on
// its own SIMD while the chain moves around the ring. Each wave holds two
// tiles of inputs in registers: the loads for tile i+1 are issued before
// tile i is processed, a whole tile period ahead of their use. The fast path
// needs D % 128 == 0 and T % (W TC) == 0 (the reference's block pads T to its
// scan chunk before it calls the kernel); any other shape takes a one lane per
// channel kernel.
#include <mutex>
#include <string>

#include "bufio.h"

namespace snhip {

namespace {

// Lane q of each quad reads lane (q + 1) & 3 / (q - 1) & 3 (DPP quad_perm).
__device__ __forceinline__ float quad_next(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x39, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_prev(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x93, 0xf, 0xf, false));
}

// IEEE division (the reference's _mm256_div_ps); the library is built without
// fast-math, so '/' is the correctly rounded quotient.
__device__ __forceinline__ float div_rn(float a, float b) { return __fdiv_rn(a, b); }

// Gate quantities of one step for the lane's two channels c0 = 2q, c1 = 2q+1
// of its group (q = lane & 3): with e the group's exp(-gate), channel c0's
// neighbours i+1, i+2 are e[c1] and the next lane's e[c0]; channel c1's are
// the next lane's e[c0] and e[c1].
struct Gate {
    float sig[2], s1[2], s2[2];
};
__device__ __forceinline__ Gate gate_of(const float (&g)[2]) {
    Gate r;
    const float e0 = expf(sub_rn(0.0f, g[0]));
    const float e1 = expf(sub_rn(0.0f, g[1]));
    const float n0 = quad_next(e0), n1 = quad_next(e1);
    const float e[2] = {e0, e1}, f1[2] = {e1, n0}, f2[2] = {n0, n1};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        r.sig[c] = div_rn(1.0f, add_rn(1.0f, e[c]));
        r.s1[c] = div_rn(1.0f, add_rn(1.0f, div_rn(e[c], f1[c])));
        r.s2[c] = div_rn(1.0f, add_rn(1.0f, div_rn(e[c], f2[c])));
    }
    return r;
}

// Workgroup-local hand-off of the carried values between the waves of the
// ring: `seq` counts completed slots. The writer's LDS stores complete
// (lgkmcnt(0)) before the flag store is issued; the reader reads the carry only
// after it has seen the flag. Global loads and stores stay in flight.
// The flag is addressed as LDS explicitly: a volatile access through a generic
// pointer would be a flat access, whose wait also drains every global load.
// The waves of a workgroup are resident together and each posts every slot in
// order, so the wait always ends; the poll count is bounded all the same
// (about a second), after which the wave goes on with whatever the carry holds.
typedef __attribute__((address_space(3))) volatile int lds_flag;
__device__ __forceinline__ lds_flag* as_lds(int* p) { return (lds_flag*)p; }
constexpr int kRingPolls = 1 << 25;
__device__ __forceinline__ void ring_wait(int* seq, int want) {
    for (int n = 0; __builtin_amdgcn_readfirstlane(*as_lds(seq)) != want && n < kRingPolls; ++n)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
__device__ __forceinline__ void ring_pass(int* seq, int next) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    wait_lds();
    *as_lds(seq) = next;
}

// Keeps the prefetch of the next tile where it is written: without this the
// scheduler sinks the loads below the current tile's arithmetic, which then
// waits for the current tile's data before the next tile's loads are issued.
__device__ __forceinline__ void issued() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

template <int TC>
struct FwdBuf {
    float ur[TC][2], g[TC][2];        // loaded; prep turns them into bp, p
};

template <int W, int TC>
__global__ __launch_bounds__(64 * W)
void k_core_fwd_buf(const float* __restrict__ q, const float* __restrict__ delta,
                    const float* __restrict__ s0, float* __restrict__ states,
                    float* __restrict__ uo, float* __restrict__ po, int T, int D) {
    using IO = BufIO<2>;
    __shared__ float carry[128];
    __shared__ int seq;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wg_per_row = D / 128;
    const int bb = blockIdx.x / wg_per_row;
    const int n0 = (blockIdx.x - bb * wg_per_row) * 128;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(q + (size_t)bb * T * 2 * D, (uint32_t)((size_t)T * 2 * D * 4));
    const uint32_t ob = (uint32_t)((size_t)T * D * 4);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(states + (size_t)bb * T * D, ob);
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(uo + (size_t)bb * T * D, ob);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(po + (size_t)bb * T * D, ob);
    const int vo = (n0 + 2 * lane) * 4, vg = vo + D * 4;
    const int rowq = 2 * D * 4, rowo = D * 4;
    float dl[2], base[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        dl[c] = delta[n0 + 2 * lane + c];
        base[c] = sub_rn(1.0f, dl[c]);
    }
    constexpr int TILE = W * TC;
    const int ntiles = T / TILE;

    FwdBuf<TC> A, Bf;
    // Tiles past the end (the prefetch of the last iteration) re-read the
    // last tile: scalar offsets are not range-checked.
    auto load = [&](FwdBuf<TC>& X, int tile) {
        const int t0 = min(tile, ntiles - 1) * TILE + w * TC;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            IO::load(X.ur[k], rq, vo, (t0 + k) * rowq);
            IO::load(X.g[k], rq, vg, (t0 + k) * rowq);
        }
    };
    // One tile: the gate algebra of every step (u and p stored at once;
    // ur <- (1 - p) u, g <- p), then the chain once the carry arrives.
    auto run = [&](FwdBuf<TC>& X, int tile) {
        const int t0 = tile * TILE + w * TC;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const Gate G = gate_of(X.g[k]);
            float u[2], p[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                u[c] = mul_rn(X.ur[k][c], mul_rn(G.s1[c], G.s2[c]));
                p[c] = fmaf(dl[c], G.sig[c], base[c]);
                X.ur[k][c] = mul_rn(sub_rn(1.0f, p[c]), u[c]);
                X.g[k][c] = p[c];
            }
            IO::store(ru, vo, (t0 + k) * rowo, u);
            IO::store(rp, vo, (t0 + k) * rowo, p);
        }
        ring_wait(&seq, tile * W + w);
        float s[2] = {carry[2 * lane], carry[2 * lane + 1]};
#pragma unroll
        for (int k = 0; k < TC; ++k) {
#pragma unroll
            for (int c = 0; c < 2; ++c) s[c] = fmaf(X.g[k][c], s[c], X.ur[k][c]);
            IO::store(rs, vo, (t0 + k) * rowo, s);
        }
        carry[2 * lane] = s[0];
        carry[2 * lane + 1] = s[1];
        ring_pass(&seq, tile * W + w + 1);
    };

    if (w == 0) {
        carry[2 * lane] = s0[(size_t)bb * D + n0 + 2 * lane];
        carry[2 * lane + 1] = s0[(size_t)bb * D + n0 + 2 * lane + 1];
        if (lane == 0) seq = 0;
    }
    __syncthreads();
    load(A, 0);
    int tile = 0;
    for (; tile + 2 <= ntiles; tile += 2) {
        load(Bf, tile + 1);
        issued();
        run(A, tile);
        load(A, tile + 2);
        issued();
        run(Bf, tile + 1);
    }
    if (tile < ntiles) run(A, tile);
}

template <int TC>
struct BwdBuf {
    // loaded: dstate, u, p, s_{t-1}, du_in, u_raw, gate. Before the chain
    // x <- s_{t-1} - u, y <- 1 - p; the chain leaves dp in x and du in di.
    float dst[TC][2], x[TC][2], p[TC][2], y[TC][2], di[TC][2], ur[TC][2], g[TC][2];
};

template <int W, int TC>
__global__ __launch_bounds__(64 * W)
void k_core_bwd_buf(const float* __restrict__ q, const float* __restrict__ delta,
                    const float* __restrict__ s0, const float* __restrict__ states,
                    const float* __restrict__ uo, const float* __restrict__ po,
                    const float* __restrict__ dstate, const float* __restrict__ du_in,
                    float* __restrict__ dq, float* __restrict__ dacc_out,
                    float* __restrict__ ds0, int T, int D) {
    using IO = BufIO<2>;
    __shared__ float carry[128];
    __shared__ float part[W][128];
    __shared__ int seq;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wg_per_row = D / 128;
    const int bb = blockIdx.x / wg_per_row;
    const int n0 = (blockIdx.x - bb * wg_per_row) * 128;
    const uint32_t qb = (uint32_t)((size_t)T * 2 * D * 4), ob = (uint32_t)((size_t)T * D * 4);
    const size_t qrow = (size_t)bb * T * 2 * D, orow = (size_t)bb * T * D;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(q + qrow, qb);
    const __amdgpu_buffer_rsrc_t rdq = make_rsrc(dq + qrow, qb);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(states + orow, ob);
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(uo + orow, ob);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(po + orow, ob);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(dstate + orow, ob);
    const __amdgpu_buffer_rsrc_t ri = make_rsrc(du_in + orow, ob);
    const int vo = (n0 + 2 * lane) * 4, vg = vo + D * 4;
    const int rowq = 2 * D * 4, rowo = D * 4;
    float dl[2], sz[2], dacc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        dl[c] = delta[n0 + 2 * lane + c];
        sz[c] = s0[(size_t)bb * D + n0 + 2 * lane + c];
    }
    constexpr int TILE = W * TC;
    const int ntiles = T / TILE;
    // Reversed step k of this wave's slot in `tile` is time t_of(tile, k).
    auto t_of = [&](int tile, int k) { return T - 1 - (tile * TILE + w * TC + k); };

    BwdBuf<TC> A, Bf;
    auto load = [&](BwdBuf<TC>& X, int tile) {
        const int tc = min(tile, ntiles - 1);
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int t = t_of(tc, k);
            const int so = t * rowo, sq = t * rowq, sp = max(t - 1, 0) * rowo;
            IO::load(X.dst[k], rd, vo, so);
            IO::load(X.y[k], ru, vo, so);
            IO::load(X.p[k], rp, vo, so);
            IO::load(X.x[k], rs, vo, sp);
            IO::load(X.di[k], ri, vo, so);
            IO::load(X.ur[k], rq, vo, sq);
            IO::load(X.g[k], rq, vg, sq);
        }
    };
    auto run = [&](BwdBuf<TC>& X, int tile) {
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const bool first = t_of(tile, k) == 0;           // s_{-1} is s0
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                X.x[k][c] = sub_rn(first ? sz[c] : X.x[k][c], X.y[k][c]);
                X.y[k][c] = sub_rn(1.0f, X.p[k][c]);
            }
        }
        ring_wait(&seq, tile * W + w);
        float ds[2] = {carry[2 * lane], carry[2 * lane + 1]};
#pragma unroll
        for (int k = 0; k < TC; ++k)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                ds[c] = add_rn(ds[c], X.dst[k][c]);
                X.x[k][c] = mul_rn(ds[c], X.x[k][c]);                 // dp
                X.di[k][c] = fmaf(ds[c], X.y[k][c], X.di[k][c]);      // du
                ds[c] = mul_rn(ds[c], X.p[k][c]);
            }
        carry[2 * lane] = ds[0];
        carry[2 * lane + 1] = ds[1];
        ring_pass(&seq, tile * W + w + 1);
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int t = t_of(tile, k);
            const Gate G = gate_of(X.g[k]);
            float dur[2], a1[2], a2[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const float du = X.di[k][c];
                dur[c] = mul_rn(du, mul_rn(G.s1[c], G.s2[c]));
                const float dw = mul_rn(du, X.ur[k][c]);
                a1[c] = mul_rn(mul_rn(dw, G.s2[c]), mul_rn(G.s1[c], sub_rn(1.0f, G.s1[c])));
                a2[c] = mul_rn(mul_rn(dw, G.s1[c]), mul_rn(G.s2[c], sub_rn(1.0f, G.s2[c])));
            }
            // a1[i-1], a2[i-2]: channel c0 = 2q reads the previous lane's
            // a1[c1] and a2[c0]; channel c1 reads its own a1[c0] and the
            // previous lane's a2[c1].
            const float pa1 = quad_prev(a1[1]), pa20 = quad_prev(a2[0]), pa21 = quad_prev(a2[1]);
            const float m1[2] = {pa1, a1[0]}, m2[2] = {pa20, pa21};
            float dg[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const float dp = X.x[k][c];
                float v = add_rn(a1[c], a2[c]);
                v = sub_rn(v, m1[c]);
                v = sub_rn(v, m2[c]);
                dg[c] = fmaf(mul_rn(dp, dl[c]), mul_rn(G.sig[c], sub_rn(1.0f, G.sig[c])), v);
                dacc[c] = fmaf(dp, sub_rn(G.sig[c], 1.0f), dacc[c]);
            }
            IO::store(rdq, vo, t * rowq, dur);
            IO::store(rdq, vg, t * rowq, dg);
        }
    };

    if (w == 0) {
        carry[2 * lane] = 0.0f;
        carry[2 * lane + 1] = 0.0f;
        if (lane == 0) seq = 0;
    }
    __syncthreads();
    load(A, 0);
    int tile = 0;
    for (; tile + 2 <= ntiles; tile += 2) {
        load(Bf, tile + 1);
        issued();
        run(A, tile);
        load(A, tile + 2);
        issued();
        run(Bf, tile + 1);
    }
    if (tile < ntiles) run(A, tile);

    part[w][2 * lane] = dacc[0];
    part[w][2 * lane + 1] = dacc[1];
    __syncthreads();
    if (w == 0) {
        float r[2] = {0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < W; ++j)
#pragma unroll
            for (int c = 0; c < 2; ++c) r[c] = add_rn(r[c], part[j][2 * lane + c]);
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            dacc_out[(size_t)bb * D + n0 + 2 * lane + c] = r[c];
            ds0[(size_t)bb * D + n0 + 2 * lane + c] = carry[2 * lane + c];
        }
    }
}

// Any shape with D % 8 == 0: one lane per channel, straight through time. A
// group's 8 channels are 8 adjacent lanes of one wave (B D is a multiple of
// 8 and waves start at multiples of 64), so whole groups are in or out of
// range together and the neighbour reads are lane shuffles.
__device__ __forceinline__ int grp_lane(int lane, int off) { return (lane & ~7) | ((lane + off) & 7); }

__global__ void k_core_fwd_gen(const float* __restrict__ q, const float* __restrict__ delta,
                               const float* __restrict__ s0, float* __restrict__ states,
                               float* __restrict__ uo, float* __restrict__ po, int B, int T, int D) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)B * D) return;
    const int lane = threadIdx.x & 63;
    const long bb = i / D;
    const int d = (int)(i - bb * D);
    const float dl = delta[d], base = sub_rn(1.0f, dl);
    float s = s0[i];
    for (int t = 0; t < T; ++t) {
        const size_t qo = ((size_t)bb * T + t) * 2 * D + d, so = ((size_t)bb * T + t) * D + d;
        const float e = expf(sub_rn(0.0f, q[qo + D]));
        const float e1 = __shfl(e, grp_lane(lane, 1)), e2 = __shfl(e, grp_lane(lane, 2));
        const float sig = div_rn(1.0f, add_rn(1.0f, e));
        const float s1 = div_rn(1.0f, add_rn(1.0f, div_rn(e, e1)));
        const float s2 = div_rn(1.0f, add_rn(1.0f, div_rn(e, e2)));
        const float u = mul_rn(q[qo], mul_rn(s1, s2));
        const float p = fmaf(dl, sig, base);
        s = fmaf(p, s, mul_rn(sub_rn(1.0f, p), u));
        states[so] = s;
        uo[so] = u;
        po[so] = p;
    }
}

__global__ void k_core_bwd_gen(const float* __restrict__ q, const float* __restrict__ delta,
                               const float* __restrict__ s0, const float* __restrict__ states,
                               const float* __restrict__ uo, const float* __restrict__ po,
                               const float* __restrict__ dstate, const float* __restrict__ du_in,
                               float* __restrict__ dq, float* __restrict__ dacc_out,
                               float* __restrict__ ds0, int B, int T, int D) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)B * D) return;
    const int lane = threadIdx.x & 63;
    const long bb = i / D;
    const int d = (int)(i - bb * D);
    const float dl = delta[d];
    float ds = 0.0f, dacc = 0.0f;
    for (int t = T - 1; t >= 0; --t) {
        const size_t qo = ((size_t)bb * T + t) * 2 * D + d, so = ((size_t)bb * T + t) * D + d;
        ds = add_rn(ds, dstate[so]);
        const float p = po[so];
        const float sprev = t > 0 ? states[so - D] : s0[i];
        const float dp = mul_rn(ds, sub_rn(sprev, uo[so]));
        const float du = fmaf(ds, sub_rn(1.0f, p), du_in[so]);
        ds = mul_rn(ds, p);
        const float e = expf(sub_rn(0.0f, q[qo + D]));
        const float e1 = __shfl(e, grp_lane(lane, 1)), e2 = __shfl(e, grp_lane(lane, 2));
        const float sig = div_rn(1.0f, add_rn(1.0f, e));
        const float s1 = div_rn(1.0f, add_rn(1.0f, div_rn(e, e1)));
        const float s2 = div_rn(1.0f, add_rn(1.0f, div_rn(e, e2)));
        dq[qo] = mul_rn(du, mul_rn(s1, s2));
        const float dw = mul_rn(du, q[qo]);
        const float a1 = mul_rn(mul_rn(dw, s2), mul_rn(s1, sub_rn(1.0f, s1)));
        const float a2 = mul_rn(mul_rn(dw, s1), mul_rn(s2, sub_rn(1.0f, s2)));
        const float m1 = __shfl(a1, grp_lane(lane, 7)), m2 = __shfl(a2, grp_lane(lane, 6));
        float v = sub_rn(sub_rn(add_rn(a1, a2), m1), m2);
        dq[qo + D] = fmaf(mul_rn(dp, dl), mul_rn(sig, sub_rn(1.0f, sig)), v);
        dacc = fmaf(dp, sub_rn(sig, 1.0f), dacc);
    }
    ds0[i] = ds;
    dacc_out[i] = dacc;
}

// ddelta[d] += sum over rows b of dacc[b, d], rows in order.
__global__ void k_core_ddelta(const float* __restrict__ dacc, float* __restrict__ ddelta, int B, int D) {
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    float r = 0.0f;
    for (int b = 0; b < B; ++b) r = add_rn(r, dacc[(size_t)b * D + d]);
    ddelta[d] = add_rn(ddelta[d], r);
}

// Ring shapes (waves per workgroup, steps per slot), from a sweep on the
// B=16, T=4096, D=2048 workload (median of 3 interleaved rounds, us per
// launch, forward / backward): W=4 TC=16 / W=4 TC=8: 479 / 842; W=4 TC=8 /
// W=4 TC=4: 454 / 847; W=8 TC=4 / W=8 TC=2: 456 / 831; W=16 TC=4 / W=16
// TC=2: 463 / 835; W=16 TC=2 / W=16 TC=1: 525 / 1733. Eight waves (two per
// SIMD) with short slots keep the most loads in flight per CU; a
// reciprocal-based variant of the divisions measured no faster.
constexpr int kFW = 8, kFTC = 4;        // forward ring
constexpr int kBW = 8, kBTC = 2;        // backward ring

bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

bool fast_ok(int B, int T, int D, int tile, std::initializer_list<const void*> ptrs) {
    if (D % 128 != 0 || T % tile != 0 || (size_t)T * 2 * D * 4 >= (1ull << 31)) return false;
    (void)B;
    for (const void* p : ptrs)
        if (!al8(p)) return false;
    return true;
}

}  // namespace

snhip_status launch_core_fwd(const float* q, const float* delta, const float* s0, float* states,
                             float* uo, float* po, int B, int T, int D, hipStream_t st) {
    if (fast_ok(B, T, D, kFW * kFTC, {q, states, uo, po})) {
        const unsigned grid = (unsigned)((long)B * D / 128);
        hipLaunchKernelGGL((k_core_fwd_buf<kFW, kFTC>), dim3(grid), dim3(64 * kFW), 0, st, q, delta, s0,
                           states, uo, po, T, D);
    } else {
        const long total = (long)B * D;
        hipLaunchKernelGGL(k_core_fwd_gen, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, q, delta,
                           s0, states, uo, po, B, T, D);
    }
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

namespace {
// Backward kernels plus the in-order row reduction of ddelta, with the (B, D)
// per-row partials in `acc` (every element is written before it is read).
snhip_status core_bwd_ws(const float* q, const float* delta, const float* s0, const float* states,
                         const float* uo, const float* po, const float* dstate, const float* du_in,
                         float* dq, float* ddelta, float* ds0, int B, int T, int D, float* acc,
                         hipStream_t st) {
    if (fast_ok(B, T, D, kBW * kBTC, {q, states, uo, po, dstate, du_in, dq})) {
        const unsigned grid = (unsigned)((long)B * D / 128);
        hipLaunchKernelGGL((k_core_bwd_buf<kBW, kBTC>), dim3(grid), dim3(64 * kBW), 0, st, q, delta, s0,
                           states, uo, po, dstate, du_in, dq, acc, ds0, T, D);
    } else {
        const long total = (long)B * D;
        hipLaunchKernelGGL(k_core_bwd_gen, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, q, delta,
                           s0, states, uo, po, dstate, du_in, dq, acc, ds0, B, T, D);
    }
    SNHIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(k_core_ddelta, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, st, acc, ddelta, B, D);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// Scratch of the allocation-free backward: the (B, D) ddelta partials of
// calls with B * D <= kCoreBwdScratchFloats (4 MiB per GPU, held for the life
// of the process). Host code uses the per-device address from
// hipGetSymbolAddress, never the array's name.
constexpr size_t kCoreBwdScratchFloats = (size_t)1 << 20;
static __device__ __align__(256) float scratch[kCoreBwdScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

// This device's address of `scratch`, resolved once per device with it current.
snhip_status scratch_ptr(float** out) {
    int dev = 0;
    SNHIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) {
        set_last_error("device index beyond the scratch table");
        return SNHIP_E_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        SNHIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_scratch[dev];
    return SNHIP_OK;
}
}  // namespace

snhip_status launch_core_bwd(const float* q, const float* delta, const float* s0, const float* states,
                             const float* uo, const float* po, const float* dstate, const float* du_in,
                             float* dq, float* ddelta, float* ds0, int B, int T, int D, hipStream_t st) {
    // Per-row sums of ddelta's terms, reduced over rows in order afterwards.
    float* acc = nullptr;
    SNHIP_CHECK(hipMallocAsync(reinterpret_cast<void**>(&acc), (size_t)B * D * sizeof(float), st));
    const snhip_status rc = core_bwd_ws(q, delta, s0, states, uo, po, dstate, du_in, dq, ddelta, ds0,
                                        B, T, D, acc, st);
    const hipError_t f = hipFreeAsync(acc, st);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(f);
    return SNHIP_OK;
}

snhip_status launch_core_bwd_noalloc(const float* q, const float* delta, const float* s0,
                                     const float* states, const float* uo, const float* po,
                                     const float* dstate, const float* du_in, float* dq, float* ddelta,
                                     float* ds0, int B, int T, int D, hipStream_t st) {
    if ((size_t)B * (size_t)D > kCoreBwdScratchFloats) {
        set_last_error("core backward without allocation: B * D = " + std::to_string((long long)B * D) +
                       " exceeds the scratch of " + std::to_string(kCoreBwdScratchFloats) + " floats");
        return SNHIP_E_INVAL;
    }
    float* acc = nullptr;
    const snhip_status rc = scratch_ptr(&acc);
    if (rc != SNHIP_OK) return rc;
    return core_bwd_ws(q, delta, s0, states, uo, po, dstate, du_in, dq, ddelta, ds0, B, T, D, acc, st);
}

}  // namespace snhip
