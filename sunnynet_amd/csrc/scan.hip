// First-order gated recurrence on gfx950: s_t = a_t * s_{t-1} + b'_t with
// b'_t = (1 - a_t) * u_t (gated) or b_t (FMA form), per channel, over (B,T,N)
// channel-major fp32 arrays.
//
// Semantics and rounding follow sunnynet/runtime/recur.c:13-48 (and the
// identical scan_f32, sunnynet/kernels/scan_avx2.c:12-45): b' is a separate
// multiply, the update is one fused multiply-add, and channels in the scalar
// tail [N & ~7, N) of the reference use a*s + b' with two roundings. The
// result is therefore bit-identical to the reference for every input.
//
// Design. A channel's recurrence is sequential in T, and cfg-sized inputs
// have only a few tens of thousands of channels, so one lane per channel would
// leave HBM idle (too few bytes in flight per CU). Each workgroup instead
// takes 64*CPL adjacent channels (one lane per CPL channels, vector loads
// along the contiguous N axis) and W waves. Time is cut into tiles of W*TC
// steps; wave w owns steps [w*TC, (w+1)*TC) of every tile and keeps them in
// VGPRs. The exact state is handed from wave to wave through LDS in W
// barrier-separated slots per tile; in its slot a wave runs its TC dependent
// FMAs from registers, passes the state on, and immediately issues the loads
// for its slot of the next tile, so every wave has a whole tile's worth of
// loads in flight while the others compute. HBM traffic is exactly one read
// of a and b and one write of out. The barrier orders LDS only, so the
// prefetches are never drained by it.
#include "bufio.h"

namespace snhip {

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
template <int CPL> struct VecT;
template <> struct VecT<1> { using T = float; };
template <> struct VecT<2> { using T = f32x2v; };
template <> struct VecT<4> { using T = f32x4v; };

// Streaming (non-temporal) vector load / store of CPL consecutive floats.
template <int CPL>
__device__ __forceinline__ void ld(float (&v)[CPL], const float* p) {
    using V = typename VecT<CPL>::T;
    const V x = __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
    if constexpr (CPL == 1) { v[0] = x; }
    else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) v[c] = x[c];
    }
}

template <int CPL>
__device__ __forceinline__ void st(float* p, const float (&v)[CPL]) {
    using V = typename VecT<CPL>::T;
    V x;
    if constexpr (CPL == 1) { x = v[0]; }
    else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) x[c] = v[c];
    }
    __builtin_nontemporal_store(x, reinterpret_cast<V*>(p));
}

template <int CPL, int W, int TC, bool GATED, bool ALLFUSED>
__global__ __launch_bounds__(64 * W)
void k_recur_scan(const float* __restrict__ a, const float* __restrict__ b,
                  const float* __restrict__ s0, float* __restrict__ out,
                  float* __restrict__ send, int B, int T, int N, int N8) {
    static_assert(W >= 2, "the hand-off pipeline needs at least two waves");
    __shared__ float carry[CPL * 64];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const long total = (long)B * N;
    const long flat_raw = ((long)blockIdx.x * 64 + lane) * CPL;
    const bool valid = flat_raw < total;
    // Lanes past the last channel load (but never store) the last valid
    // vector, so loads need no predicate.
    const long flat = valid ? flat_raw : total - CPL;
    const long bb = flat / N;
    const int n = (int)(flat - bb * N);
    const size_t base = (size_t)bb * T * N + n;
    bool fused[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) fused[c] = ALLFUSED || (n + c) < N8;

    constexpr int TILE = W * TC;
    const int ntiles = (T + TILE - 1) / TILE;
    const int nfull = T / TILE;
    float av[TC][CPL], bv[TC][CPL];

    // Time indices are clamped to T-1, so every prefetch is in bounds and
    // branch-free; only the final partial tile checks t < T when stepping.
    auto load_slot = [&](int tile) {
        const int t0 = tile * TILE + w * TC;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const size_t off = base + (size_t)min(t0 + k, T - 1) * N;
            ld<CPL>(av[k], a + off);
            ld<CPL>(bv[k], b + off);
        }
    };
    // b' = (1 - a) * u, computed off the critical path (in the slot before
    // this wave's own), exactly once per loaded slot.
    auto prep = [&]() {
        if constexpr (GATED) {
#pragma unroll
            for (int k = 0; k < TC; ++k)
#pragma unroll
                for (int c = 0; c < CPL; ++c) bv[k][c] = mul_rn(sub_rn(1.0f, av[k][c]), bv[k][c]);
        }
    };
    auto step = [&](float (&s)[CPL], int k) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            if constexpr (ALLFUSED) s[c] = fmaf(av[k][c], s[c], bv[k][c]);
            else s[c] = fused[c] ? fmaf(av[k][c], s[c], bv[k][c])
                                 : add_rn(mul_rn(av[k][c], s[c]), bv[k][c]);
        }
    };

    // The initial state enters through the same LDS slot as every later
    // carry, so no slot ever waits on a global load into the state registers
    // (such a wait would also drain the slot's own output stores).
    if (w == 0) {
        float s[CPL];
        ld<CPL>(s, s0 + (size_t)bb * N + n);
#pragma unroll
        for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = s[c];
    }
    load_slot(0);
    if (w == 0) prep();
    __syncthreads();
    // Slot j of tile t: wave j steps its TC time steps; wave j+1 prepares
    // its own slot of tile t; at j = W-1 wave 0 prepares its slot of t+1.
    for (int tile = 0; tile < nfull; ++tile) {
        for (int j = 0; j < W; ++j) {
            if (w == j) {
                float s[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) s[c] = carry[c * 64 + lane];
                float* po = out + base + (size_t)(tile * TILE + j * TC) * N;
#pragma unroll
                for (int k = 0; k < TC; ++k) {
                    step(s, k);
                    if (valid) st<CPL>(po + (size_t)k * N, s);
                }
#pragma unroll
                for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = s[c];
                if (tile + 1 < ntiles) load_slot(tile + 1);
            } else if (w == j + 1 || (j == W - 1 && w == 0 && tile + 1 < ntiles)) {
                prep();
            }
            barrier_lds();
        }
    }
    if (nfull < ntiles) {
        for (int j = 0; j < W; ++j) {
            if (w == j) {
                float s[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) s[c] = carry[c * 64 + lane];
                const int t0 = nfull * TILE + j * TC;
#pragma unroll
                for (int k = 0; k < TC; ++k) {
                    if (t0 + k < T) {
                        step(s, k);
                        if (valid) st<CPL>(out + base + (size_t)(t0 + k) * N, s);
                    }
                }
#pragma unroll
                for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = s[c];
            } else if (w == j + 1) {
                prep();
            }
            barrier_lds();
        }
    }
    if (w == 0 && valid) {
        float s[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) s[c] = carry[c * 64 + lane];
        st<CPL>(send + (size_t)bb * N + n, s);
    }
}

// Fast path for the common layout: every workgroup's 64*CPL channels lie in
// one batch row (N % (64*CPL) == 0) and a row fits a 2 GiB buffer window.
// Same slot pipeline as above, but all global traffic goes through buffer
// resources: the per-step row offset t*N*4 is a scalar (SGPR) operand, so the
// active slot issues only its FMAs and stores (no per-access 64-bit address
// arithmetic), and the prefetch registers hold data only, which leaves room
// for deeper time chunks. Prefetches past T re-read step T - 1 (the scalar
// row offset is not range-checked by the hardware) and are never used.

template <int CPL, int W, int TC, bool GATED>
__global__ __launch_bounds__(64 * W)
void k_recur_scan_buf(const float* __restrict__ a, const float* __restrict__ b,
                      const float* __restrict__ s0, float* __restrict__ out,
                      float* __restrict__ send, int T, int N) {
    static_assert(W >= 2, "the hand-off pipeline needs at least two waves");
    using IO = BufIO<CPL>;
    __shared__ float carry[CPL * 64];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wg_per_row = N / (64 * CPL);
    const int bb = blockIdx.x / wg_per_row;
    const int n0 = (blockIdx.x - bb * wg_per_row) * 64 * CPL;
    const size_t row = (size_t)bb * T * N;
    const uint32_t nbytes = (uint32_t)((size_t)T * N * 4);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a + row, nbytes);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(b + row, nbytes);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + row, nbytes);
    const int voff = (n0 + lane * CPL) * 4;
    const int rowb = N * 4;

    constexpr int TILE = W * TC;
    const int ntiles = (T + TILE - 1) / TILE;
    const int nfull = T / TILE;
    // bv holds the loaded b; bp the step addend b' (prepared off the critical
    // path). Separate arrays keep the two lifetimes disjoint for the allocator.
    float av[TC][CPL], bv[TC][CPL], bp[TC][CPL];

    // Steps past T (the last tile's tail) load step T - 1 instead: the row
    // offset is the scalar operand, which the buffer range check does not
    // cover. Those values are never used.
    auto load_slot = [&](int tile) {
        const int t0 = tile * TILE + w * TC;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int so = min(t0 + k, T - 1) * rowb;
            IO::load(av[k], ra, voff, so);
            IO::load(bv[k], rb, voff, so);
        }
    };
    auto prep = [&]() {
        if constexpr (GATED) {
#pragma unroll
            for (int k = 0; k < TC; ++k)
#pragma unroll
                for (int c = 0; c < CPL; ++c) bp[k][c] = mul_rn(sub_rn(1.0f, av[k][c]), bv[k][c]);
        }
    };

    if (w == 0) {
        float s[CPL];
        ld<CPL>(s, s0 + (size_t)bb * N + n0 + lane * CPL);
#pragma unroll
        for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = s[c];
    }
    load_slot(0);
    if (w == 0) prep();
    __syncthreads();
    for (int tile = 0; tile < nfull; ++tile) {
        for (int j = 0; j < W; ++j) {
            if (w == j) {
                float s[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) s[c] = carry[c * 64 + lane];
                const int t0 = tile * TILE + j * TC;
#pragma unroll
                for (int k = 0; k < TC; ++k) {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) s[c] = fmaf(av[k][c], s[c], GATED ? bp[k][c] : bv[k][c]);
                    IO::store(ro, voff, (t0 + k) * rowb, s);
                }
#pragma unroll
                for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = s[c];
                if (tile + 1 < ntiles) load_slot(tile + 1);
            } else if (w == j + 1 || (j == W - 1 && w == 0 && tile + 1 < ntiles)) {
                prep();
            }
            barrier_lds();
        }
    }
    if (nfull < ntiles) {
        for (int j = 0; j < W; ++j) {
            if (w == j) {
                float s[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) s[c] = carry[c * 64 + lane];
                const int t0 = nfull * TILE + j * TC;
#pragma unroll
                for (int k = 0; k < TC; ++k) {
                    if (t0 + k < T) {
#pragma unroll
                        for (int c = 0; c < CPL; ++c) s[c] = fmaf(av[k][c], s[c], GATED ? bp[k][c] : bv[k][c]);
                        IO::store(ro, voff, (t0 + k) * rowb, s);
                    }
                }
#pragma unroll
                for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = s[c];
            } else if (w == j + 1) {
                prep();
            }
            barrier_lds();
        }
    }
    if (w == 0) {
        float s[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) s[c] = carry[c * 64 + lane];
        st<CPL>(send + (size_t)bb * N + n0 + lane * CPL, s);
    }
}

template <bool GATED>
__global__ void k_recur_step(const float* __restrict__ a, const float* __restrict__ b,
                             float* __restrict__ s, long total, int N, int N8) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int n = (int)(i % N);
    const float x = a[i];
    const float bp = GATED ? mul_rn(sub_rn(1.0f, x), b[i]) : b[i];
    s[i] = (n < N8) ? fmaf(x, s[i], bp) : add_rn(mul_rn(x, s[i]), bp);
}

namespace {
template <int CPL, int W, int TC>
hipError_t launch_cfg(const float* a, const float* b, const float* s0, float* out,
                      float* send, int B, int T, int N, int gated, hipStream_t st) {
    const long lanes = ((long)B * N + CPL - 1) / CPL;
    const unsigned grid = (unsigned)((lanes + 63) / 64);
    const int N8 = N & ~7;
    const dim3 g(grid), blk(64 * W);
    if (N == N8) {
        if (gated)
            hipLaunchKernelGGL((k_recur_scan<CPL, W, TC, true, true>), g, blk, 0, st,
                               a, b, s0, out, send, B, T, N, N8);
        else
            hipLaunchKernelGGL((k_recur_scan<CPL, W, TC, false, true>), g, blk, 0, st,
                               a, b, s0, out, send, B, T, N, N8);
    } else {
        if (gated)
            hipLaunchKernelGGL((k_recur_scan<CPL, W, TC, true, false>), g, blk, 0, st,
                               a, b, s0, out, send, B, T, N, N8);
        else
            hipLaunchKernelGGL((k_recur_scan<CPL, W, TC, false, false>), g, blk, 0, st,
                               a, b, s0, out, send, B, T, N, N8);
    }
    return hipGetLastError();
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }
}  // namespace

template <int CPL, int W, int TC>
hipError_t launch_buf(const float* a, const float* b, const float* s0, float* out, float* send,
                      int B, int T, int N, int gated, hipStream_t st) {
    const unsigned grid = (unsigned)((long)B * N / (64 * CPL));
    if (gated)
        hipLaunchKernelGGL((k_recur_scan_buf<CPL, W, TC, true>), dim3(grid), dim3(64 * W), 0, st,
                           a, b, s0, out, send, T, N);
    else
        hipLaunchKernelGGL((k_recur_scan_buf<CPL, W, TC, false>), dim3(grid), dim3(64 * W), 0, st,
                           a, b, s0, out, send, T, N);
    return hipGetLastError();
}

// Launch-shape selection. SNHIP_SCAN_SHAPE="kind,cpl,w,tc" (kind "buf" or
// "gen") pins one compiled shape for the tuning sweep and tests; otherwise the
// buffer kernel when the layout allows it, else the generic kernel.
snhip_status launch_recur_scan(const float* a, const float* b, const float* s0,
                               float* out, float* send, int B, int T, int N,
                               int gated, hipStream_t st) {
    const bool al8 = aligned(a, 8) && aligned(b, 8) && aligned(s0, 8) && aligned(out, 8) &&
                     aligned(send, 8);
    const bool al16 = aligned(a, 16) && aligned(b, 16) && aligned(s0, 16) &&
                      aligned(out, 16) && aligned(send, 16);
    const long chans = (long)B * N;
    auto buf_ok = [&](int cpl, int tile) {
        return N % (64 * cpl) == 0 && (cpl < 2 || al8) && (cpl < 4 || al16) &&
               (long)(T + tile) * N * 4 < (1L << 31);
    };
    char kind = 'g';
    int cpl = 1, w = 8, tc = 16;
    if (N % 2 == 0 && al8 && chans / 128 >= 192) cpl = 2;
    if (buf_ok(2, 2 * 32) && chans / 128 >= 128) { kind = 'b'; cpl = 2; w = 2; tc = 32; }
    else if (buf_ok(1, 4 * 32)) { kind = 'b'; cpl = 1; w = 4; tc = 32; }
    if (const char* env = getenv("SNHIP_SCAN_SHAPE")) {
        char k[8] = {0};
        int c = 0, ww = 0, t = 0;
        if (sscanf(env, "%3[a-z],%d,%d,%d", k, &c, &ww, &t) == 4) {
            kind = k[0]; cpl = c; w = ww; tc = t;
        }
        if (kind == 'b' && !buf_ok(cpl, w * tc)) return SNHIP_E_INVAL;
        if (kind == 'g' && ((cpl == 2 && (N % 2 || !al8)) || (cpl == 4 && (N % 4 || !al16))))
            return SNHIP_E_INVAL;
    }
    hipError_t e = hipErrorInvalidValue;
#define SNHIP_GEN_CASE(C, WW, TT)                                                   \
    if (kind == 'g' && cpl == C && w == WW && tc == TT)                             \
        e = launch_cfg<C, WW, TT>(a, b, s0, out, send, B, T, N, gated, st);         \
    else
#define SNHIP_BUF_CASE(C, WW, TT)                                                   \
    if (kind == 'b' && cpl == C && w == WW && tc == TT)                             \
        e = launch_buf<C, WW, TT>(a, b, s0, out, send, B, T, N, gated, st);         \
    else
    SNHIP_GEN_CASE(1, 8, 16)
    SNHIP_GEN_CASE(2, 8, 16)
    SNHIP_GEN_CASE(2, 2, 32)
    SNHIP_GEN_CASE(4, 4, 16)
    SNHIP_BUF_CASE(1, 4, 32)
    SNHIP_BUF_CASE(1, 4, 64)
    SNHIP_BUF_CASE(2, 2, 32)
    SNHIP_BUF_CASE(2, 2, 64)
    SNHIP_BUF_CASE(2, 4, 32)
    SNHIP_BUF_CASE(2, 4, 64)
    SNHIP_BUF_CASE(2, 8, 32)
    SNHIP_BUF_CASE(4, 2, 32)
    { set_last_error("SNHIP_SCAN_SHAPE names a shape that is not compiled"); return SNHIP_E_UNSUPPORTED; }
#undef SNHIP_GEN_CASE
#undef SNHIP_BUF_CASE
    if (e != hipSuccess) {
        set_last_error(std::string("recur_scan launch: ") + hipGetErrorString(e));
        return SNHIP_E_DEVICE;
    }
    return SNHIP_OK;
}

snhip_status launch_recur_step(const float* a, const float* b, float* s, int B, int N,
                               int gated, hipStream_t st) {
    const long total = (long)B * N;
    const unsigned grid = (unsigned)((total + 255) / 256);
    if (gated)
        hipLaunchKernelGGL((k_recur_step<true>), dim3(grid), dim3(256), 0, st, a, b, s, total, N, N & ~7);
    else
        hipLaunchKernelGGL((k_recur_step<false>), dim3(grid), dim3(256), 0, st, a, b, s, total, N, N & ~7);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// ---------------------------------------------------------------------------
// Backward of the gated scan s_t = p_t s_{t-1} + (1 - p_t) nu_t
// (sunnynet/kernels/scan_avx2.c:50-99): per channel, in reverse time,
//   ds += dout_t;  dnu_t = ds (1 - p_t);  dp_t = ds (s_{t-1} - nu_t);  ds *= p_t
// with s_{-1} = s0, and ds0 = ds after t = 0. The reference's 8-wide path and
// scalar tail use these unfused operations in this order, so the result is
// bit-identical. Same slot pipeline as k_recur_scan_buf, walking time
// backwards: wave w owns reversed steps [w TC, (w + 1) TC) of every tile of
// W TC steps; while the active wave runs its TC dependent add/multiply pairs
// the next wave prepares s_{t-1} - nu_t and 1 - p_t, off the carried chain.
// HBM traffic per step: four reads (dout, p, nu, s_{t-1}), two writes.
template <int CPL, int W, int TC>
__global__ __launch_bounds__(64 * W)
void k_scan_bwd_buf(const float* __restrict__ p, const float* __restrict__ nu,
                    const float* __restrict__ s0, const float* __restrict__ out,
                    const float* __restrict__ dout, float* __restrict__ dp,
                    float* __restrict__ dnu, float* __restrict__ ds0, int T, int N) {
    static_assert(W >= 2, "the hand-off pipeline needs at least two waves");
    using IO = BufIO<CPL>;
    __shared__ float carry[CPL * 64];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wg_per_row = N / (64 * CPL);
    const int bb = blockIdx.x / wg_per_row;
    const int n0 = (blockIdx.x - bb * wg_per_row) * 64 * CPL;
    const size_t row = (size_t)bb * T * N;
    const uint32_t nbytes = (uint32_t)((size_t)T * N * 4);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p + row, nbytes);
    const __amdgpu_buffer_rsrc_t rn = make_rsrc(nu + row, nbytes);
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + row, nbytes);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(dout + row, nbytes);
    const __amdgpu_buffer_rsrc_t rgp = make_rsrc(dp + row, nbytes);
    const __amdgpu_buffer_rsrc_t rgn = make_rsrc(dnu + row, nbytes);
    const int voff = (n0 + lane * CPL) * 4;
    const int rowb = N * 4;

    constexpr int TILE = W * TC;
    const int ntiles = (T + TILE - 1) / TILE;
    // pv: p; gv: dout; dv: nu, then s_{t-1} - nu; qv: s_{t-1}, then 1 - p.
    float pv[TC][CPL], gv[TC][CPL], dv[TC][CPL], qv[TC][CPL], sz[CPL];
    ld<CPL>(sz, s0 + (size_t)bb * N + n0 + lane * CPL);

    // Time step of reversed step k of this wave's slot in `tile`.
    auto t_of = [&](int tile, int k) { return T - 1 - (tile * TILE + w * TC + k); };
    // Steps before 0 (the last tile's tail) load step 0 (the scalar row offset
    // is not range-checked); they are never used.
    auto load_slot = [&](int tile) {
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int t = max(t_of(tile, k), 0);
            const int so = t * rowb, sp = max(t - 1, 0) * rowb;
            IO::load(pv[k], rp, voff, so);
            IO::load(gv[k], rd, voff, so);
            IO::load(dv[k], rn, voff, so);
            IO::load(qv[k], ro, voff, sp);
        }
    };
    auto prep = [&](int tile) {
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const bool first = t_of(tile, k) == 0;           // s_{-1} is s0
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                dv[k][c] = sub_rn(first ? sz[c] : qv[k][c], dv[k][c]);
                qv[k][c] = sub_rn(1.0f, pv[k][c]);
            }
        }
    };
    auto run_slot = [&](int tile) {
        float ds[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) ds[c] = carry[c * 64 + lane];
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            const int t = t_of(tile, k);
            if (t < 0) break;
            float gn[CPL], gp[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                ds[c] = add_rn(gv[k][c], ds[c]);
                gn[c] = mul_rn(ds[c], qv[k][c]);
                gp[c] = mul_rn(ds[c], dv[k][c]);
                ds[c] = mul_rn(ds[c], pv[k][c]);
            }
            IO::store(rgn, voff, t * rowb, gn);
            IO::store(rgp, voff, t * rowb, gp);
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = ds[c];
    };

    if (w == 0)
#pragma unroll
        for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = 0.0f;
    load_slot(0);
    if (w == 0) prep(0);
    __syncthreads();
    for (int tile = 0; tile < ntiles; ++tile) {
        for (int j = 0; j < W; ++j) {
            if (w == j) {
                run_slot(tile);
                if (tile + 1 < ntiles) load_slot(tile + 1);
            } else if (w == j + 1) {
                prep(tile);
            } else if (j == W - 1 && w == 0 && tile + 1 < ntiles) {
                prep(tile + 1);
            }
            barrier_lds();
        }
    }
    if (w == 0) {
        float ds[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) ds[c] = carry[c * 64 + lane];
        st<CPL>(ds0 + (size_t)bb * N + n0 + lane * CPL, ds);
    }
}

// Any layout: one lane per channel, straight through time.
__global__ void k_scan_bwd_gen(const float* __restrict__ p, const float* __restrict__ nu,
                               const float* __restrict__ s0, const float* __restrict__ out,
                               const float* __restrict__ dout, float* __restrict__ dp,
                               float* __restrict__ dnu, float* __restrict__ ds0, int B, int T, int N) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)B * N) return;
    const long bb = i / N;
    const int n = (int)(i - bb * N);
    const size_t rb = (size_t)bb * T * N + n;
    float ds = 0.0f;
    for (int t = T - 1; t >= 0; --t) {
        const size_t off = rb + (size_t)t * N;
        ds = add_rn(dout[off], ds);
        const float pv = p[off];
        const float sprev = t > 0 ? out[off - N] : s0[(size_t)bb * N + n];
        dnu[off] = mul_rn(ds, sub_rn(1.0f, pv));
        dp[off] = mul_rn(ds, sub_rn(sprev, nu[off]));
        ds = mul_rn(ds, pv);
    }
    ds0[(size_t)bb * N + n] = ds;
}

snhip_status launch_scan_bwd(const float* p, const float* nu, const float* s0, const float* out,
                             const float* dout, float* dp, float* dnu, float* ds0, int B, int T,
                             int N, hipStream_t st) {
    const bool al8 = aligned(p, 8) && aligned(nu, 8) && aligned(s0, 8) && aligned(out, 8) &&
                     aligned(dout, 8) && aligned(dp, 8) && aligned(dnu, 8) && aligned(ds0, 8);
    constexpr int C = 2, WW = 2, TT = 16;
    const bool buf = N % (64 * C) == 0 && al8 && (long)T * N * 4 < (1L << 31) &&
                     (long)B * N / 128 >= 128;
    if (buf) {
        const unsigned grid = (unsigned)((long)B * N / (64 * C));
        hipLaunchKernelGGL((k_scan_bwd_buf<C, WW, TT>), dim3(grid), dim3(64 * WW), 0, st, p, nu, s0, out,
                           dout, dp, dnu, ds0, T, N);
    } else {
        const long total = (long)B * N;
        hipLaunchKernelGGL(k_scan_bwd_gen, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p, nu,
                           s0, out, dout, dp, dnu, ds0, B, T, N);
    }
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// ---- achievable-bandwidth calibration: plain streaming kernels over the
// scan's byte pattern (two fp32 arrays read, one written) and over its reads
// alone, float4 per lane, non-temporal like the scan, grid-stride. They give
// the bandwidth a straightforward stream reaches on the device, beside the
// nominal HBM peak the scan is quoted against.
namespace {
typedef float v4f_ __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_hbm_add(const v4f_* __restrict__ a, const v4f_* __restrict__ b,
                                                 v4f_* __restrict__ c, size_t n4) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + stride < n4; i += 2 * stride) {
        const v4f_ x0 = __builtin_nontemporal_load(a + i), x1 = __builtin_nontemporal_load(a + i + stride);
        const v4f_ y0 = __builtin_nontemporal_load(b + i), y1 = __builtin_nontemporal_load(b + i + stride);
        __builtin_nontemporal_store(x0 + y0, c + i);
        __builtin_nontemporal_store(x1 + y1, c + i + stride);
    }
    for (; i < n4; i += stride) c[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void k_hbm_read2(const v4f_* __restrict__ a, const v4f_* __restrict__ b,
                                                   v4f_* __restrict__ c, size_t n4) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    v4f_ acc = {0.f, 0.f, 0.f, 0.f};
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
        acc += __builtin_nontemporal_load(a + i) + __builtin_nontemporal_load(b + i);
    // one store per workgroup-sized slice of c keeps the sums live
    if (threadIdx.x == 0) c[blockIdx.x] = acc;
}
}  // namespace

}  // namespace snhip

extern "C" snhip_status snhip_abi_hbm_probe_dev(int32_t kind, const float* a, const float* b, float* c,
                                                 int64_t n, int32_t grid, void* stream) {
    using namespace snhip;
    if (!a || !b || !c || n <= 0 || n % 4 || grid <= 0 || (kind != 0 && kind != 1) ||
        !aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16) || (kind == 1 && (int64_t)grid * 4 > n))
        return SNHIP_E_INVAL;
    const size_t n4 = (size_t)n / 4;
    if (kind == 0)
        hipLaunchKernelGGL(k_hbm_add, dim3((unsigned)grid), dim3(256), 0, as_stream(stream),
                           reinterpret_cast<const v4f_*>(a), reinterpret_cast<const v4f_*>(b),
                           reinterpret_cast<v4f_*>(c), n4);
    else
        hipLaunchKernelGGL(k_hbm_read2, dim3((unsigned)grid), dim3(256), 0, as_stream(stream),
                           reinterpret_cast<const v4f_*>(a), reinterpret_cast<const v4f_*>(b),
                           reinterpret_cast<v4f_*>(c), n4);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}
