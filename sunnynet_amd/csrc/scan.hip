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
#include "common.h"

namespace snhip {

template <int CPL> struct VecT;
template <> struct VecT<1> { using T = float; };
template <> struct VecT<2> { using T = float2; };
template <> struct VecT<4> { using T = float4; };

template <int CPL>
__device__ __forceinline__ void ld(float (&v)[CPL], const float* p) {
    using V = typename VecT<CPL>::T;
    V x = *reinterpret_cast<const V*>(p);
    if constexpr (CPL == 1) { v[0] = x; }
    else if constexpr (CPL == 2) { v[0] = x.x; v[1] = x.y; }
    else { v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; }
}

template <int CPL>
__device__ __forceinline__ void st(float* p, const float (&v)[CPL]) {
    using V = typename VecT<CPL>::T;
    V x;
    if constexpr (CPL == 1) { x = v[0]; }
    else if constexpr (CPL == 2) { x.x = v[0]; x.y = v[1]; }
    else { x.x = v[0]; x.y = v[1]; x.z = v[2]; x.w = v[3]; }
    *reinterpret_cast<V*>(p) = x;
}

template <int CPL, int W, int TC, bool GATED>
__global__ __launch_bounds__(64 * W)
void k_recur_scan(const float* __restrict__ a, const float* __restrict__ b,
                  const float* __restrict__ s0, float* __restrict__ out,
                  float* __restrict__ send, int B, int T, int N, int N8) {
    __shared__ float carry[CPL * 64];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const long flat = ((long)blockIdx.x * 64 + lane) * CPL;
    const bool valid = flat < (long)B * N;
    const long bb = valid ? flat / N : 0;
    const int n = valid ? (int)(flat - bb * N) : 0;
    const size_t base = (size_t)bb * T * N + n;
    bool fused[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) fused[c] = (n + c) < N8;

    constexpr int TILE = W * TC;
    const int ntiles = (T + TILE - 1) / TILE;
    float av[TC][CPL], bv[TC][CPL];

    auto load_slot = [&](int tile) {
        const int t0 = tile * TILE + w * TC;
        const float* pa = a + base + (size_t)t0 * N;
        const float* pb = b + base + (size_t)t0 * N;
#pragma unroll
        for (int k = 0; k < TC; ++k) {
            if (valid && t0 + k < T) {
                ld<CPL>(av[k], pa + (size_t)k * N);
                ld<CPL>(bv[k], pb + (size_t)k * N);
            }
        }
    };

    load_slot(0);
    for (int tile = 0; tile < ntiles; ++tile) {
        for (int j = 0; j < W; ++j) {
            if (w == j) {
                float s[CPL];
                if (tile == 0 && j == 0) {
                    if (valid) ld<CPL>(s, s0 + (size_t)bb * N + n);
                    else {
#pragma unroll
                        for (int c = 0; c < CPL; ++c) s[c] = 0.0f;
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) s[c] = carry[c * 64 + lane];
                }
                const int t0 = tile * TILE + j * TC;
                float* po = out + base + (size_t)t0 * N;
#pragma unroll
                for (int k = 0; k < TC; ++k) {
                    if (t0 + k < T) {
#pragma unroll
                        for (int c = 0; c < CPL; ++c) {
                            const float x = av[k][c];
                            const float bp = GATED ? mul_rn(sub_rn(1.0f, x), bv[k][c]) : bv[k][c];
                            s[c] = fused[c] ? fmaf(x, s[c], bp) : add_rn(mul_rn(x, s[c]), bp);
                        }
                        if (valid) st<CPL>(po + (size_t)k * N, s);
                    }
                }
#pragma unroll
                for (int c = 0; c < CPL; ++c) carry[c * 64 + lane] = s[c];
                if (tile + 1 < ntiles) load_slot(tile + 1);
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
    if (gated)
        hipLaunchKernelGGL((k_recur_scan<CPL, W, TC, true>), dim3(grid), dim3(64 * W), 0, st,
                           a, b, s0, out, send, B, T, N, N8);
    else
        hipLaunchKernelGGL((k_recur_scan<CPL, W, TC, false>), dim3(grid), dim3(64 * W), 0, st,
                           a, b, s0, out, send, B, T, N, N8);
    return hipGetLastError();
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }
}  // namespace

// Launch-shape selection. SNHIP_SCAN_SHAPE="cpl,w,tc" pins one of the compiled
// shapes (used by the tuning sweep); otherwise the widest vector width the
// layout allows, with enough workgroups to cover the chip.
snhip_status launch_recur_scan(const float* a, const float* b, const float* s0,
                               float* out, float* send, int B, int T, int N,
                               int gated, hipStream_t st) {
    int cpl = 1, w = 8, tc = 16;
    const bool al8 = aligned(a, 8) && aligned(b, 8) && aligned(s0, 8) && aligned(out, 8) &&
                     aligned(send, 8);
    const bool al16 = aligned(a, 16) && aligned(b, 16) && aligned(s0, 16) &&
                      aligned(out, 16) && aligned(send, 16);
    const long chans = (long)B * N;
    if (N % 2 == 0 && al8 && chans / 128 >= 192) cpl = 2;
    if (N % 4 == 0 && al16 && chans / 256 >= 256) cpl = 4;
    if (const char* env = getenv("SNHIP_SCAN_SHAPE")) {
        int c = 0, ww = 0, t = 0;
        if (sscanf(env, "%d,%d,%d", &c, &ww, &t) == 3) { cpl = c; w = ww; tc = t; }
        if ((cpl == 2 && (N % 2 || !al8)) || (cpl == 4 && (N % 4 || !al16))) return SNHIP_E_INVAL;
    }
    hipError_t e = hipErrorInvalidValue;
#define SNHIP_SCAN_CASE(C, WW, TT)                                                  \
    if (cpl == C && w == WW && tc == TT)                                            \
        e = launch_cfg<C, WW, TT>(a, b, s0, out, send, B, T, N, gated, st);         \
    else
    SNHIP_SCAN_CASE(1, 8, 16)
    SNHIP_SCAN_CASE(1, 16, 16)
    SNHIP_SCAN_CASE(2, 8, 16)
    SNHIP_SCAN_CASE(2, 16, 8)
    SNHIP_SCAN_CASE(2, 8, 32)
    SNHIP_SCAN_CASE(2, 4, 32)
    SNHIP_SCAN_CASE(4, 8, 16)
    SNHIP_SCAN_CASE(4, 8, 8)
    { set_last_error("SNHIP_SCAN_SHAPE names a shape that is not compiled"); return SNHIP_E_UNSUPPORTED; }
#undef SNHIP_SCAN_CASE
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

}  // namespace snhip
