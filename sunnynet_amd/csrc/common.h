// Shared host/device helpers for the SunnyNet HIP backend (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "snhip_abi.h"

namespace snhip {

// Per-thread text of the last HIP failure, exposed by snhip_abi_last_error.
void set_last_error(const std::string& msg);
const std::string& last_error();

// Records the failing call and returns SNHIP_E_DEVICE from the enclosing
// function (which must return snhip_status).
#define SNHIP_CHECK(expr)                                                     \
    do {                                                                      \
        hipError_t e_ = (expr);                                               \
        if (e_ != hipSuccess) {                                               \
            ::snhip::set_last_error(std::string(#expr) + ": " +               \
                                    hipGetErrorString(e_));                   \
            return SNHIP_E_DEVICE;                                            \
        }                                                                     \
    } while (0)

// Same, for functions returning a pointer (returns nullptr).
#define SNHIP_CHECK_NULL(expr)                                                \
    do {                                                                      \
        hipError_t e_ = (expr);                                               \
        if (e_ != hipSuccess) {                                               \
            ::snhip::set_last_error(std::string(#expr) + ": " +               \
                                    hipGetErrorString(e_));                   \
            return nullptr;                                                   \
        }                                                                     \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Unsigned value of an environment variable (at least lo), or dflt if unset.
// Read at call time, so a test may change it between calls of one handle.
inline unsigned env_unsigned(const char* name, unsigned dflt, unsigned lo) {
    const char* e = getenv(name);
    if (!e) return dflt;
    const long v = atol(e);
    return v < (long)lo ? lo : (unsigned)v;
}

// Launches a grid-synchronizing persistent kernel whose grid is sized to
// co-reside: cooperatively (the runtime checks residency), or, with
// SNHIP_COOP=0, as an ordinary launch of the same grid (for tools that do not
// handle cooperative launches; every grid-wide wait in these kernels is
// bounded, so a grid that did not co-reside ends in a reported time-out).
inline hipError_t launch_persistent(const void* k, dim3 grid, dim3 block, void** args, hipStream_t st) {
    if (env_unsigned("SNHIP_COOP", 1, 0) == 0) return hipLaunchKernel(k, grid, block, args, 0, st);
    return hipLaunchCooperativeKernel(k, grid, block, args, 0, st);
}

// Waits for this wave's outstanding LDS operations only (gfx9 s_waitcnt
// encoding: vmcnt = 63, expcnt = 7, lgkmcnt = 0); global loads stay in flight.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Workgroup barrier that orders LDS traffic but does not drain outstanding
// global loads (a full __syncthreads() would wait for every prefetch).
__device__ __forceinline__ void barrier_lds() {
    wait_lds();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Reference-order arithmetic helpers. The library is compiled with
// -ffp-contract=off, so these stay separate roundings.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float sub_rn(float a, float b) { return __fsub_rn(a, b); }

}  // namespace snhip

// Internal launchers shared across translation units.
namespace snhip {
snhip_status launch_scan_bwd(const float* p, const float* nu, const float* s0, const float* out,
                             const float* dout, float* dp, float* dnu, float* ds0, int B, int T,
                             int N, hipStream_t st);
snhip_status launch_core_fwd(const float* q, const float* delta, const float* s0, float* states,
                             float* uo, float* po, int B, int T, int D, hipStream_t st);
snhip_status launch_core_bwd(const float* q, const float* delta, const float* s0, const float* states,
                             const float* uo, const float* po, const float* dstate, const float* du_in,
                             float* dq, float* ddelta, float* ds0, int B, int T, int D, hipStream_t st);
snhip_status launch_core_bwd_noalloc(const float* q, const float* delta, const float* s0,
                                     const float* states, const float* uo, const float* po,
                                     const float* dstate, const float* du_in, float* dq, float* ddelta,
                                     float* ds0, int B, int T, int D, hipStream_t st);
snhip_status launch_recur_scan(const float* a, const float* b, const float* s0,
                               float* out, float* send, int B, int T, int N,
                               int gated, hipStream_t st);
snhip_status launch_recur_step(const float* a, const float* b, float* s, int B,
                               int N, int gated, hipStream_t st);
snhip_status launch_quant_i4(const float* x, uint8_t* q, float* scale, int rows,
                             int N, int block, hipStream_t st);
snhip_status launch_dequant_i4(const uint8_t* q, const float* scale, float* x,
                               int rows, int N, int block, hipStream_t st);
}  // namespace snhip
