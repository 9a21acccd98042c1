// Exchange words of the one-launch RWKV-7 steps (rkpersist.hip, rkexact.hip).
//
// Every exchanged value has its own 64-bit word: the epoch of the launch step
// that wrote it in the high half, the value's bits in the low half, stored
// and loaded as one single-copy-atomic word at agent scope. A reader polls a
// word until it carries its step's epoch, so data and readiness travel in one
// round trip and no grid barrier is needed.
#pragma once

#include "common.h"

namespace snhip {
namespace rkx {

typedef unsigned long long u64;

__device__ __forceinline__ void ex_put_bits(u64* p, uint32_t bits, unsigned ep) {
    __hip_atomic_store(p, ((u64)ep << 32) | (u64)bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ex_put(u64* p, float v, unsigned ep) { ex_put_bits(p, __float_as_uint(v), ep); }
__device__ __forceinline__ u64 ex_get(const u64* p) {
    return __hip_atomic_load(const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool ex_ok(u64 w, unsigned ep) { return (uint32_t)(w >> 32) == ep; }
__device__ __forceinline__ float ex_f(u64 w) { return __uint_as_float((uint32_t)w); }

struct PollCtl {
    unsigned* err;
    unsigned limit;
    unsigned want;   // the step's epoch (plus the test stall)
};

// Re-polls the words of w still short of the epoch (word k from src[k];
// words a thread does not take start out ready) until all carry it. False on
// a time-out (the thread then sets the error word) or when another
// workgroup reported one. (Two rounds in flight at once, the next issued
// before the one in hand is waited for, made the waits longer: the doubled
// polling traffic delayed the producers more than it shortened the polls.)
template <int W>
__device__ __forceinline__ bool ex_spin(u64 (&w)[W], const u64* const (&src)[W], const PollCtl& pc) {
    unsigned spins = 0;
    while (true) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < W; ++k) all = all && ex_ok(w[k], pc.want);
        if (all) return true;
        if ((++spins & 255) == 0) {
            if (__hip_atomic_load(pc.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
            if (spins > pc.limit) {
                __hip_atomic_store(pc.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return false;
            }
        }
#pragma unroll
        for (int k = 0; k < W; ++k)
            if (!ex_ok(w[k], pc.want)) w[k] = ex_get(src[k]);
    }
}

// Words [0, n) of src into dst (LDS), word i by thread i mod NTH; W words per
// thread at most (n <= W NTH). The workgroup's barrier between the polls and
// the writes: every wave is done with what dst held before (the caller's
// agreement barrier then orders the writes before any read).
template <int W, int NTH>
__device__ __forceinline__ bool poll_vec(const u64* src, int n, float* dst, const PollCtl& pc) {
    const int tid = threadIdx.x;
    u64 w[W];
    const u64* at[W];
#pragma unroll
    for (int k = 0; k < W; ++k) {
        const int i = k * NTH + tid;
        at[k] = src + min(i, n - 1);
        w[k] = i < n ? ex_get(at[k]) : ((u64)pc.want << 32);
    }
    const bool ok = ex_spin(w, at, pc);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < W; ++k) {
        const int i = k * NTH + tid;
        if (i < n) dst[i] = ex_f(w[k]);
    }
    return ok;
}

// Plain values shared with other workgroups (the token-shift vectors).
__device__ __forceinline__ void st_ag(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_ag(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This workgroup's share [lo, hi) of n rows.
__device__ __forceinline__ void share(int n, int wg, int G, int& lo, int& hi) {
    lo = (int)((long)n * wg / G);
    hi = (int)((long)n * (wg + 1) / G);
}

// Keeps loads issued so far where they are (the optimizer would sink them to
// their use, past a wait).
__device__ __forceinline__ void issued() { asm volatile("" ::: "memory"); }

}  // namespace rkx
}  // namespace snhip
