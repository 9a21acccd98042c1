// Buffer-resource loads and stores of 1, 2 or 4 consecutive floats for the
// streaming kernels (gated scan, fused core): the per-step row offset is the
// scalar (SGPR) operand, so a kernel walking time issues no per-access 64-bit
// address arithmetic. The hardware range-checks only the vector offset, never
// the scalar one: callers clamp the scalar offset into the buffer themselves.
#pragma once

#include "common.h"

namespace snhip {

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Cache policy of every scan load and store: non-temporal ("nt"), i.e.
// streamed through the caches without displacing other lines. Each byte is
// touched exactly once, and on gfx950 this raises the sustained rate of the
// 2-read/1-write mix by about 10 % over the default policy.
constexpr int kStream = 2;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int CPL> struct BufIO;
template <> struct BufIO<1> {
    static __device__ __forceinline__ void load(float (&v)[1], __amdgpu_buffer_rsrc_t r, int vo, int so) {
        v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, kStream));
    }
    static __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r, int vo, int so, const float (&v)[1]) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, vo, so, kStream);
    }
};
template <> struct BufIO<2> {
    using U = u32x2;
    static __device__ __forceinline__ void load(float (&v)[2], __amdgpu_buffer_rsrc_t r, int vo, int so) {
        U x = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, kStream);
        v[0] = __uint_as_float(x[0]); v[1] = __uint_as_float(x[1]);
    }
    static __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r, int vo, int so, const float (&v)[2]) {
        U x; x[0] = __float_as_uint(v[0]); x[1] = __float_as_uint(v[1]);
        __builtin_amdgcn_raw_buffer_store_b64(x, r, vo, so, kStream);
    }
};
template <> struct BufIO<4> {
    using U = u32x4;
    static __device__ __forceinline__ void load(float (&v)[4], __amdgpu_buffer_rsrc_t r, int vo, int so) {
        U x = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, kStream);
        for (int c = 0; c < 4; ++c) v[c] = __uint_as_float(x[c]);
    }
    static __device__ __forceinline__ void store(__amdgpu_buffer_rsrc_t r, int vo, int so, const float (&v)[4]) {
        U x;
        for (int c = 0; c < 4; ++c) x[c] = __float_as_uint(v[c]);
        __builtin_amdgcn_raw_buffer_store_b128(x, r, vo, so, kStream);
    }
};

// Raw (stride 0) buffer descriptor word 3 for gfx9-family targets.
constexpr int kBufDword3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufDword3);
}

}  // namespace snhip
