// expf and tanhf rounded exactly as the host C library rounds them.
//
// The reference runtime is C compiled against glibc, so its transcendentals
// are glibc's: expf is the table-driven double-precision algorithm of ARM's
// optimized-routines (exp(x) = 2^(k/32) 2^(r/32), a 32-entry table of
// 2^(i/32) and a cubic in r, one final rounding to float) in the form glibc
// selects on x86-64 CPUs with FMA (every product feeding a sum fused), and
// tanhf is
// fdlibm's (tanh via expm1f with its reduction by ln2_hi/ln2_lo and a
// degree-5 polynomial in x^2/4). Both are restated here from their published
// algorithms so that a device step that otherwise follows the reference's
// operation order produces the reference's bits. Host and device share the
// code; tests compare it with the host libm on the CPU and on the GPU.
//
// The table entries are derived, not copied: T[i] = bits(2^(i/32)) - (i << 47),
// with 2^(i/32) the correctly rounded double.
//
// Notices of the works whose published constants and steps are restated here:
//
// expf: ARM optimized-routines (math/expf.c, math/exp2f_data.c), as carried
// by glibc (sysdeps/ieee754/flt-32/e_expf.c).
//   Copyright (c) 2017-2018, Arm Limited.
//   SPDX-License-Identifier: MIT
//   Permission is hereby granted, free of charge, to any person obtaining a
//   copy of this software and associated documentation files (the
//   "Software"), to deal in the Software without restriction, including
//   without limitation the rights to use, copy, modify, merge, publish,
//   distribute, sublicense, and/or sell copies of the Software, and to permit
//   persons to whom the Software is furnished to do so, subject to the
//   following conditions: The above copyright notice and this permission
//   notice shall be included in all copies or substantial portions of the
//   Software. THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND,
//   EXPRESS OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF
//   MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN
//   NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM,
//   DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR
//   OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE
//   USE OR OTHER DEALINGS IN THE SOFTWARE.
//
// expm1f / tanhf: fdlibm (s_expm1.c, s_tanh.c; float forms s_expm1f.c,
// s_tanhf.c, conversion to float by Ian Lance Taylor, Cygnus Support).
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice
//   is preserved.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace snhip {
namespace refmath {

__host__ __device__ __forceinline__ uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
__host__ __device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ __forceinline__ uint64_t d2u(double x) { return __builtin_bit_cast(uint64_t, x); }
__host__ __device__ __forceinline__ double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// bits(2^(i/32)) - (i << 47), i = 0..31
inline constexpr uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// glibc expf (round to nearest), with the table read from tab (kExp2Tab's
// entries; a kernel may pass a copy in LDS: indexed per lane, the constant
// array is a global-memory load on the critical path).
__host__ __device__ inline float expf_tab(float x, const uint64_t* tab) {
    constexpr double kN = 32.0;
    constexpr double C0 = 0x1.c6af84b912394p-5 / kN / kN / kN;
    constexpr double C1 = 0x1.ebfce50fac4f3p-3 / kN / kN;
    constexpr double C2 = 0x1.62e42ff0c52d6p-1 / kN;
    constexpr double InvLn2N = 0x1.71547652b82fep+0 * kN;
    constexpr double Shift = 0x1.8p+52;
    const uint32_t abstop = (f2u(x) >> 20) & 0x7ff;
    if (abstop >= (0x42b00000u >> 20)) {                       // |x| >= 88 or NaN
        if (f2u(x) == 0xff800000u) return 0.0f;                 // -inf
        if (abstop >= (0x7f800000u >> 20)) return x + x;        // inf or NaN
        if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);         // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                    // underflow
    }
    // The host library is its FMA build (x86-64 with FMA): every product
    // that feeds a sum is fused, including x InvLn2N into both of its uses.
    const double xd = (double)x;
    double kd = fma(InvLn2N, xd, Shift);                        // round to nearest int
    const uint64_t ki = d2u(kd);
    kd -= Shift;
    const double r = fma(InvLn2N, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    const double s = u2d(t);
    const double p = fma(C0, r, C1);
    const double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(p, r2, y);
    y = y * s;
    return (float)y;
}

__host__ __device__ inline float expf(float x) { return expf_tab(x, kExp2Tab); }

// fdlibm expm1f.
__host__ __device__ inline float expm1f(float x) {
    constexpr float o_threshold = 8.8721679688e+01f, ln2_hi = 6.9313812256e-01f,
                    ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    constexpr float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                    Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    constexpr float huge = 1.0e+30f, tiny = 1.0e-30f;
    uint32_t hx = f2u(x);
    const uint32_t xsb = hx & 0x80000000u;
    float y = xsb ? -x : x;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {                                    // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {                                // |x| >= 88.72...
            if (hx > 0x7f800000u) return x + x;                 // NaN
            if (hx == 0x7f800000u) return xsb ? -1.0f : x;      // +-inf
            if (x > o_threshold) return huge * huge;            // overflow
        }
        if (xsb) return tiny - 1.0f;                            // x < -27 ln2
    }
    float hi, lo, c = 0.0f, t;
    int32_t k;
    if (hx > 0x3eb17218u) {                                     // |x| > ln2 / 2
        if (hx < 0x3F851592u) {                                 // and < 1.5 ln2
            if (!xsb) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int32_t)(invln2 * x + (xsb ? -0.5f : 0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;                                // exact
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {                              // |x| < 2^-25
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    if (k <= -2 || k > 56) {
        y = 1.0f - (e - x);
        y = u2f(f2u(y) + ((uint32_t)k << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        t = u2f(0x3f800000u - (0x1000000u >> k));               // 1 - 2^-k
        y = t - (e - x);
        y = u2f(f2u(y) + ((uint32_t)k << 23));
    } else {
        t = u2f((uint32_t)(0x7f - k) << 23);                    // 2^-k
        y = x - (e + t);
        y += 1.0f;
        y = u2f(f2u(y) + ((uint32_t)k << 23));
    }
    return y;
}

// fdlibm tanhf.
__host__ __device__ inline float tanhf(float x) {
    const uint32_t jx = f2u(x), ix = jx & 0x7fffffffu;
    if (ix >= 0x7f800000u) return (jx >> 31) ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;
    float z;
    if (ix < 0x41b00000u) {                                     // |x| < 22
        if (ix < 0x24000000u) return x * (1.0f + x);            // |x| < 2^-55
        const float ax = u2f(ix);
        if (ix >= 0x3f800000u) {                                // |x| >= 1
            const float t = expm1f(2.0f * ax);
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            const float t = expm1f(-2.0f * ax);
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f - 1.0e-30f;
    }
    return (jx >> 31) ? -z : z;
}

// The reference's logistic, 1 / (1 + expf(-x)) (rwkv7.c).
__host__ __device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
__host__ __device__ __forceinline__ float sigmoid_tab(float x, const uint64_t* tab) {
    return 1.0f / (1.0f + expf_tab(-x, tab));
}

}  // namespace refmath
}  // namespace snhip
