// Sequential sums held across one wave's lanes (rkexact.hip, rkseq.hip).
//
// A sum of n values in element order, s = s + v[0], s = s + v[1], ..., run by
// one thread reading them from LDS, costs a read's issue per four adds. Here
// wave lane j holds values [N j, N (j + 1)) in registers: each lane adds its
// values to the running sum of the lanes before it, which passes from lane j
// to lane j + 1 as a wave-uniform value (readlane). The additions and their
// order are those of the one-thread sum.
#pragma once

#include "common.h"

namespace snhip {

// The sum of the 64 N values (value N j + e in lane j, v[e]); every lane
// returns it. The whole wave must be active.
template <int N>
__device__ __forceinline__ float lane_seq_sum(const float (&v)[N]) {
    float acc = 0.0f;
    for (int j = 0; j < 64; ++j) {
        float a = acc;
#pragma unroll
        for (int e = 0; e < N; ++e) a = a + v[e];
        acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), j));
    }
    return acc;
}

// LayerNorm statistics of n = 64 N values laid out as above: mean = (sum in
// order) / n, then rstd = 1 / sqrt((sum of (v - mean)^2 in order) / n + eps).
// v is overwritten with the squared deviations.
template <int N>
__device__ __forceinline__ void lane_ln_stats(float (&v)[N], int n, float eps, float& mean, float& rstd) {
    mean = lane_seq_sum(v) / (float)n;
#pragma unroll
    for (int e = 0; e < N; ++e) {
        const float d = v[e] - mean;
        v[e] = d * d;
    }
    rstd = 1.0f / sqrtf(lane_seq_sum(v) / (float)n + eps);
}

}  // namespace snhip
