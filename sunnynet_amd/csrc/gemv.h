// Batched matrix-vector products for decode (gemv.hip), shared by the
// SunnyNet and RWKV-7 handles.
#pragma once

#include "common.h"

namespace snhip {

// Epilogue of a row's dot product acc (y = the output element).
enum GemvEpi {
    EPI_STORE = 0,    // y = acc
    EPI_WEDGE = 1,    // y = acc (1 + a/2 / (1 + |acc|))            (sunnynet.c:270-271)
    EPI_RESID = 2,    // y = acc + (b s + sfb + y)                   (sunnynet.c:276)
    EPI_ARGMAX = 3,   // y = acc, and per-block argmax keys into best
    EPI_ADD = 4,      // y = y + acc                                 (rwkv7.c:300,314)
    EPI_RELU2 = 5,    // y = max(acc, 0)^2                           (rwkv7.c:308-312)
};

// Y[b, m] = sum_k W[m, k] X[b, k] for sequences b < B; W row-major
// (M, Kd): fp32 rows in w, or INT4 codes in q ((M, Kd/2) bytes, quant.c
// packing) with scales sc ((M, Kd/block)).
struct GemvJob {
    const float* w;
    const uint8_t* q;
    const float* sc;
    int M, Kd, B;
    const float* X; int ldx;
    float* Y; int ldy;
    int epi;
    float a_tanh, b_gain;
    const float* s; int lds;
    const float* sfb; int ldf;
    unsigned long long* best;   // EPI_ARGMAX: per-block packed maxima, [b * nblk + blk]
    int nblk;                   // set by launch_gemv
    int xact;                   // activation applied to X as it is staged (GemvAct)
};

// Elementwise activation of a job's input vector, applied while staging it.
enum GemvAct {
    ACT_NONE = 0,
    ACT_TANH = 1,      // tanhf(x)                       (rwkv7.c:235)
    ACT_SIGMOID = 2,   // 1 / (1 + expf(-x))             (rwkv7.c:256)
};

constexpr int kGemvMaxJobs = 8;

// Orderable key of (value, index): larger value wins, then smaller index,
// so the maximum key is torch.argmax's first maximal index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}

// Workgroups a job takes (its argmax partial count).
int gemv_blocks(const GemvJob& j, int block);
// Up to kGemvMaxJobs independent jobs in one launch, all fp32 (block = 0) or
// all INT4 with group size block (32 or 64). Sets each job's nblk.
hipError_t launch_gemv(GemvJob* jobs, int n, int block, hipStream_t st);

}  // namespace snhip
