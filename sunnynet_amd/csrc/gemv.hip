// Batched GEMV for decode (gemv.h).
//
// Each wave streams whole weight rows; X is staged in LDS in chunks of BT
// sequences. fp32: a lane holds float4 columns k = 4 lane + 256 i, two rows
// in flight per wave. INT4: X is transposed inside each group in LDS
// (xs[j * ngroups + g] = x[g * BLK + j]) so lanes reading the same in-group
// position of different groups hit different banks; 64 / ngroups rows per
// wave pass when the group count divides 64. Dequantization is quant.c's
// (q - 8) * scale, bit-identical to sn_dequant_i4. Reductions are
// wave-parallel, so sums agree with the sequential reference to float
// rounding, not bit for bit.
#include "gemv.h"

namespace snhip {
namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const f32x4v g_f32x4;
typedef __attribute__((address_space(1))) const u32x4v g_u32x4;
__device__ __forceinline__ float4 ldg4(const float* p) {
    const f32x4v v = *(g_f32x4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldgq(const uint8_t* p) {
    const u32x4v v = *(g_u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

struct GemvJobs {
    GemvJob j[kGemvMaxJobs];
    int n;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float seg_sum(float v, int seg) {
    for (int o = seg >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ void epilogue(const GemvJob& J, int b, int m, float acc) {
    float* y = J.Y + (size_t)b * J.ldy + m;
    switch (J.epi) {
        case EPI_WEDGE:
            *y = acc * (1.0f + 0.5f * J.a_tanh / (1.0f + fabsf(acc)));
            break;
        case EPI_RESID:
            *y = acc + (J.b_gain * J.s[(size_t)b * J.lds + m] + J.sfb[(size_t)b * J.ldf + m] + *y);
            break;
        case EPI_ADD:
            *y = *y + acc;
            break;
        case EPI_RELU2: {
            const float t = acc > 0.0f ? acc : 0.0f;
            *y = t * t;
            break;
        }
        default:   // EPI_STORE, EPI_ARGMAX (the maximum is reduced by k_gemv)
            *y = acc;
    }
}

template <int BLK, int BT>
__global__ __launch_bounds__(256) void k_gemv(GemvJobs JS) {
    extern __shared__ float xs[];
    int ji = 0, blk = blockIdx.x;
    while (ji + 1 < JS.n && blk >= JS.j[ji].nblk) {
        blk -= JS.j[ji].nblk;
        ++ji;
    }
    const GemvJob& J = JS.j[ji];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int M = J.M, Kd = J.Kd, B = J.B;
    const int nw = J.nblk * 4;
    const int gw = blk * 4 + wv;

    const bool amax = J.epi == EPI_ARGMAX;
    __shared__ unsigned long long kbest[4][BT];
    for (int b0 = 0; b0 < B; b0 += BT) {
        const int nb = min(BT, B - b0);
        unsigned long long best[BT];
#pragma unroll
        for (int bb = 0; bb < BT; ++bb) best[bb] = 0ull;
        __syncthreads();
        const int xact = J.xact;
        auto xval = [&](float v) {
            return xact == ACT_TANH ? tanhf(v) : xact == ACT_SIGMOID ? 1.0f / (1.0f + expf(-v)) : v;
        };
        if constexpr (BLK == 0) {
            for (int i = threadIdx.x; i < nb * Kd; i += 256) {
                const int bb = i / Kd, k = i - bb * Kd;
                xs[i] = xval(J.X[(size_t)(b0 + bb) * J.ldx + k]);
            }
        } else {
            const int ng = Kd / BLK;
            for (int i = threadIdx.x; i < nb * Kd; i += 256) {
                const int bb = i / Kd, k = i - bb * Kd;
                const int g = k / BLK, j = k - g * BLK;
                xs[bb * Kd + j * ng + g] = xval(J.X[(size_t)(b0 + bb) * J.ldx + k]);
            }
        }
        __syncthreads();

        if constexpr (BLK == 0) {
            for (int r = gw * 2; r < M; r += nw * 2) {
                const bool two = r + 1 < M;
                const float* w0 = J.w + (size_t)r * Kd;
                const float* w1 = two ? w0 + Kd : w0;
                float a0[BT], a1[BT];
#pragma unroll
                for (int bb = 0; bb < BT; ++bb) { a0[bb] = 0.0f; a1[bb] = 0.0f; }
                for (int k = lane * 4; k < Kd; k += 256) {
                    const float4 x0 = ldg4(w0 + k);
                    const float4 x1 = ldg4(w1 + k);
#pragma unroll
                    for (int bb = 0; bb < BT; ++bb) {
                        if (bb < nb) {
                            const float4 xv = *reinterpret_cast<const float4*>(xs + bb * Kd + k);
                            a0[bb] = fmaf(x0.x, xv.x, a0[bb]); a0[bb] = fmaf(x0.y, xv.y, a0[bb]);
                            a0[bb] = fmaf(x0.z, xv.z, a0[bb]); a0[bb] = fmaf(x0.w, xv.w, a0[bb]);
                            a1[bb] = fmaf(x1.x, xv.x, a1[bb]); a1[bb] = fmaf(x1.y, xv.y, a1[bb]);
                            a1[bb] = fmaf(x1.z, xv.z, a1[bb]); a1[bb] = fmaf(x1.w, xv.w, a1[bb]);
                        }
                    }
                }
#pragma unroll
                for (int bb = 0; bb < BT; ++bb) {
                    if (bb < nb) {
                        const float s0 = wave_sum(a0[bb]);
                        const float s1 = wave_sum(a1[bb]);
                        if (lane == 0) {
                            epilogue(J, b0 + bb, r, s0);
                            if (two) epilogue(J, b0 + bb, r + 1, s1);
                        }
                        if (amax) {
                            unsigned long long k = argmax_key(s0, r);
                            if (two) k = max(k, argmax_key(s1, r + 1));
                            best[bb] = max(best[bb], k);
                        }
                    }
                }
            }
        } else {
            constexpr int HB = BLK / 2;              // bytes per group
            const int ng = Kd / BLK;
            const int seg = (ng < 64 && (64 % ng) == 0) ? ng : 64;
            const int rpi = 64 / seg;                // rows per wave pass
            const int lrow = lane / seg, lg = lane - lrow * seg;
            for (int r0 = gw * rpi; r0 < M; r0 += nw * rpi) {
                const int r = r0 + lrow;
                const bool live = r < M;
                float acc[BT];
#pragma unroll
                for (int bb = 0; bb < BT; ++bb) acc[bb] = 0.0f;
                if (live) {
                    const uint8_t* qr = J.q + (size_t)r * (Kd / 2);
                    const float* sr = J.sc + (size_t)r * ng;
                    for (int g = lg; g < ng; g += seg) {
                        uint4 qv[HB / 16];
#pragma unroll
                        for (int h = 0; h < HB / 16; ++h) qv[h] = ldgq(qr + (size_t)g * HB + h * 16);
                        const float sc = sr[g];
#pragma unroll
                        for (int j = 0; j < HB; ++j) {
                            const uint4& qq = qv[j >> 4];
                            const int wi = (j >> 2) & 3;
                            const uint32_t word = wi == 0 ? qq.x : wi == 1 ? qq.y : wi == 2 ? qq.z : qq.w;
                            const uint32_t byte = (word >> ((j & 3) * 8)) & 0xFFu;
                            // quant.c:82-83, bit-identical dequantization
                            const float wl = (float)((int)(byte & 0x0Fu) - 8) * sc;
                            const float wh = (float)((int)(byte >> 4) - 8) * sc;
#pragma unroll
                            for (int bb = 0; bb < BT; ++bb) {
                                if (bb < nb) {
                                    const float* xb = xs + bb * Kd;
                                    acc[bb] = fmaf(wl, xb[j * ng + g], acc[bb]);
                                    acc[bb] = fmaf(wh, xb[(j + HB) * ng + g], acc[bb]);
                                }
                            }
                        }
                    }
                }
#pragma unroll
                for (int bb = 0; bb < BT; ++bb) {
                    if (bb < nb) {
                        const float t = seg_sum(acc[bb], seg);
                        if (live && lg == 0) epilogue(J, b0 + bb, r, t);
                        if (amax && live && lg == 0) best[bb] = max(best[bb], argmax_key(t, r));
                    }
                }
            }
        }
        if (amax) {
            // Per-wave maximum (int4 keeps one candidate per row segment),
            // then per block; one plain store per (sequence, block).
#pragma unroll
            for (int bb = 0; bb < BT; ++bb) {
                unsigned long long k = best[bb];
                for (int o = 32; o > 0; o >>= 1) {
                    const unsigned long long other =
                        ((unsigned long long)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
                        (uint32_t)__shfl_xor((int)(k & 0xFFFFFFFFull), o, 64);
                    k = max(k, other);
                }
                if (lane == 0) kbest[wv][bb] = k;
            }
            __syncthreads();
            if (threadIdx.x < (unsigned)nb) {
                const int bb = threadIdx.x;
                const unsigned long long k = max(max(kbest[0][bb], kbest[1][bb]),
                                                 max(kbest[2][bb], kbest[3][bb]));
                J.best[(size_t)(b0 + bb) * J.nblk + blk] = k;
            }
        }
    }
}

template <int BLK>
hipError_t launch_fmt(const GemvJobs& js, int nblk, int kd, int bt, hipStream_t st) {
    const dim3 grid(nblk), blk(256);
    if (bt == 1)
        hipLaunchKernelGGL((k_gemv<BLK, 1>), grid, blk, (size_t)kd * 4, st, js);
    else
        hipLaunchKernelGGL((k_gemv<BLK, 8>), grid, blk, (size_t)kd * 4 * 8, st, js);
    return hipGetLastError();
}

}  // namespace

int gemv_blocks(const GemvJob& j, int block) {
    int rows_per_wave = 2;
    if (j.q) {
        const int ng = j.Kd / block;
        rows_per_wave = (ng < 64 && 64 % ng == 0) ? 64 / ng : 1;
    }
    const int rows_per_block = 4 * rows_per_wave;
    const int nb = (j.M + rows_per_block - 1) / rows_per_block;
    return nb > 4096 ? 4096 : nb;
}

hipError_t launch_gemv(GemvJob* jobs, int n, int block, hipStream_t st) {
    if (n < 1 || n > kGemvMaxJobs) return hipErrorInvalidValue;
    GemvJobs js{};
    int total = 0, kd = 0, B = 0;
    for (int i = 0; i < n; ++i) {
        jobs[i].nblk = gemv_blocks(jobs[i], block);
        js.j[i] = jobs[i];
        total += jobs[i].nblk;
        kd = std::max(kd, jobs[i].Kd);
        B = std::max(B, jobs[i].B);
    }
    js.n = n;
    const int bt = (B > 1 && (size_t)kd * 4 * 8 <= 65536) ? 8 : 1;
    if (!jobs[0].q) return launch_fmt<0>(js, total, kd, bt, st);
    if (block == 32) return launch_fmt<32>(js, total, kd, bt, st);
    return launch_fmt<64>(js, total, kd, bt, st);
}

}  // namespace snhip
