// FP32 MFMA GEMM for gfx950 (see gemm.h).
//
// Tile 64 (rows of X) x 64 (rows of W) x 32 (k), 4 waves in a 2 x 2 layout,
// each wave owning one 32 x 32 block of v_mfma_f32_32x32x2f32 accumulators
// (16 VGPRs per lane). Per 32-wide k tile, X and W are staged in LDS (rows
// padded to 36 floats so the 16-byte fragment reads of 8 consecutive rows
// touch distinct banks). The MFMA's two k-slots are fed from one 16-byte LDS
// read per operand: within each group of 8 k values, lanes 0-31 supply
// k = 0..3 and lanes 32-63 k = 4..7, one value per MFMA, so four MFMAs cover
// the 8 values. Both operands use the same permutation, so every product
// X[m,k] W[n,k] is summed exactly once.
//
// INT4 weights are dequantized while staging the W tile: (q - 8) * scale,
// the bit-identical form of sn_dequant_i4 (quant.c:82-83).
//
// Skinny shapes (few tiles, e.g. decode with 64 sequences) split K across
// blocks; partials are summed in a fixed order by a second kernel, so
// results are deterministic.
#include "gemm.h"

namespace snhip {
namespace {

constexpr int BM = 64, BN = 64, BK = 32, LDSK = BK + 4;
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ const float* xrow(const GemmArgs& g, int m) {
    if (g.shift_T > 0) {
        const int t = m % g.shift_T;
        return t == 0 ? g.X0 + (long)(m / g.shift_T) * g.ldx0 : g.X + (long)(m - 1) * g.ldx;
    }
    return g.X + (long)m * g.ldx;
}

__device__ __forceinline__ void gemm_epilogue(const GemmArgs& g, int m, int n, float acc) {
    float* y = g.Y + (long)m * g.ldy + n;
    if (g.epi == GEPI_STORE) {
        *y = acc;
    } else if (g.epi == GEPI_WEDGE) {
        *y = acc * (1.0f + 0.5f * g.a_tanh / (1.0f + fabsf(acc)));       // sunnynet.c:270-271
    } else if (g.epi == GEPI_RESID) {
        *y = acc + (g.b_gain * g.s[(long)m * g.lds + n] + g.sfb[(long)m * g.ldf + n] + *y);  // :276
    } else if (g.epi == GEPI_ADD) {
        *y = *y + acc;                                                    // rwkv7.c:300,314
    } else {
        const float t = acc > 0.0f ? acc : 0.0f;                          // rwkv7.c:308-312
        *y = t * t;
    }
}

template <int BLK>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g, int kchunk, float* __restrict__ part) {
    __shared__ __align__(16) float As[BM * LDSK];
    __shared__ __align__(16) float Bs[BN * LDSK];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w >> 1, wn = w & 1;
    const int r = lane & 31, h = lane >> 5;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kbeg = blockIdx.z * kchunk;
    const int kend = min(g.K, kbeg + kchunk);
    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

    for (int kt = kbeg; kt < kend; kt += BK) {
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            const int row = (tid >> 3) + 32 * pass, c4 = tid & 7;
            const int m = m0 + row;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < g.M) v = *reinterpret_cast<const float4*>(xrow(g, m) + kt + 4 * c4);
            *reinterpret_cast<float4*>(As + row * LDSK + 4 * c4) = v;
        }
        if constexpr (BLK == 0) {
#pragma unroll
            for (int pass = 0; pass < 2; ++pass) {
                const int row = (tid >> 3) + 32 * pass, c4 = tid & 7;
                const int n = n0 + row;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (n < g.N) v = *reinterpret_cast<const float4*>(g.w + (long)n * g.K + kt + 4 * c4);
                *reinterpret_cast<float4*>(Bs + row * LDSK + 4 * c4) = v;
            }
        } else {
            if (tid < BN) {
                const int n = n0 + tid;
                float vals[BK];
#pragma unroll
                for (int j = 0; j < BK; ++j) vals[j] = 0.0f;
                if (n < g.N) {
                    const int grp = kt / BLK;
                    const float sc = g.sc[(long)n * (g.K / BLK) + grp];
                    const uint8_t* qb = g.q + (long)n * (g.K / 2) + (long)grp * (BLK / 2);
                    if constexpr (BLK == 32) {
                        const uint4 qq = *reinterpret_cast<const uint4*>(qb);
                        const uint32_t wd[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
                        for (int j = 0; j < 16; ++j) {
                            const uint32_t byte = (wd[j >> 2] >> ((j & 3) * 8)) & 0xFFu;
                            vals[j] = (float)((int)(byte & 0x0Fu) - 8) * sc;
                            vals[16 + j] = (float)((int)(byte >> 4) - 8) * sc;
                        }
                    } else {
                        // BLK = 64: this k tile is the low (elements 0-31) or
                        // high (32-63) nibbles of the group's 32 bytes.
                        const bool high = (kt % BLK) != 0;
                        const uint4 q0 = *reinterpret_cast<const uint4*>(qb);
                        const uint4 q1 = *reinterpret_cast<const uint4*>(qb + 16);
                        const uint32_t wd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
                        for (int j = 0; j < 32; ++j) {
                            const uint32_t byte = (wd[j >> 2] >> ((j & 3) * 8)) & 0xFFu;
                            const uint32_t nib = high ? (byte >> 4) : (byte & 0x0Fu);
                            vals[j] = (float)((int)nib - 8) * sc;
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < BK; j += 4)
                    *reinterpret_cast<float4*>(Bs + tid * LDSK + j) =
                        make_float4(vals[j], vals[j + 1], vals[j + 2], vals[j + 3]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < BK / 8; ++q) {
            const float4 a4 = *reinterpret_cast<const float4*>(As + (wm * 32 + r) * LDSK + 8 * q + 4 * h);
            const float4 b4 = *reinterpret_cast<const float4*>(Bs + (wn * 32 + r) * LDSK + 8 * q + 4 * h);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.x, b4.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.y, b4.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.z, b4.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.w, b4.w, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    // D[i][j]: lane holds column j = lane % 32; register i covers row
    // (i / 4) * 8 + (lane / 32) * 4 + i % 4 of the wave's 32 x 32 block.
    const int n = n0 + wn * 32 + r;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = m0 + wm * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
        if (m < g.M && n < g.N) {
            if (part) part[((long)blockIdx.z * g.M + m) * g.N + n] = acc[i];
            else gemm_epilogue(g, m, n, acc[i]);
        }
    }
}

// Sum split-K partials in split order, then apply the epilogue.
__global__ void k_gemm_reduce(GemmArgs g, int splits, const float* __restrict__ part) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long MN = (long)g.M * g.N;
    if (idx >= MN) return;
    // Loads issued ahead of the (in-order) sum, four splits at a time.
    float acc = part[idx];
    int z = 1;
    for (; z + 4 <= splits; z += 4) {
        const float p0 = part[(long)z * MN + idx], p1 = part[(long)(z + 1) * MN + idx];
        const float p2 = part[(long)(z + 2) * MN + idx], p3 = part[(long)(z + 3) * MN + idx];
        acc += p0; acc += p1; acc += p2; acc += p3;
    }
    for (; z < splits; ++z) acc += part[(long)z * MN + idx];
    gemm_epilogue(g, (int)(idx / g.N), (int)(idx % g.N), acc);
}

}  // namespace

snhip_status launch_gemm(const GemmArgs& g, float* work, size_t work_floats, hipStream_t st) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.K % BK) {
        set_last_error("gemm: K must be a positive multiple of 32");
        return SNHIP_E_INVAL;
    }
    if (g.q && g.block != 32 && g.block != 64) {
        set_last_error("gemm: INT4 block must be 32 or 64");
        return SNHIP_E_INVAL;
    }
    const int gx = (g.N + BN - 1) / BN, gy = (g.M + BM - 1) / BM;
    const int ktiles = g.K / BK;
    int splits = 1;
    if (work && gx * gy < 192) {
        splits = (384 + gx * gy - 1) / (gx * gy);
        splits = std::min(splits, std::max(1, ktiles / 2));
        while (splits > 1 && (size_t)splits * g.M * g.N > work_floats) --splits;
    }
    const int kchunk = ((ktiles + splits - 1) / splits) * BK;
    splits = (g.K + kchunk - 1) / kchunk;
    float* part = splits > 1 ? work : nullptr;
    const dim3 grid(gx, gy, splits);
    if (!g.q)
        hipLaunchKernelGGL(k_gemm<0>, grid, dim3(256), 0, st, g, kchunk, part);
    else if (g.block == 32)
        hipLaunchKernelGGL(k_gemm<32>, grid, dim3(256), 0, st, g, kchunk, part);
    else
        hipLaunchKernelGGL(k_gemm<64>, grid, dim3(256), 0, st, g, kchunk, part);
    SNHIP_CHECK(hipGetLastError());
    if (part) {
        const long MN = (long)g.M * g.N;
        hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, st, g,
                           splits, part);
        SNHIP_CHECK(hipGetLastError());
    }
    return SNHIP_OK;
}

}  // namespace snhip

extern "C" snhip_status snhip_abi_linear_dev(const float* x, const float* w, float* y, int32_t M,
                                             int32_t N, int32_t K, void* stream) {
    if (!x || !w || !y || M <= 0 || N <= 0 || K <= 0) return SNHIP_E_INVAL;
    if (K % 32 || ((uintptr_t)x | (uintptr_t)w) % 16) return SNHIP_E_UNSUPPORTED;
    snhip::GemmArgs g{};
    g.X = x; g.ldx = K;
    g.w = w;
    g.M = M; g.N = N; g.K = K;
    g.Y = y; g.ldy = N;
    g.epi = snhip::GEPI_STORE;
    return snhip::launch_gemm(g, nullptr, 0, snhip::as_stream(stream));
}
