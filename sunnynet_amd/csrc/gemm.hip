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
// Shapes with few tiles split K across blocks; partials are summed in a
// fixed order by a second kernel, so results are deterministic. Products with
// at most 64 rows of X (batched decode) take the skinny path below instead.
#include "gemm.h"

#include <algorithm>
#include <cstdlib>

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

// ---------------------------------------------------------------------------
// Skinny path (M <= 64 rows of X: batched decode).
//
// A workgroup of 4 waves owns a tile of 64 weight rows, all M rows of X and a
// k range [kbeg, kbeg + kc). Its waves take the range's 32-wide k steps round
// robin and load both operands straight from global memory into registers:
// lane (r, h) reads 16 consecutive k, k = kb + 16h + j (j = 0..15), of X rows
// r and 32 + r and of weight rows n0 + r and n0 + 32 + r. MFMA j multiplies
// component j of both operands, so its two k slots are kb + j and kb + 16 + j
// and a step's 16 MFMAs cover its 32 k once. Each wave keeps a 64 x 64 block in
// four 32 x 32 accumulators and prefetches its next step while multiplying.
// The four waves' blocks are summed through LDS in wave order. When the k
// range is split over several workgroups, each stores its block to a partial
// buffer and counts itself in on the tile's counter; the last to arrive sums
// the partials in split order (a fixed order, whatever the arrival order),
// applies the epilogue and re-arms the counter. Partials and counters are
// exchanged with device-coherent stores and loads.
constexpr int SK_W = 4, SK_BN = 64, SK_KS = 32, SK_T = 4096;

typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const f32x4v g_f32x4;
typedef __attribute__((address_space(1))) const u32x4v g_u32x4;
typedef __attribute__((address_space(1))) const float g_f32;

__device__ __forceinline__ float ldc(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stc(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }

struct SkJob {
    GemmArgs g;
    int ntiles, splits, kc;
    float* part;        // splits x ntiles x 4096 floats when splits > 1
    unsigned* cnt;      // ntiles counters
};
struct SkJobs {
    SkJob j[2];
    int blk1;           // first block of job 1
};

// One step's operands of a lane: X rows r, 32 + r and weight rows n0 + r,
// n0 + 32 + r (fp32 values, or INT4 codes and their group scale).
template <int BLK> struct SkFrag;
template <> struct SkFrag<0> { f32x4v a[2][4], b[2][4]; };
template <int BLK> struct SkFrag { f32x4v a[2][4]; u32x4v q[2]; float sc[2]; };

template <int BLK>
__device__ __forceinline__ void sk_load(SkFrag<BLK>& f, const float* xa0, const float* xa1,
                                        const GemmArgs& g, int nb0, int nb1, int kb, int h) {
    // kb: absolute k of the step; xa*: row pointers at k = 16h
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        f.a[0][c] = *(g_f32x4*)(xa0 + kb + 4 * c);
        f.a[1][c] = *(g_f32x4*)(xa1 + kb + 4 * c);
    }
    if constexpr (BLK == 0) {
        const float* w0 = g.w + (long)nb0 * g.K + kb + 16 * h;
        const float* w1 = g.w + (long)nb1 * g.K + kb + 16 * h;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            f.b[0][c] = *(g_f32x4*)(w0 + 4 * c);
            f.b[1][c] = *(g_f32x4*)(w1 + 4 * c);
        }
    } else {
        // Group `kb / BLK`; its byte j holds k = j (low nibble) and
        // j + BLK/2 (high nibble). BLK 32: both lane halves read the group's
        // 16 bytes; BLK 64: half h reads bytes 16h..16h+15.
        const int grp = kb / BLK;
        const long qo = (long)grp * (BLK / 2) + (BLK == 64 ? 16 * h : 0);
        f.q[0] = *(g_u32x4*)(g.q + (long)nb0 * (g.K / 2) + qo);
        f.q[1] = *(g_u32x4*)(g.q + (long)nb1 * (g.K / 2) + qo);
        f.sc[0] = *(g_f32*)(g.sc + (long)nb0 * (g.K / BLK) + grp);
        f.sc[1] = *(g_f32*)(g.sc + (long)nb1 * (g.K / BLK) + grp);
    }
}

template <int BLK>
__device__ __forceinline__ void sk_mma(floatx16 (&acc)[2][2], const SkFrag<BLK>& f, int nshift) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float a0 = f.a[0][j >> 2][j & 3], a1 = f.a[1][j >> 2][j & 3];
        float b0, b1;
        if constexpr (BLK == 0) {
            b0 = f.b[0][j >> 2][j & 3];
            b1 = f.b[1][j >> 2][j & 3];
        } else {
            // (q - 8) * scale: sn_dequant_i4's arithmetic (quant.c:82-83)
            const int sh = 8 * (j & 3) + nshift;
            b0 = (float)((int)((f.q[0][j >> 2] >> sh) & 0xFu) - 8) * f.sc[0];
            b1 = (float)((int)((f.q[1][j >> 2] >> sh) & 0xFu) - 8) * f.sc[1];
        }
        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
}

template <int BLK>
__device__ __forceinline__ void sk_run(const SkJob& J, int local, float* red, int* s_last) {
    const GemmArgs& g = J.g;
    const int tile = local % J.ntiles, z = local / J.ntiles;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, h = lane >> 5;
    const int n0 = tile * SK_BN;
    const int kbeg = z * J.kc;
    const int nst = (min(g.K, kbeg + J.kc) - kbeg) / SK_KS;
    // Rows past M or N read a valid row; their results are never stored.
    const float* xa0 = g.X + (long)min(r, g.M - 1) * g.ldx + 16 * h;
    const float* xa1 = g.X + (long)min(32 + r, g.M - 1) * g.ldx + 16 * h;
    const int nb0 = min(n0 + r, g.N - 1), nb1 = min(n0 + 32 + r, g.N - 1);
    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[0][0][i] = acc[0][1][i] = acc[1][0][i] = acc[1][1][i] = 0.0f;
    // BLK 32: half h takes the low (h = 0) or high nibbles of the same bytes;
    // BLK 64: a step is the low or high half of its group, alike for all lanes.
    auto nshift = [&](int kb) { return BLK == 32 ? 4 * h : (BLK == 64 ? ((kb & 32) >> 3) : 0); };
    if (w < nst) {
        // The next step is always loaded (clamped to the last step, so every
        // iteration issues the same loads) before this step's MFMAs; the
        // scheduling fence keeps those loads ahead of the MFMAs.
        SkFrag<BLK> f0, f1;
        int s = w;
        sk_load<BLK>(f0, xa0, xa1, g, nb0, nb1, kbeg + s * SK_KS, h);
        // Two steps per iteration (fragments f0 then f1), then at most one.
        for (; s + SK_W < nst; s += 2 * SK_W) {
            sk_load<BLK>(f1, xa0, xa1, g, nb0, nb1, kbeg + (s + SK_W) * SK_KS, h);
            __builtin_amdgcn_sched_barrier(0);
            sk_mma<BLK>(acc, f0, nshift(kbeg + s * SK_KS));
            __builtin_amdgcn_sched_barrier(0);
            sk_load<BLK>(f0, xa0, xa1, g, nb0, nb1, kbeg + min(s + 2 * SK_W, nst - 1) * SK_KS, h);
            __builtin_amdgcn_sched_barrier(0);
            sk_mma<BLK>(acc, f1, nshift(kbeg + (s + SK_W) * SK_KS));
            __builtin_amdgcn_sched_barrier(0);
        }
        if (s < nst) sk_mma<BLK>(acc, f0, nshift(kbeg + s * SK_KS));
    }
    // Wave blocks to LDS: accumulator register i of lane (r, h) is row
    // (i / 4) * 8 + h * 4 + i % 4 and column r of its 32 x 32 block.
    float* my = red + w * SK_T;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                my[(mi * 32 + (i >> 2) * 8 + h * 4 + (i & 3)) * 64 + ni * 32 + r] = acc[mi][ni][i];
    __syncthreads();
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int o = e * 256 + tid;
        v[e] = ((red[o] + red[SK_T + o]) + red[2 * SK_T + o]) + red[3 * SK_T + o];
    }
    if (J.splits > 1) {
        float* pp = J.part + ((size_t)z * J.ntiles + tile) * SK_T;
#pragma unroll
        for (int e = 0; e < 16; ++e) stc(pp + e * 256 + tid, v[e]);
        // Every partial store has completed before the tile counter moves.
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const unsigned old = __hip_atomic_fetch_add(J.cnt + tile, 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            *s_last = old + 1 == (unsigned)J.splits;
        }
        __syncthreads();
        if (!*s_last) return;
        // Summed in split order; the loads of four splits (64 values per
        // thread) are in flight together.
        const float* p0 = J.part + (size_t)tile * SK_T + tid;
        const size_t zs = (size_t)J.ntiles * SK_T;
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = ldc(p0 + e * 256);
        int zz = 1;
        for (; zz + 4 <= J.splits; zz += 4) {
            float t[4][16];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 16; ++e) t[q][e] = ldc(p0 + (zz + q) * zs + e * 256);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] += t[q][e];
        }
        for (; zz < J.splits; ++zz) {
            float t[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) t[e] = ldc(p0 + zz * zs + e * 256);
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] += t[e];
        }
        if (tid == 0) __hip_atomic_store(J.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (g.epi == GEPI_COMPETE) {
        // The tile's 64 rows are 4 groups of 8 u rows then 8 g rows: channels
        // tile * 32 .. + 31 (sunnynet.c:252-266, as k_compete_state).
        __syncthreads();
#pragma unroll
        for (int e = 0; e < 16; ++e) red[e * 256 + tid] = v[e];
        __syncthreads();
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int o = e * 256 + tid;
            const int m = o >> 5, cl = o & 31;
            if (m >= g.M) continue;
            const int off = cl & 7;
            const float* qr = red + m * 64 + (cl >> 3) * 16;
            const float gi = qr[8 + off];
            const float uu = qr[off] * (sgm(gi - qr[8 + ((off + 1) & 7)]) *
                                        sgm(gi - qr[8 + ((off + 2) & 7)]));
            const int i = tile * 32 + cl;
            float p = 1.0f - g.delta[i] * (1.0f - sgm(gi));
            if (g.clamp && p < g.p_floor) p = g.p_floor;
            float* sp = const_cast<float*>(g.s) + (long)m * g.lds + i;
            *sp = p * *sp + (1.0f - p) * uu;
            g.Y[(long)m * g.ldy + i] = uu;
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int o = e * 256 + tid;
        const int m = o >> 6, n = n0 + (o & 63);
        if (m < g.M && n < g.N) gemm_epilogue(g, m, n, v[e]);
    }
}

// ---------------------------------------------------------------------------
// Tiny-tile path (M <= 64 with N up to 8192, or M <= 16 with any N; K a multiple of 64 up to 3072: the
// per-layer products of batched decode). A workgroup computes one 16 x 16
// tile of Y (16 rows of X x 16 weight rows) with no exchange between
// workgroups: its nw waves split K into 64-wide chunks (wave w takes chunks
// w, w + nw, ..., NC of them) and issue every operand load of their chunks
// before the first MFMA. v_mfma_f32_16x16x4f32 takes A[l % 16][slot l / 16]
// and B[slot l / 16][l % 16] from lane l; lane (r, q) loads 16 consecutive k,
// k = c + 16q + j, of X row m0 + r and weight row n0 + r, and MFMA j multiplies
// component j of both, so a chunk's 16 MFMAs cover its 64 k once. Lane l,
// result register v holds Y[4 (l / 16) + v][l % 16]. The waves' tiles are
// summed through LDS in wave order before the epilogue. With 16-row tiles a
// decode batch of 64 already gives 128-512 workgroups per product, and a
// tile of U rows is exactly one group of 8 channels (8 u rows, 8 g rows).
constexpr int TT_CH = 64, TT_MAXW = 8;
typedef float f32x4acc __attribute__((ext_vector_type(4)));

struct TtJob {
    GemmArgs g;
    int mb, ntiles;     // 16-row blocks of X, 16-row tiles of W
    int nw;             // waves (chunks = nw * NC)
    int xcd;            // blocks b, b + 8, ... take the mb blocks of one weight tile
};
struct TtJobs {
    TtJob j[2];
    int blk1;
};

template <int BLK> struct TtFrag;
template <> struct TtFrag<0> { f32x4v a[4], b[4]; };
template <int BLK> struct TtFrag { f32x4v a[4]; u32x4v q; float sc; };

template <int BLK>
__device__ __forceinline__ void tt_load(TtFrag<BLK>& f, const float* xr, const GemmArgs& g, int nr,
                                        int c, int q) {
    const int k0 = c + 16 * q;
#pragma unroll
    for (int i = 0; i < 4; ++i) f.a[i] = *(g_f32x4*)(xr + k0 + 4 * i);
    if constexpr (BLK == 0) {
        const float* wr = g.w + (long)nr * g.K + k0;
#pragma unroll
        for (int i = 0; i < 4; ++i) f.b[i] = *(g_f32x4*)(wr + 4 * i);
    } else {
        // BLK 32: k0 opens the low (q even) or high (q odd) half of group
        // k0 / 32, whose 16 bytes hold both. BLK 64: quarter q of group c / 64
        // is the low (q < 2) or high nibbles of bytes 16 (q & 1) ..+15.
        const int grp = k0 / BLK;
        const long qo = (long)grp * (BLK / 2) + (BLK == 64 ? 16 * (q & 1) : 0);
        f.q = *(g_u32x4*)(g.q + (long)nr * (g.K / 2) + qo);
        f.sc = *(g_f32*)(g.sc + (long)nr * (g.K / BLK) + grp);
    }
}

template <int BLK>
__device__ __forceinline__ void tt_mma(f32x4acc (&acc)[4], const TtFrag<BLK>& f, int q) {
    const int nshift = BLK == 32 ? 4 * (q & 1) : (BLK == 64 ? 4 * (q >> 1) : 0);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float a = f.a[j >> 2][j & 3];
        float b;
        if constexpr (BLK == 0) {
            b = f.b[j >> 2][j & 3];
        } else {
            // (q - 8) * scale: sn_dequant_i4's arithmetic (quant.c:82-83)
            b = (float)((int)((f.q[j >> 2] >> (8 * (j & 3) + nshift)) & 0xFu) - 8) * f.sc;
        }
        acc[j & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j & 3], 0, 0, 0);
    }
}

template <int BLK, int NC>
__device__ __forceinline__ void tt_run(const TtJob& J, int local, float* red) {
    const GemmArgs& g = J.g;
    int nt, mbk;
    if (J.xcd) {
        const int x = local & 7, sl = local >> 3;
        nt = (sl / J.mb) * 8 + x;
        mbk = sl - (sl / J.mb) * J.mb;
    } else {
        nt = local / J.mb;
        mbk = local - nt * J.mb;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int m0 = mbk * 16, n0 = nt * 16;
    // Rows past M or N read a valid row; their results are never stored.
    const float* xr = g.X + (long)min(m0 + r, g.M - 1) * g.ldx;
    const int nr = min(n0 + r, g.N - 1);
    TtFrag<BLK> f[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) tt_load<BLK>(f[i], xr, g, nr, (w + i * J.nw) * TT_CH, q);
    __builtin_amdgcn_sched_barrier(0);
    f32x4acc acc[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[a] = f32x4acc{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NC; ++i) tt_mma<BLK>(acc, f[i], q);
    const f32x4acc t = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
    for (int v = 0; v < 4; ++v) red[w * 256 + (4 * q + v) * 16 + r] = t[v];
    __syncthreads();
    // Wave-order sum of the tile into tile[] (256 values, any block size).
    const int nthr = J.nw * 64;
    float* tile = red + TT_MAXW * 256;
    for (int o = tid; o < 256; o += nthr) {
        float sum = red[o];
        for (int ww = 1; ww < J.nw; ++ww) sum += red[ww * 256 + o];
        tile[o] = sum;
    }
    __syncthreads();
    if (g.epi == GEPI_COMPETE) {
        // Tile nt is channel group nt: rows 0-7 u, 8-15 g (sunnynet.c:252-266,
        // as k_compete_state).
        for (int o = tid; o < 128; o += nthr) {
            const int mm = o >> 3, off = o & 7, m = m0 + mm;
            if (m >= g.M) continue;
            const float* qr = tile + mm * 16;
            const float gi = qr[8 + off];
            const float uu = qr[off] * (sgm(gi - qr[8 + ((off + 1) & 7)]) *
                                        sgm(gi - qr[8 + ((off + 2) & 7)]));
            const int i = nt * 8 + off;
            float p = 1.0f - g.delta[i] * (1.0f - sgm(gi));
            if (g.clamp && p < g.p_floor) p = g.p_floor;
            float* sp = const_cast<float*>(g.s) + (long)m * g.lds + i;
            *sp = p * *sp + (1.0f - p) * uu;
            g.Y[(long)m * g.ldy + i] = uu;
        }
        return;
    }
    for (int o = tid; o < 256; o += nthr) {
        const int m = m0 + (o >> 4), n = n0 + (o & 15);
        if (m < g.M && n < g.N) gemm_epilogue(g, m, n, tile[o]);
    }
}

template <int BLK, int NC, int NJ>
__global__ __launch_bounds__(512) void k_gemm_tt(TtJobs J) {
    __shared__ __align__(16) float red[TT_MAXW * 256 + 256];
    const int b = blockIdx.x;
    if (NJ == 2 && b >= J.blk1) tt_run<BLK, NC>(J.j[1], b - J.blk1, red);
    else tt_run<BLK, NC>(J.j[0], b, red);
}

template <int BLK, int NJ>
__global__ __launch_bounds__(256) void k_gemm_sk(SkJobs J) {
    __shared__ __align__(16) float red[SK_W * SK_T];
    __shared__ int s_last;
    const int b = blockIdx.x;
    if (NJ == 2 && b >= J.blk1) sk_run<BLK>(J.j[1], b - J.blk1, red, &s_last);
    else sk_run<BLK>(J.j[0], b, red, &s_last);
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
    // Fewer than ~4 tiles per CU leaves the LDS pipeline of each workgroup
    // exposed: split K so that about 1024 workgroups run (at least 4 k-tiles
    // each), within the partial buffer.
    int splits = 1;
    if (work && gx * gy < 1024) {
        splits = (1024 + gx * gy - 1) / (gx * gy);
        splits = std::min(splits, std::max(1, ktiles / 4));
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

namespace {

// Split plan of one skinny product: ntiles tiles of 64 weight rows, k range
// per workgroup kc (a multiple of 32), splits workgroups per tile. Aims for
// about `target` workgroups (one per CU by default) with at least SK_W steps
// per workgroup, within the partial buffer and counters given.
struct SkPlan { int ntiles, splits, kc; size_t part_floats; };

int sk_target() {
    static int t = [] {
        const char* e = getenv("SNHIP_GEMM_SK_WG");
        const int v = e ? atoi(e) : 0;
        return v > 0 ? v : 256;
    }();
    return t;
}

SkPlan sk_plan(const GemmArgs& g, size_t part_avail, int cnt_avail) {
    SkPlan p{};
    p.ntiles = (g.N + SK_BN - 1) / SK_BN;
    const int ksteps = g.K / SK_KS;
    int splits = (sk_target() + p.ntiles - 1) / p.ntiles;
    splits = std::max(1, std::min(splits, ksteps / SK_W));
    for (;;) {
        const int per = (ksteps + splits - 1) / splits;
        p.kc = per * SK_KS;
        p.splits = (ksteps + per - 1) / per;
        p.part_floats = p.splits > 1 ? (size_t)p.splits * p.ntiles * SK_T : 0;
        if (p.splits == 1 || (p.part_floats <= part_avail && p.ntiles <= cnt_avail)) break;
        --splits;
    }
    return p;
}

SkJob sk_job(const GemmArgs& g, const SkPlan& p, float* part, unsigned* cnt) {
    SkJob j{};
    j.g = g;
    j.ntiles = p.ntiles; j.splits = p.splits; j.kc = p.kc;
    j.part = part; j.cnt = cnt;
    return j;
}

int sk_block(const GemmArgs& g) { return g.q ? g.block : 0; }

snhip_status sk_launch(const SkJobs& J, int nj, int blocks, int blk, hipStream_t st) {
#define SNHIP_SK(B, N) hipLaunchKernelGGL((k_gemm_sk<B, N>), dim3(blocks), dim3(256), 0, st, J)
    if (nj == 1) {
        if (blk == 0) SNHIP_SK(0, 1); else if (blk == 32) SNHIP_SK(32, 1); else SNHIP_SK(64, 1);
    } else {
        if (blk == 0) SNHIP_SK(0, 2); else if (blk == 32) SNHIP_SK(32, 2); else SNHIP_SK(64, 2);
    }
#undef SNHIP_SK
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// Tiny-tile plan: chunks = K / 64 split as nw waves x nc chunks (nw <= 8,
// nc one of the compiled counts).
struct TtPlan { bool ok; int mb, ntiles, nw, nc, xcd; };

TtPlan tt_plan(const GemmArgs& g) {
    TtPlan p{};
    // Wide products (the LM head) take this path only for up to 16 rows of X
    // (one row block, no padding to 64 rows); measured at vocab 32000:
    // INT4 B=8 head step 424 -> 405 us, but fp32 B=64 603 -> 661 us and
    // INT4 B=32 (two row blocks) 428 -> 433 us.
    if (g.M > 64 || g.shift_T != 0 || g.K % TT_CH || (g.N > 8192 && g.M > 16)) return p;
    const int nch = g.K / TT_CH;
    for (int nc : {1, 2, 3, 4, 6}) {
        if (nch % nc == 0 && nch / nc <= TT_MAXW) {
            p.ok = true;
            p.nc = nc;
            p.nw = nch / nc;
            break;
        }
    }
    p.mb = (g.M + 15) / 16;
    p.ntiles = (g.N + 15) / 16;
    p.xcd = p.mb > 1 && p.ntiles % 8 == 0;
    return p;
}

TtJob tt_job(const GemmArgs& g, const TtPlan& p) {
    TtJob j{};
    j.g = g;
    j.mb = p.mb; j.ntiles = p.ntiles; j.nw = p.nw; j.xcd = p.xcd;
    return j;
}

template <int BLK, int NJ>
void tt_launch_nc(const TtJobs& J, int blocks, int nc, int nw, hipStream_t st) {
    const dim3 grid(blocks), blk(64 * nw);
    switch (nc) {
    case 1: hipLaunchKernelGGL((k_gemm_tt<BLK, 1, NJ>), grid, blk, 0, st, J); break;
    case 2: hipLaunchKernelGGL((k_gemm_tt<BLK, 2, NJ>), grid, blk, 0, st, J); break;
    case 3: hipLaunchKernelGGL((k_gemm_tt<BLK, 3, NJ>), grid, blk, 0, st, J); break;
    case 4: hipLaunchKernelGGL((k_gemm_tt<BLK, 4, NJ>), grid, blk, 0, st, J); break;
    default: hipLaunchKernelGGL((k_gemm_tt<BLK, 6, NJ>), grid, blk, 0, st, J); break;
    }
}

snhip_status tt_launch(const TtJobs& J, int nj, int blocks, int blk, int nc, int nw,
                       hipStream_t st) {
    if (nj == 1) {
        if (blk == 0) tt_launch_nc<0, 1>(J, blocks, nc, nw, st);
        else if (blk == 32) tt_launch_nc<32, 1>(J, blocks, nc, nw, st);
        else tt_launch_nc<64, 1>(J, blocks, nc, nw, st);
    } else {
        if (blk == 0) tt_launch_nc<0, 2>(J, blocks, nc, nw, st);
        else if (blk == 32) tt_launch_nc<32, 2>(J, blocks, nc, nw, st);
        else tt_launch_nc<64, 2>(J, blocks, nc, nw, st);
    }
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

snhip_status check_args(const GemmArgs& g) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.K % BK) {
        set_last_error("gemm: K must be a positive multiple of 32");
        return SNHIP_E_INVAL;
    }
    if (g.q && g.block != 32 && g.block != 64) {
        set_last_error("gemm: INT4 block must be 32 or 64");
        return SNHIP_E_INVAL;
    }
    return SNHIP_OK;
}

}  // namespace

bool gemm_skinny(const GemmArgs& g, const GemmWork& w) {
    return g.M <= 64 && g.shift_T == 0 && w.cnt != nullptr && g.K % SK_KS == 0;
}

bool gemm_fuses_compete(const GemmArgs& g, const GemmWork& w) {
    const TtPlan tp = tt_plan(g);
    if (tp.ok) return g.N % 16 == 0;
    return gemm_skinny(g, w) && g.N % SK_BN == 0;
}

snhip_status launch_gemm(const GemmArgs& g, const GemmWork& w, hipStream_t st) {
    snhip_status rc = check_args(g);
    if (rc != SNHIP_OK) return rc;
    if (g.epi == GEPI_COMPETE && !gemm_fuses_compete(g, w)) {
        set_last_error("gemm: the gate epilogue needs the tiny-tile or skinny path");
        return SNHIP_E_UNSUPPORTED;
    }
    const TtPlan tp = tt_plan(g);
    if (tp.ok) {
        TtJobs J{};
        J.j[0] = tt_job(g, tp);
        J.blk1 = tp.mb * tp.ntiles;
        return tt_launch(J, 1, J.blk1, sk_block(g), tp.nc, tp.nw, st);
    }
    if (!gemm_skinny(g, w)) return launch_gemm(g, w.part, w.part_floats, st);
    const SkPlan p = sk_plan(g, w.part_floats, w.ncnt);
    SkJobs J{};
    J.j[0] = sk_job(g, p, w.part, w.cnt);
    J.blk1 = p.ntiles * p.splits;
    return sk_launch(J, 1, J.blk1, sk_block(g), st);
}

snhip_status launch_gemm2(const GemmArgs& a, const GemmArgs& b, const GemmWork& w,
                          hipStream_t st) {
    snhip_status rc;
    if ((rc = check_args(a)) != SNHIP_OK || (rc = check_args(b)) != SNHIP_OK) return rc;
    const bool plain = a.epi != GEPI_COMPETE && b.epi != GEPI_COMPETE && sk_block(a) == sk_block(b);
    const TtPlan ta = tt_plan(a), tb = tt_plan(b);
    if (plain && ta.ok && tb.ok && ta.nc == tb.nc && ta.nw == tb.nw) {
        TtJobs J{};
        J.j[0] = tt_job(a, ta);
        J.j[1] = tt_job(b, tb);
        J.blk1 = ta.mb * ta.ntiles;
        return tt_launch(J, 2, J.blk1 + tb.mb * tb.ntiles, sk_block(a), ta.nc, ta.nw, st);
    }
    if (!plain || ta.ok || tb.ok || !gemm_skinny(a, w) || !gemm_skinny(b, w)) {
        if ((rc = launch_gemm(a, w, st)) != SNHIP_OK) return rc;
        return launch_gemm(b, w, st);
    }
    // Job 0 takes the front of the scratch, job 1 the rest.
    const SkPlan pa = sk_plan(a, w.part_floats / 2, w.ncnt / 2);
    const SkPlan pb = sk_plan(b, w.part_floats / 2, w.ncnt / 2);
    SkJobs J{};
    J.j[0] = sk_job(a, pa, w.part, w.cnt);
    J.j[1] = sk_job(b, pb, w.part + w.part_floats / 2, w.cnt + w.ncnt / 2);
    J.blk1 = pa.ntiles * pa.splits;
    return sk_launch(J, 2, J.blk1 + pb.ntiles * pb.splits, sk_block(a), st);
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
