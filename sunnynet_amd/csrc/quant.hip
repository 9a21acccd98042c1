// Group-wise symmetric INT4 quantization in the reference's format
// (sunnynet/runtime/quant.c:34-87). One thread per (row, group): scale =
// amax / 7 (1 when amax == 0), q = clamp(rint(w * (1/scale)), -8, 7) + 8,
// byte k = q[k] | q[k + block/2] << 4. Every operation is a single correctly
// rounded IEEE op, so the output is bit-identical to the reference.
#include "common.h"

namespace snhip {

__global__ void k_quant_i4(const float* __restrict__ x, uint8_t* __restrict__ q,
                           float* __restrict__ scale, int rows, int N, int block) {
    const int nb = N / block, half = block / 2;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)rows * nb) return;
    const long r = gid / nb;
    const int g = (int)(gid - r * nb);
    const float* xr = x + (size_t)r * N + (size_t)g * block;
    float amax = 0.0f;
    for (int i = 0; i < block; ++i) amax = fmaxf(amax, fabsf(xr[i]));
    const float sc = amax > 0.0f ? __fdiv_rn(amax, 7.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, sc);
    scale[(size_t)r * nb + g] = sc;
    uint8_t* qb = q + (size_t)r * (N / 2) + (size_t)g * half;
    for (int k = 0; k < half; ++k) {
        int lo = (int)rintf(__fmul_rn(xr[k], inv));
        int hi = (int)rintf(__fmul_rn(xr[half + k], inv));
        lo = lo < -8 ? -8 : (lo > 7 ? 7 : lo);
        hi = hi < -8 ? -8 : (hi > 7 ? 7 : hi);
        qb[k] = (uint8_t)((lo + 8) | ((hi + 8) << 4));
    }
}

__global__ void k_dequant_i4(const uint8_t* __restrict__ q, const float* __restrict__ scale,
                             float* __restrict__ x, int rows, int N, int block) {
    const int half = block / 2, nb = N / block;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;   // byte index
    if (i >= (long)rows * (N / 2)) return;
    const long r = i / (N / 2);
    const int kb = (int)(i - r * (N / 2));
    const int g = kb / half, k = kb - g * half;
    const uint8_t byte = q[i];
    const float sc = scale[(size_t)r * nb + g];
    float* xr = x + (size_t)r * N + (size_t)g * block;
    xr[k] = __fmul_rn((float)((int)(byte & 0x0F) - 8), sc);
    xr[half + k] = __fmul_rn((float)((int)(byte >> 4) - 8), sc);
}

snhip_status launch_quant_i4(const float* x, uint8_t* q, float* scale, int rows, int N,
                             int block, hipStream_t st) {
    const long groups = (long)rows * (N / block);
    if (groups == 0) return SNHIP_OK;
    hipLaunchKernelGGL(k_quant_i4, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st,
                       x, q, scale, rows, N, block);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

snhip_status launch_dequant_i4(const uint8_t* q, const float* scale, float* x, int rows, int N,
                               int block, hipStream_t st) {
    const long bytes = (long)rows * (N / 2);
    if (bytes == 0) return SNHIP_OK;
    hipLaunchKernelGGL(k_dequant_i4, dim3((unsigned)((bytes + 255) / 256)), dim3(256), 0, st,
                       q, scale, x, rows, N, block);
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

}  // namespace snhip
