/* SunnyNet HIP backend: stable C ABI.
 *
 * Mirrors the reference's stable ABI, sunnynet/runtime/sn_abi.h:24-100 and
 * docs/ABI.md, under the prefix snhip_abi_ so both libraries can live in one
 * process. Same status codes, same version packing, same rules: only symbols
 * declared here are stable; unknown capability bits must be ignored; additive
 * changes bump MINOR.
 *
 * Pointer convention. The entry points that keep the reference's name and
 * signature take HOST pointers, exactly like the reference (the library copies
 * to and from the GPU). The *_dev entry points take DEVICE pointers plus a
 * hipStream_t (passed as void*, NULL = the null stream) and never synchronize.
 */
#ifndef SNHIP_ABI_H
#define SNHIP_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SNHIP_ABI_VERSION_MAJOR 1
#define SNHIP_ABI_VERSION_MINOR 1
#define SNHIP_ABI_VERSION_PATCH 0
#define SNHIP_ABI_VERSION \
    ((SNHIP_ABI_VERSION_MAJOR << 16) | (SNHIP_ABI_VERSION_MINOR << 8) | \
     SNHIP_ABI_VERSION_PATCH)

/* Capability bits 0..4 keep the reference's meaning (sn_abi.h:34-38). */
#define SNHIP_CAP_RECUR_SCAN  (1u << 0)   /* snhip_abi_recur_scan            */
#define SNHIP_CAP_RECUR_STEP  (1u << 1)   /* snhip_abi_recur_step            */
#define SNHIP_CAP_QUANT_I8    (1u << 2)   /* not provided by this backend    */
#define SNHIP_CAP_RWKV7       (1u << 3)   /* snhip_abi_rwkv7_*               */
#define SNHIP_CAP_THREADS     (1u << 4)   /* snhip_abi_set/get_threads       */
/* Additions of this backend (MINOR 1). */
#define SNHIP_CAP_DEVICE_PTR  (1u << 8)   /* *_dev entry points              */
#define SNHIP_CAP_SUNNY_MODEL (1u << 9)   /* snhip_load / snhip_step ...     */
#define SNHIP_CAP_INT4        (1u << 10)  /* INT4 group quantization         */
#define SNHIP_CAP_BATCH       (1u << 11)  /* batched decode                  */
#define SNHIP_CAP_PREFILL     (1u << 12)  /* chunked batched prefill         */

/* Status codes: the reference's (sn_abi.h:41-46) plus SN_E_DEVICE. */
#define SNHIP_OK              0
#define SNHIP_E_INVAL        -1   /* NULL pointer or non-positive dimension */
#define SNHIP_E_NOMEM        -2   /* allocation failed (host or device)     */
#define SNHIP_E_IO           -3   /* open or read failed                    */
#define SNHIP_E_FORMAT       -4   /* magic / version / size mismatch        */
#define SNHIP_E_UNSUPPORTED  -5   /* not supported by this build            */
#define SNHIP_E_DEVICE       -6   /* HIP runtime error (no GPU, launch ...) */

typedef int32_t snhip_status;

/* ------------------------------------------------------------ version */
/* sn_abi.h:52 */
int32_t snhip_abi_version(void);
/* sn_abi.h:55 */
uint32_t snhip_abi_caps(void);
/* sn_abi.h:58: SNHIP_OK when caller_major == SNHIP_ABI_VERSION_MAJOR. */
snhip_status snhip_abi_check(int32_t caller_major);
/* sn_abi.h:62: writes "1.1.0"; returns the needed length incl. NUL. */
int32_t snhip_abi_version_string(char* buf, int32_t buflen);
/* sn_abi.h:65: writes "hip". */
int32_t snhip_abi_backend_string(char* buf, int32_t buflen);
/* Last HIP error text of this thread ("" if none). Same length protocol. */
int32_t snhip_abi_last_error(char* buf, int32_t buflen);

/* ------------------------------------------------------------ threads */
/* sn_abi.h:68-69. Host threads used for host-side preparation (blob
 * transposes and quantization at load). n <= 0 -> SNHIP_E_INVAL. */
snhip_status snhip_abi_set_threads(int32_t n);
int32_t snhip_abi_get_threads(void);

/* ------------------------------------------- first-order recurrence */
/* s_t = a_t * s_{t-1} + b_t per channel; gated != 0 means b is u and
 * b_t = (1 - a_t) * u_t. Bit-identical to the reference C runtime
 * (sunnynet/runtime/recur.c:13-48, 109-131).
 *
 * sn_abi.h:74-75 — a, b, s (B, N) fp32 host pointers; s updated in place. */
snhip_status snhip_abi_recur_step(const float* a, const float* b, float* s,
                                  int32_t B, int32_t N, int32_t gated);
/* sn_abi.h:78-80 — a, b, out (B, T, N); s0, send (B, N); host pointers. */
snhip_status snhip_abi_recur_scan(const float* a, const float* b,
                                  const float* s0, float* out, float* send,
                                  int32_t B, int32_t T, int32_t N,
                                  int32_t gated);
/* Device-pointer forms of the two above (no reference counterpart; the
 * reference has no device memory). Enqueued on `stream`. */
snhip_status snhip_abi_recur_step_dev(const float* a, const float* b, float* s,
                                      int32_t B, int32_t N, int32_t gated,
                                      void* stream);
snhip_status snhip_abi_recur_scan_dev(const float* a, const float* b,
                                      const float* s0, float* out, float* send,
                                      int32_t B, int32_t T, int32_t N,
                                      int32_t gated, void* stream);

/* sunnynet/kernels/scan_avx2.c:50-99 (scan_bwd_f32), device pointers: the
 * gradients of the gated scan s_t = p_t s_{t-1} + (1 - p_t) nu_t. Inputs p, nu,
 * out (the forward states) and dout (B,T,N), s0 (B,N); outputs dp, dnu
 * (B,T,N) and ds0 (B,N), bit-identical to the reference. Enqueued on `stream`. */
snhip_status snhip_abi_scan_bwd_dev(const float* p, const float* nu, const float* s0,
                                    const float* out, const float* dout, float* dp,
                                    float* dnu, float* ds0, int32_t B, int32_t T,
                                    int32_t N, void* stream);

/* sunnynet/kernels/core_avx2.c:34-73 (core_fwd_f32), device pointers: the
 * fused compete gate + decay gate + gated scan of a block. q (B,T,2D) holds
 * [u_raw | gate] per step, delta (D), s0 (B,D); outputs states, u, p (B,T,D).
 * D must be a multiple of 8 (groups of 8 channels, as the reference's kernel
 * assumes). Every operation is the reference's except expf (the device's,
 * within 1 ulp). Enqueued on `stream`. */
snhip_status snhip_abi_core_fwd_dev(const float* q, const float* delta, const float* s0,
                                    float* states, float* u, float* p, int32_t B,
                                    int32_t T, int32_t D, void* stream);
/* sunnynet/kernels/core_avx2.c:78-149 (core_bwd_f32), device pointers: from
 * the forward's inputs and outputs and the upstream gradients dstate, du_in
 * (B,T,D), writes dq (B,T,2D) and ds0 (B,D), and ADDS the delta gradient into
 * ddelta (D) as the reference does (its caller zeroes it). ddelta's terms are
 * summed in a fixed order, so repeated calls give identical results.
 * Enqueued on `stream` (allocates a B*D float workspace stream-ordered). */
snhip_status snhip_abi_core_bwd_dev(const float* q, const float* delta, const float* s0,
                                    const float* states, const float* u, const float* p,
                                    const float* dstate, const float* du_in, float* dq,
                                    float* ddelta, float* ds0, int32_t B, int32_t T,
                                    int32_t D, void* stream);

/* Bandwidth calibration (no counterpart in the reference): plain streaming
 * kernels over n fp32 values, float4 per lane, non-temporal, grid-stride, on
 * `grid` workgroups of 256 threads. kind 0: c = a + b (two arrays read, one
 * written: the gated scan's byte pattern); kind 1: a and b read (their sums
 * land in c[0 .. grid), so c needs 4 * grid floats). n a multiple of 4, the
 * arrays 16-byte aligned. Enqueued on `stream`. */
snhip_status snhip_abi_hbm_probe_dev(int32_t kind, const float* a, const float* b, float* c,
                                     int64_t n, int32_t grid, void* stream);

/* snhip_abi_core_bwd_dev without any device allocation: same arguments,
 * kernels and results (bit for bit). No counterpart in the reference; for
 * callers that cannot allocate (code under HIP graph capture, tight serving or
 * training loops, harnesses that forbid hipMalloc). The (B, D) ddelta
 * partials live in a fixed per-GPU scratch array of 2^20 floats (4 MiB, held
 * until the process ends): B * D above 1048576 returns SNHIP_E_INVAL with an
 * error text. Calls that overlap on one GPU share that array and race; serialize
 * them (one stream, or events). The first call on a device resolves the array's
 * address there. */
snhip_status snhip_abi_core_bwd_dev_noalloc(const float* q, const float* delta, const float* s0,
                                            const float* states, const float* u, const float* p,
                                            const float* dstate, const float* du_in, float* dq,
                                            float* ddelta, float* ds0, int32_t B, int32_t T,
                                            int32_t D, void* stream);

/* ----------------------------------------------- INT4 (group-wise) */
/* Format of sunnynet/runtime/quant.c:34-87: W (rows, N) row-major; groups of
 * `block` inputs share scale = amax/7 (1 if amax == 0); byte k of a group
 * holds element k (low nibble) and element k + block/2 (high nibble), values
 * q + 8 with q in [-8, 7]. Bit-identical to sn_quant_i4 / sn_dequant_i4.
 * Device pointers; N % block == 0, block even. */
snhip_status snhip_abi_quant_i4_dev(const float* x, uint8_t* q, float* scale,
                                    int32_t rows, int32_t N, int32_t block,
                                    void* stream);
snhip_status snhip_abi_dequant_i4_dev(const uint8_t* q, const float* scale,
                                      float* x, int32_t rows, int32_t N,
                                      int32_t block, void* stream);

/* ------------------------------------------------------- dense linear */
/* y (M, N) = x (M, K) w^T with w row-major (N, K), fp32, on the FP32 matrix
 * cores (torch.nn.functional.linear without bias). Device pointers, 16-byte
 * aligned, K % 32 == 0. No reference counterpart: the batched decode and the
 * chunked prefill are built on it. */
snhip_status snhip_abi_linear_dev(const float* x, const float* w, float* y, int32_t M,
                                  int32_t N, int32_t K, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SNHIP_ABI_H */
