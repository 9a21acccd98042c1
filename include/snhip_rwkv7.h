/* RWKV-7 decode handle on the HIP backend.
 *
 * Mirrors the reference's sunnynet/runtime/rwkv7.h:14-28 (sn_rk_load /
 * sn_rk_step / sn_rk_prefill / sn_rk_reset / sn_rk_free / sn_rk_vocab /
 * sn_rk_ready) with the prefix snhip_rk_ and the same argument order, meaning
 * and error behaviour: the loader reads the reference's v3 blob
 * (experiments/_export_rwkv7.py format) and returns NULL on an IO, magic,
 * version, dimension or allocation failure; void functions tolerate a NULL
 * handle; logits buffers of the mirrored calls are caller-owned HOST memory of
 * length vocab; prefill feeds the tokens in order (rwkv7.c:362-364).
 *
 * Weights: INT4-tagged matrices of the blob (group 64) stay INT4 and are
 * dequantized in registers, bit-identically to sn_dequant_i4; fp32 matrices
 * stay fp32 unless snhip_rk_load_ex asks for INT4 (then every fp32 matrix whose
 * input length is a multiple of `block` is quantized at load). The reference
 * runs INT4 matrices as W4A8; this backend keeps activations fp32 (W4A32).
 *
 * Extensions: max_batch independent sequences, device-pointer entry points on a
 * caller stream, on-device greedy decoding, state import/export:
 *   S     (B, layers, n_head, head_size, head_size)  fp32, S[.., i, j] row i
 *   shift (B, layers, 2, dim)                         fp32 (time mix, channel mix)
 */
#ifndef SNHIP_RWKV7_H
#define SNHIP_RWKV7_H

#include <stdint.h>

#include "snhip_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct SnHipRwkv7 SnHipRwkv7;

/* Weight format for snhip_rk_load_ex besides SNHIP_WEIGHTS_F32 (0) and
 * SNHIP_WEIGHTS_INT4 (1) of snhip.h: every matrix as the blob stores it. */
#define SNHIP_WEIGHTS_STORED 2

/* rwkv7.h:16: B = 1, each matrix as stored in the blob. */
SnHipRwkv7* snhip_rk_load(const char* path);
/* Same checks; max_batch sequences; weight_format SNHIP_WEIGHTS_STORED,
 * SNHIP_WEIGHTS_F32 (INT4 blob matrices dequantized at load) or
 * SNHIP_WEIGHTS_INT4 (fp32 blob matrices quantized at load with group `block`,
 * 32 or 64, where block divides their input length). */
SnHipRwkv7* snhip_rk_load_ex(const char* path, int32_t max_batch, int32_t weight_format,
                             int32_t block);
/* rwkv7.h:17-18 */
void snhip_rk_free(SnHipRwkv7* m);
void snhip_rk_reset(SnHipRwkv7* m);
/* rwkv7.h:21-22: sequence 0; logits host, length vocab. */
void snhip_rk_step(SnHipRwkv7* m, int token, float* logits);
void snhip_rk_prefill(SnHipRwkv7* m, const int* tokens, int n, float* logits);
/* rwkv7.h:24-25 (sn_rk_dbg, rwkv7.c:366-374): sequence 0 steps `token`
 * through layers 0..layer (their state advances, later layers are untouched)
 * on the per-kernel step, which repeats the reference's rounding, and out
 * (host, 9 * dim floats) receives that layer's xn, r, k, v, a, g, ww, y and
 * output x, each (dim,), in the reference's order and bit for bit.
 * SNHIP_E_INVAL for a bad token or layer. */
snhip_status snhip_rk_dbg(SnHipRwkv7* m, int token, int layer, float* out);
/* rwkv7.h:27-28 */
int snhip_rk_vocab(const SnHipRwkv7* m);
int snhip_rk_ready(const SnHipRwkv7* m);

/* ---- extensions ---------------------------------------------------------- */
/* Time-outs: the one-launch steps update S and shift in place
 * layer by layer; a call whose launch timed out returns SNHIP_E_DEVICE and the
 * handle refuses every stepping call (SNHIP_E_DEVICE) until snhip_rk_reset or
 * snhip_rk_set_state_dev. The void mirrors drop the status: use
 * snhip_abi_rwkv7_step / snhip_abi_rwkv7_prefill to see it. */
snhip_status snhip_rk_set_stream(SnHipRwkv7* m, void* stream);
int32_t snhip_rk_max_batch(const SnHipRwkv7* m);
/* Workgroups of the one-launch step that runs steps of a single sequence
 * (one cooperative launch per call of greedy steps, one per step otherwise),
 * or 0 when steps of one sequence take the per-kernel step (no cooperative
 * launch, a shape it does not take, or SNHIP_RK_EXACT=0 in the environment
 * at load). By default it is the exact-order kernel, whose logits equal the
 * reference's sn_rk_step bit for bit. With SNHIP_RK_PERSIST=1 at load it is
 * instead a kernel that sums in parallel, not bit-exact (measured up to
 * 1.3e-4 from sn_rk_step). Calls that take either return once their steps
 * have finished, so that a time-out of an exchange wait is reported as
 * SNHIP_E_DEVICE. No reference counterpart. */
int32_t snhip_rk_persist_grid(const SnHipRwkv7* m);
/* 1 when that one-launch step is the exact-order kernel, else 0. */
int32_t snhip_rk_persist_exact(const SnHipRwkv7* m);
/* Workgroups of the launch when steps of B sequences run as B copies of that
 * one-launch step, each sequence on its own equal slice of the grid (B *
 * slice; for B = 1 the value above), or 0 when steps of B sequences take the
 * per-kernel path. B <= 8 by default; SNHIP_RK_PERSIST_MI=n in the
 * environment at load sets the limit (1: off, at most 32). Each sequence's
 * results equal its one-sequence launch's bit for bit; time-outs behave as
 * for one sequence. No reference counterpart. */
int32_t snhip_rk_persist_grid_batch(const SnHipRwkv7* m, int32_t B);
/* One step of sequences [0, B): tokens_dev (B) int32, logits_dev (B, vocab). */
snhip_status snhip_rk_step_batch_dev(SnHipRwkv7* m, const int32_t* tokens_dev, int32_t B,
                                     float* logits_dev);
/* Greedy decoding on the device (first maximal logit): feeds tokens_dev (B),
 * out_tokens_dev (n_steps, B) receives each step's choice; logits_dev (B,
 * vocab), if not NULL, the last step's logits. */
snhip_status snhip_rk_decode_greedy_dev(SnHipRwkv7* m, const int32_t* tokens_dev, int32_t B,
                                        int32_t n_steps, int32_t* out_tokens_dev,
                                        float* logits_dev);
snhip_status snhip_rk_get_state_dev(SnHipRwkv7* m, float* S_dev, float* shift_dev, int32_t B);
snhip_status snhip_rk_set_state_dev(SnHipRwkv7* m, const float* S_dev, const float* shift_dev,
                                    int32_t B);

/* expf and tanhf as the step computes them: restatements of the host C
 * library's algorithms (glibc expf, fdlibm tanhf), so that they round as the
 * reference's CPU runtime does. x, e, t hold n floats; _host computes on the
 * CPU, _dev on the GPU (device pointers, enqueued on `stream`). For tests of
 * the restatement against the host libm; no reference counterpart. */
snhip_status snhip_refmath_host(const float* x, float* e, float* t, int32_t n);
snhip_status snhip_refmath_dev(const float* x, float* e, float* t, int32_t n, void* stream);

/* Stable-ABI mirror of sn_abi.h:88-100 (sn_abi_rwkv7_*): status codes of
 * snhip_abi.h; logits host memory of at least snhip_abi_rwkv7_vocab floats. */
SnHipRwkv7* snhip_abi_rwkv7_load(const char* blob_path);
snhip_status snhip_abi_rwkv7_step(SnHipRwkv7* m, int32_t token, float* logits);
snhip_status snhip_abi_rwkv7_prefill(SnHipRwkv7* m, const int32_t* tokens, int32_t n,
                                     float* logits);
snhip_status snhip_abi_rwkv7_reset(SnHipRwkv7* m);
void snhip_abi_rwkv7_free(SnHipRwkv7* m);
int32_t snhip_abi_rwkv7_vocab(const SnHipRwkv7* m);

#ifdef __cplusplus
}
#endif
#endif /* SNHIP_RWKV7_H */
