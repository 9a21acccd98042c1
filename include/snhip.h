/* SunnyNet HIP backend: whole-model decode handle.
 *
 * Mirrors the reference's internal C ABI, sunnynet/runtime/sunnynet.h:18-47
 * (sn_load / sn_step / sn_prefill / sn_reset / sn_free / sn_vocab / sn_ready),
 * with the prefix snhip_ and the same argument order, meaning and error
 * behaviour: loaders return NULL on an IO, magic, dimension or allocation
 * failure; void functions tolerate a NULL handle; logits buffers of the
 * mirrored calls are caller-owned HOST memory of length vocab. The weight file
 * is the reference's packed fp32 runtime blob.
 *
 * Extensions (no reference counterpart; the reference is B=1, host-only):
 * batched decode over independent sequences, device-pointer entry points on a
 * caller stream, INT4 group-quantized weights, on-device greedy decoding, and
 * state import/export in the torch SunnyState layout:
 *   s    (B, layers, dim)             fp32
 *   hist (B, layers, taps-1, dim)     fp32, hist[..., 0, :] the newest input.
 *
 * A handle owns its device memory and is not reentrant (one caller at a time),
 * like the reference's (per-handle scratch, sunnynet.c:214).
 */
#ifndef SNHIP_H
#define SNHIP_H

#include <stdint.h>

#include "snhip_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct SnHipModel SnHipModel;

/* Weight formats for snhip_load_ex. */
#define SNHIP_WEIGHTS_F32   0   /* fp32, as in the blob                        */
#define SNHIP_WEIGHTS_INT4  1   /* V, U, W_z, W_c, W_s_eff and the LM head
                                   quantized at load with quant.c's symmetric
                                   group format; embedding lookup stays fp32  */
#define SNHIP_WEIGHTS_F16   3   /* sn_load_h's values (sunnynet.c:455-579): the
                                   same matrices rounded to fp16 (nearest even)
                                   at load; the single-sequence persistent step
                                   reads them as fp16 (half the bytes), the
                                   other paths from an fp32 copy of the values */

/* sunnynet.h:22-23: B = 1, fp32 weights. */
SnHipModel* snhip_load(const char* path, int vocab, int dim, int inner, int rank,
                       int taps, int layers, int group, int tied);

/* sunnynet.h:25-28 (sn_load_h): B = 1, weight_format SNHIP_WEIGHTS_F16. */
SnHipModel* snhip_load_h(const char* path, int vocab, int dim, int inner, int rank,
                         int taps, int layers, int group, int tied);

/* Same checks as snhip_load; max_batch sequences, weight_format SNHIP_WEIGHTS_*,
 * block = INT4 group size along the input dim (even, divides dim, inner, rank).
 * path may also name an INT4 blob (magic 'SNQ4', written by
 * `python -m sunnynet_amd.blob --int4`; no counterpart in the reference):
 * its codes and scales load as stored, with weight_format SNHIP_WEIGHTS_INT4
 * and block equal to the blob's group size; snhip_load refuses it. */
SnHipModel* snhip_load_ex(const char* path, int vocab, int dim, int inner, int rank,
                          int taps, int layers, int group, int tied,
                          int32_t max_batch, int32_t weight_format, int32_t block);

/* sunnynet.h:30 */
void snhip_free(SnHipModel* m);
/* sunnynet.h:31: zero every sequence's state and conv history. */
void snhip_reset(SnHipModel* m);
/* sunnynet.h:34: one decode step of sequence 0; logits: host, length vocab. */
void snhip_step(SnHipModel* m, int token, float* logits);
/* sunnynet.h:37: feed n tokens of sequence 0 in order; last logits to host.
 * Runs the chunked prefill (snhip_prefill_batch_dev with B = 1). */
void snhip_prefill(SnHipModel* m, const int* tokens, int n, float* logits);
/* sunnynet.h:39-40 */
int snhip_vocab(const SnHipModel* m);
int snhip_ready(const SnHipModel* m);

/* sunnynet.h:42-47. n <= 0 keeps the current setting. The decode products run
 * on the GPU; the count sizes host-side work (blob preparation at load) and is
 * the same setting as snhip_abi_set_threads / snhip_abi_get_threads.
 * snhip_recommended_threads: physical cores ((physical id, core id) pairs of
 * /proc/cpuinfo), the logical count if none are listed, 0 if unreadable. */
void snhip_set_threads(int n);
int snhip_get_threads(void);
int snhip_recommended_threads(void);

/* ---- extensions ---------------------------------------------------------- */
/* snhip_prefill with a status: SNHIP_E_INVAL for out-of-range tokens or bad
 * arguments, SNHIP_E_DEVICE for a HIP failure or a refused handle (below). */
snhip_status snhip_prefill_host(SnHipModel* m, const int32_t* tokens, int32_t n, float* logits);

/* Time-outs. Every wait of the persistent kernels is bounded; a call whose
 * launch timed out returns SNHIP_E_DEVICE once its work has finished (calls
 * that run a persistent kernel wait for it). The workgroups of a launch stop
 * independently, so a timed-out call may have written part of the state of the
 * sequences it stepped (some channels of sequence 0 in a single-sequence call,
 * some layers in a batched step): the handle then refuses every stepping call
 * (SNHIP_E_DEVICE) until snhip_reset, or snhip_set_state_dev over at least
 * those sequences, gives them a valid state. */

/* Stream for all later work of this handle (NULL = the null stream). */
snhip_status snhip_set_stream(SnHipModel* m, void* stream);
int32_t snhip_max_batch(const SnHipModel* m);

/* One decode step of sequences [0, B): tokens_dev (B) int32 on the device,
 * logits_dev (B, vocab) fp32 on the device. Enqueued on the handle's stream. */
snhip_status snhip_step_batch_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                  float* logits_dev);
/* Same with host tokens and host logits (synchronous). Tokens are range-checked. */
snhip_status snhip_step_batch(SnHipModel* m, const int32_t* tokens, int32_t B, float* logits);

/* Chunked prefill of sequences [0, B) from their current state: tokens_dev
 * (B, T) int32 row-major on the device. Runs the model over the whole prompt
 * with matrix-core GEMMs and the fused gate + exact sequential scan, T cut in
 * chunks with the state carried between them; leaves s and hist as stepping
 * token by token would (to float rounding). logits_dev (B, vocab), if not
 * NULL, receives the last token's logits (the sn_prefill contract). */
snhip_status snhip_prefill_batch_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                     int32_t T, float* logits_dev);

/* sn_dbg_layer (sunnynet/runtime/sunnynet.c:336-345): steps sequence 0 from
 * the embedding of `token` through layers 0..layer (updating their state and
 * history, as the reference does) and writes that layer's intermediates to
 * the HOST buffer dbg of 7 dim + rank + 2 inner floats, in the reference's
 * order (sunnynet.c:278-289): LN_in output, at (after the conv), v = V at, the
 * gate half of U v, u (after the competitive gate), the new state, z (after
 * the wedge), LN_I(z), W_eff s_old and the layer's output. Runs the per-kernel
 * (GEMV) step. SNHIP_E_INVAL for a token or layer out of range. */
snhip_status snhip_dbg_layer(SnHipModel* m, int32_t token, int32_t layer, float* dbg);

/* The same chunked prefill with the logits of every position: logits_all_dev
 * (B, T, vocab) fp32 on the device, row (b, t) at offset (b T + t) vocab,
 * computed by the tied head over the final norm of each position (MFMA GEMM).
 * Replaces SunnyNet.forward(idx, state, return_state=True)
 * (sunnynet/model.py:89-111), which returns (B, T, V) logits and the state:
 * the state is left in the handle (snhip_get_state_dev; history newest first). */
snhip_status snhip_prefill_all_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                   int32_t T, float* logits_all_dev);

/* Greedy decoding on the device: feeds tokens_dev (B), then repeatedly takes
 * the first maximal logit as the next token, for n_steps steps. out_tokens_dev
 * (n_steps, B) receives the tokens chosen after each step; logits_dev (B,
 * vocab), if not NULL, the last step's logits. No host synchronization, except
 * that a call running a persistent kernel waits for it (Time-outs above). */
snhip_status snhip_decode_greedy_dev(SnHipModel* m, const int32_t* tokens_dev, int32_t B,
                                     int32_t n_steps, int32_t* out_tokens_dev,
                                     float* logits_dev);

/* Grid size of the persistent single-sequence decode (B = 1 steps and greedy
 * decoding run every layer of every step in one cooperative launch), or 0 when
 * this handle uses the per-kernel step (shape above 2048 wide, taps > 8, no
 * cooperative launch, or SNHIP_PERSIST=0 in the environment at load). */
int32_t snhip_persistent_grid(const SnHipModel* m);

/* Workgroups of the persistent decode when steps of B sequences run as B
 * copies of the single-sequence kernel in one cooperative launch, each
 * sequence on its own equal slice of the grid (B * slice; the slice for B = 1
 * is snhip_persistent_grid), or 0 when steps of B sequences take another path.
 * Defaults: B <= 16 for INT4 rows, B <= 4 for fp32 / fp16 rows;
 * SNHIP_PERSIST_MI in the environment at load sets the limit (1: off). No
 * counterpart in the reference: its C runtime steps one sequence at a time
 * (sunnynet.c:212). */
int32_t snhip_persistent_grid_batch(const SnHipModel* m, int32_t B);

/* Grid size of the persistent batched step (steps of 3 to 64 sequences that
 * the single-sequence kernel does not take run every layer in one cooperative
 * launch, then the head), or 0 when this handle
 * uses the per-kernel step for them (shapes other than the compiled product
 * depths, max_batch below 3, no cooperative launch, or SNHIP_BATCH_PERSIST=0
 * in the environment at load). No counterpart in the reference: its C runtime
 * steps one sequence at a time (sunnynet.c:212). */
int32_t snhip_batch_grid(const SnHipModel* m);

/* State of sequences [0, B) in the SunnyState layout above, device pointers. */
snhip_status snhip_get_state_dev(SnHipModel* m, float* s_dev, float* hist_dev, int32_t B);
snhip_status snhip_set_state_dev(SnHipModel* m, const float* s_dev, const float* hist_dev,
                                 int32_t B);

#ifdef __cplusplus
}
#endif
#endif /* SNHIP_H */
