/* CPU oracle for the SunnyNet token loop.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the CPU
 * baseline leg of bench.py may load this library, and only as the checker.
 * The HIP product library never links, calls or falls back to it.
 *
 * Each function restates the reference algorithm in plain ISO C with the
 * reference's operation order (explicit fmaf() exactly where the reference
 * uses an FMA intrinsic, no implicit contraction), so that its outputs are
 * bit-identical to the reference C runtime compiled from its own sources.
 */
#ifndef SN_ORACLE_H
#define SN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- first-order recurrence: sunnynet/runtime/recur.c:13-48, 109-131 ---- */
void orc_recur_scan(const float* a, const float* b, const float* s0,
                    float* out, float* send, int B, int T, int N, int gated);
void orc_recur_step(const float* a, const float* b, float* s, int B, int N,
                    int gated);

/* ---- gated-scan backward: sunnynet/kernels/scan_avx2.c:50-99 ----
 * Reverse time per channel: ds += dout_t; dnu_t = ds (1 - p_t);
 * dp_t = ds (s_{t-1} - nu_t) (s_{-1} = s0); ds *= p_t; ds0 = ds at the end. */
void orc_scan_bwd(const float* p, const float* nu, const float* s0, const float* out,
                  const float* dout, float* dp, float* dnu, float* ds0, int B, int T, int N);

/* ---- fused compete + gate + scan, forward and backward:
 * sunnynet/kernels/core_avx2.c:34-149. Groups of 8 channels; within a group,
 * e = expf(-g), s1 = 1 / (1 + e_i / e_{i+1}), s2 = 1 / (1 + e_i / e_{i+2}),
 * u = u_raw s1 s2, p = fma(delta, sigma, 1 - delta), s = fma(p, s, (1 - p) u).
 * The backward accumulates ddelta += over b in order (the reference's result
 * with one OpenMP thread). */
void orc_core_fwd(const float* q, const float* delta, const float* s0, float* states, float* uo,
                  float* po, int B, int T, int D);
void orc_core_bwd(const float* q, const float* delta, const float* s0, const float* states,
                  const float* uo, const float* po, const float* dstate, const float* du_in,
                  float* dq, float* ddelta, float* ds0, int B, int T, int D);

/* ---- group-wise INT4: sunnynet/runtime/quant.c:34-87 ---- */
void orc_quant_i4(const float* x, uint8_t* q, float* scale, int rows, int N,
                  int block);
void orc_dequant_i4(const uint8_t* q, const float* scale, float* x, int rows,
                    int N, int block);

/* ---- whole-model decode step: sunnynet/runtime/sunnynet.c:123-454 ----
 * The oracle parses the packed fp32 blob (experiments/_export_runtime.py:3-17)
 * held in caller memory, flips the (in,out) matrices to (out,in) like
 * sn_load, and keeps `batch` independent sequences (each is exactly one
 * reference handle). */
typedef struct OrcSn OrcSn;
OrcSn* orc_sn_new(const void* blob, int64_t nbytes, int batch);
void orc_sn_free(OrcSn* m);
void orc_sn_reset(OrcSn* m);
/* hdr[10] = vocab, D, I, R, K, L, group, tied, clamp, batch */
void orc_sn_dims(const OrcSn* m, int32_t* hdr);
/* One decode step for every sequence: tokens[batch] -> logits[batch][vocab]. */
void orc_sn_step(OrcSn* m, const int32_t* tokens, float* logits);
/* Step one sequence only. */
void orc_sn_step_one(OrcSn* m, int b, int32_t token, float* logits);
/* State in the torch SunnyState layout: s (batch,L,D), hist (batch,L,K-1,D)
 * with hist[...,0,:] the newest entry. */
void orc_sn_get_state(const OrcSn* m, float* s, float* hist);
void orc_sn_set_state(OrcSn* m, const float* s, const float* hist);
/* Per-layer intermediates of sequence b (sunnynet.c:278-290 order):
 * raw, at, v, gate, u, s, zn, yn, sfb, out. Advances that layer's state. */
void orc_sn_dbg_layer(OrcSn* m, int b, int32_t token, int layer, float* dbg);

/* ---- RWKV-7 decode: sunnynet/runtime/rwkv7.c:143-508 (blob v3) ---- */
typedef struct OrcRk OrcRk;
/* block: INT4 group size used by tag-1 matrices in the blob (the reference
 * hard-codes 64, rwkv7.c:35). */
/* The host C library's expf and tanhf over n inputs: what the reference's
 * runtime computes (its transcendentals are libm's). */
void orc_libm(const float* x, float* e, float* t, int64_t n);

OrcRk* orc_rk_new(const void* blob, int64_t nbytes, int batch, int block);
void orc_rk_free(OrcRk* m);
void orc_rk_reset(OrcRk* m);
/* hdr[8] = L, D, HS, NH, F, vocab, q4, batch */
void orc_rk_dims(const OrcRk* m, int32_t* hdr);
void orc_rk_step(OrcRk* m, const int32_t* tokens, float* logits);
void orc_rk_step_one(OrcRk* m, int b, int32_t token, float* logits);
/* state: S (batch,L,NH,HS,HS), shift (batch,L,2,D) */
void orc_rk_get_state(const OrcRk* m, float* S, float* shift);
void orc_rk_set_state(OrcRk* m, const float* S, const float* shift);

#ifdef __cplusplus
}
#endif
#endif
