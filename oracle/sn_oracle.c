/* CPU oracle for the SunnyNet token loop: recurrence, INT4 format and the
 * whole-model decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see sn_oracle.h). Restates the reference's C
 * runtime in scalar ISO C with the same operation order; built with
 * -std=c11 -ffp-contract=off so that a*b+c stays two roundings exactly where
 * the reference's -std=c11 build keeps it two roundings, and fmaf() appears
 * exactly where the reference calls _mm256_fmadd_ps.
 */
#include "sn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* recur.c:13-48. Channels [0, N&~7) take the 8-wide AVX2 path: b' = (1-a)*u,
 * then s = fma(a, s, b'). The scalar tail [N&~7, N) computes a*s + b' with
 * two roundings (recur.c:36-46). */
void orc_recur_scan(const float* a, const float* b, const float* s0,
                    float* out, float* send, int B, int T, int N, int gated) {
    const int N8 = N & ~7;
    #pragma omp parallel for schedule(static)
    for (int bb = 0; bb < B; ++bb) {
        const float* ab = a + (size_t)bb * T * N;
        const float* bbb = b + (size_t)bb * T * N;
        float* ob = out + (size_t)bb * T * N;
        for (int d = 0; d < N; ++d) {
            float s = s0[(size_t)bb * N + d];
            for (int t = 0; t < T; ++t) {
                const size_t off = (size_t)t * N + d;
                const float av = ab[off];
                float bv = bbb[off];
                if (gated) bv = (1.0f - av) * bv;
                if (d < N8) s = fmaf(av, s, bv);
                else s = av * s + bv;
                ob[off] = s;
            }
            send[(size_t)bb * N + d] = s;
        }
    }
}

/* scan_avx2.c:50-99. The 8-wide path and the scalar tail use the same
 * operations in the same order (add, then sub and mul for each output, then
 * mul), none fused, so one scalar loop restates both. */
void orc_scan_bwd(const float* p, const float* nu, const float* s0, const float* out,
                  const float* dout, float* dp, float* dnu, float* ds0, int B, int T, int N) {
    #pragma omp parallel for schedule(static)
    for (int bb = 0; bb < B; ++bb) {
        const size_t rb = (size_t)bb * T * N;
        for (int d = 0; d < N; ++d) {
            float ds = 0.0f;
            for (int t = T - 1; t >= 0; --t) {
                const size_t off = rb + (size_t)t * N + d;
                ds = dout[off] + ds;
                const float pv = p[off];
                const float sprev = t > 0 ? out[off - N] : s0[(size_t)bb * N + d];
                dnu[off] = ds * (1.0f - pv);
                dp[off] = ds * (sprev - nu[off]);
                ds = ds * pv;
            }
            ds0[(size_t)bb * N + d] = ds;
        }
    }
}

/* core_avx2.c:34-73, lane by lane (lane i of a group reads e of lanes i+1,
 * i+2 mod 8 where the reference permutes). */
void orc_core_fwd(const float* q, const float* delta, const float* s0, float* states, float* uo,
                  float* po, int B, int T, int D) {
    #pragma omp parallel for schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int d0 = 0; d0 < D; d0 += 8) {
            float s[8], e[8];
            for (int i = 0; i < 8; ++i) s[i] = s0[(size_t)b * D + d0 + i];
            for (int t = 0; t < T; ++t) {
                const size_t qo = ((size_t)b * T + t) * 2 * D + d0;
                const size_t so = ((size_t)b * T + t) * D + d0;
                for (int i = 0; i < 8; ++i) e[i] = expf(0.0f - q[qo + D + i]);
                for (int i = 0; i < 8; ++i) {
                    const float dl = delta[d0 + i];
                    const float sig = 1.0f / (1.0f + e[i]);
                    const float s1 = 1.0f / (1.0f + e[i] / e[(i + 1) & 7]);
                    const float s2 = 1.0f / (1.0f + e[i] / e[(i + 2) & 7]);
                    const float u = q[qo + i] * (s1 * s2);
                    const float p = fmaf(dl, sig, 1.0f - dl);
                    s[i] = fmaf(p, s[i], (1.0f - p) * u);
                    states[so + i] = s[i];
                    uo[so + i] = u;
                    po[so + i] = p;
                }
            }
        }
    }
}

/* core_avx2.c:78-149, lane by lane in the reference's operation order. */
void orc_core_bwd(const float* q, const float* delta, const float* s0, const float* states,
                  const float* uo, const float* po, const float* dstate, const float* du_in,
                  float* dq, float* ddelta, float* ds0, int B, int T, int D) {
    float* acc = (float*)calloc((size_t)B * D, sizeof(float));
    #pragma omp parallel for schedule(static)
    for (int b = 0; b < B; ++b) {
        for (int d0 = 0; d0 < D; d0 += 8) {
            float ds[8] = {0}, dacc[8] = {0}, e[8], a1[8], a2[8];
            for (int t = T - 1; t >= 0; --t) {
                const size_t qo = ((size_t)b * T + t) * 2 * D + d0;
                const size_t so = ((size_t)b * T + t) * D + d0;
                float dp[8], du[8];
                for (int i = 0; i < 8; ++i) {
                    ds[i] = ds[i] + dstate[so + i];
                    const float u = uo[so + i], p = po[so + i];
                    const float sprev = t > 0 ? states[so + i - D] : s0[(size_t)b * D + d0 + i];
                    dp[i] = ds[i] * (sprev - u);
                    du[i] = fmaf(ds[i], 1.0f - p, du_in[so + i]);
                    ds[i] = ds[i] * p;
                }
                for (int i = 0; i < 8; ++i) e[i] = expf(0.0f - q[qo + D + i]);
                float sig[8], s1[8], s2[8];
                for (int i = 0; i < 8; ++i) {
                    sig[i] = 1.0f / (1.0f + e[i]);
                    s1[i] = 1.0f / (1.0f + e[i] / e[(i + 1) & 7]);
                    s2[i] = 1.0f / (1.0f + e[i] / e[(i + 2) & 7]);
                    const float w = s1[i] * s2[i];
                    const float dw = du[i] * q[qo + i];
                    dq[qo + i] = du[i] * w;
                    const float ds1 = dw * s2[i], ds2 = dw * s1[i];
                    a1[i] = ds1 * (s1[i] * (1.0f - s1[i]));
                    a2[i] = ds2 * (s2[i] * (1.0f - s2[i]));
                }
                for (int i = 0; i < 8; ++i) {
                    float dg = a1[i] + a2[i];
                    dg = dg - a1[(i + 7) & 7];
                    dg = dg - a2[(i + 6) & 7];
                    dg = fmaf(dp[i] * delta[d0 + i], sig[i] * (1.0f - sig[i]), dg);
                    dacc[i] = fmaf(dp[i], sig[i] - 1.0f, dacc[i]);
                    dq[qo + D + i] = dg;
                }
            }
            for (int i = 0; i < 8; ++i) {
                ds0[(size_t)b * D + d0 + i] = ds[i];
                acc[(size_t)b * D + d0 + i] = dacc[i];
            }
        }
    }
    for (int b = 0; b < B; ++b)
        for (int d = 0; d < D; ++d) ddelta[d] += acc[(size_t)b * D + d];
    free(acc);
}

/* recur.c:109-131, same lane split as the scan. */
void orc_recur_step(const float* a, const float* b, float* s, int B, int N,
                    int gated) {
    const int N8 = N & ~7;
    for (int bb = 0; bb < B; ++bb) {
        for (int d = 0; d < N; ++d) {
            const size_t o = (size_t)bb * N + d;
            const float av = a[o];
            float bv = b[o];
            if (gated) bv = (1.0f - av) * bv;
            s[o] = (d < N8) ? fmaf(av, s[o], bv) : av * s[o] + bv;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* quant.c:34-65: per row, groups of `block` inputs share scale = amax/7
 * (1 when amax == 0); q = clamp(rint(w * (1/scale)), -8, 7) + 8; byte k of a
 * group holds element k (low nibble) and element k + block/2 (high nibble). */
void orc_quant_i4(const float* x, uint8_t* q, float* scale, int rows, int N,
                  int block) {
    if (block <= 0) block = 64;
    const int nb = N / block, half = block / 2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * N;
        uint8_t* qr = q + (size_t)r * (N / 2);
        float* sr = scale + (size_t)r * nb;
        for (int g = 0; g < nb; ++g) {
            const int lo = g * block;
            float amax = 0.0f;
            for (int i = 0; i < block; ++i) {
                const float v = fabsf(xr[lo + i]);
                if (v > amax) amax = v;
            }
            const float sc = amax > 0.0f ? amax / 7.0f : 1.0f;
            const float inv = 1.0f / sc;
            sr[g] = sc;
            for (int k = 0; k < half; ++k) {
                int lo4 = (int)nearbyintf(xr[lo + k] * inv);
                int hi4 = (int)nearbyintf(xr[lo + half + k] * inv);
                lo4 = lo4 < -8 ? -8 : (lo4 > 7 ? 7 : lo4);
                hi4 = hi4 < -8 ? -8 : (hi4 > 7 ? 7 : hi4);
                qr[(size_t)g * half + k] = (uint8_t)((lo4 + 8) | ((hi4 + 8) << 4));
            }
        }
    }
}

/* quant.c:67-87: w = ((q & 15) - 8) * scale, ((q >> 4) - 8) * scale. */
void orc_dequant_i4(const uint8_t* q, const float* scale, float* x, int rows,
                    int N, int block) {
    if (block <= 0) block = 64;
    const int nb = N / block, half = block / 2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const uint8_t* qr = q + (size_t)r * (N / 2);
        const float* sr = scale + (size_t)r * nb;
        float* xr = x + (size_t)r * N;
        for (int g = 0; g < nb; ++g) {
            const float sc = sr[g];
            for (int k = 0; k < half; ++k) {
                const uint8_t byte = qr[(size_t)g * half + k];
                xr[g * block + k] = (float)((int)(byte & 0x0F) - 8) * sc;
                xr[g * block + half + k] = (float)((int)(byte >> 4) - 8) * sc;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Whole-model decode step, sunnynet/runtime/sunnynet.c. */

#define ORC_SN_MAGIC 0x4E4E5355

typedef struct {
    const float *ni_g, *ni_c, *nm_g, *nm_c, *dw, *delta;
    float *V, *U, *Wz, *Wc, *Ws;   /* row-major (out,in), owned */
    float a_tanh, b_gain;
} OrcLayer;

struct OrcSn {
    int vocab, D, I, R, K, L, G, tied, clamp, batch, kh;
    float eps, p_floor;
    float* blob;                   /* owned copy of the fp32 payload */
    OrcLayer* layers;
    const float *no_g, *no_c, *embed;
    float* head;                   /* (vocab, D), owned */
    float* s;                      /* (batch, L, D) */
    float* hist;                   /* (batch, L, kh, D), [.,.,0,:] newest */
    float* sc;                     /* per-layer scratch */
    float* top;                    /* x, lout, nrm */
};

/* sunnynet.c:123-138: y[j] = sum_i W[j,i] x[i]; eight FMA lanes over i, lane
 * k holds i = k mod 8, then t0+t1+...+t7 left to right, then the scalar tail
 * with two roundings. Rows are independent, so threading is value-neutral. */
static void sn_gemv(float* y, const float* x, const float* W, int in, int out) {
    #pragma omp parallel for schedule(static)
    for (int j = 0; j < out; ++j) {
        const float* row = W + (size_t)j * in;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int i = 0;
        for (; i + 8 <= in; i += 8)
            for (int k = 0; k < 8; ++k) acc[k] = fmaf(row[i + k], x[i + k], acc[k]);
        float s = acc[0];
        for (int k = 1; k < 8; ++k) s = s + acc[k];
        for (; i < in; ++i) s = s + row[i] * x[i];
        y[j] = s;
    }
}

static float sgnf(float x) { return 1.0f / (1.0f + expf(-x)); }

/* sunnynet.c:198-210: two-pass mean / variance, rstd = 1/sqrt(var + eps). */
static void sn_layernorm(float* y, const float* x, const float* g,
                         const float* c, int n, float eps) {
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) sum = sum + x[i];
    const float mean = sum / (float)n;
    float vsum = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float d = x[i] - mean;
        vsum = vsum + d * d;
    }
    const float rstd = 1.0f / sqrtf(vsum / (float)n + eps);
    for (int i = 0; i < n; ++i) y[i] = (x[i] - mean) * rstd * g[i] + c[i];
}

/* (in,out) row-major block -> (out,in) row-major copy (sunnynet.c:170-194). */
static float* flip_copy(const float* src, int in, int out) {
    float* dst = (float*)malloc(sizeof(float) * (size_t)in * out);
    if (!dst) return NULL;
    #pragma omp parallel for schedule(static)
    for (int j = 0; j < out; ++j)
        for (int i = 0; i < in; ++i) dst[(size_t)j * in + i] = src[(size_t)i * out + j];
    return dst;
}

/* sunnynet.c:212-291 for one sequence. */
static void sn_layer_step(OrcSn* m, int l, float* s_l, float* hist_l,
                          const float* x, float* out, float* dbg) {
    const OrcLayer* L = &m->layers[l];
    const int D = m->D, I = m->I, R = m->R, K = m->K, G = m->G;
    float* raw = m->sc;
    float* at = raw + D;
    float* v = at + D;
    float* q = v + R;
    float* u = q + 2 * D;
    float* gate = u + D;
    float* zn = gate + D;
    float* yn = zn + I;
    float* sfb = yn + I;

    sn_layernorm(raw, x, L->ni_g, L->ni_c, D, m->eps);
    if (K > 1) {
        for (int i = 0; i < D; ++i) {
            float acc = raw[i] * L->dw[(size_t)(K - 1) * D + i];
            for (int k = 0; k < K - 1; ++k)
                acc = acc + hist_l[(size_t)k * D + i] * L->dw[(size_t)(K - 2 - k) * D + i];
            at[i] = raw[i] + acc;
        }
        for (int k = K - 2; k >= 1; --k)
            memcpy(hist_l + (size_t)k * D, hist_l + (size_t)(k - 1) * D, sizeof(float) * D);
        memcpy(hist_l, raw, sizeof(float) * D);
    } else {
        memcpy(at, raw, sizeof(float) * D);
    }

    sn_gemv(v, at, L->V, D, R);
    sn_gemv(q, v, L->U, R, 2 * D);
    memcpy(u, q, sizeof(float) * D);
    memcpy(gate, q + D, sizeof(float) * D);
    for (int i = 0; i < D; ++i) {
        const int base = (i / G) * G, off = i - base;
        u[i] = u[i] * (sgnf(gate[i] - gate[base + (off + 1) % G]) *
                       sgnf(gate[i] - gate[base + (off + 2) % G]));
    }
    sn_gemv(sfb, s_l, L->Ws, D, D);      /* uses the state before the update */
    for (int i = 0; i < D; ++i) {
        float p = 1.0f - L->delta[i] * (1.0f - sgnf(gate[i]));
        if (m->clamp && p < m->p_floor) p = m->p_floor;
        s_l[i] = p * s_l[i] + (1.0f - p) * u[i];
    }
    sn_gemv(zn, u, L->Wz, D, I);
    for (int i = 0; i < I; ++i)
        zn[i] = zn[i] * (1.0f + 0.5f * L->a_tanh / (1.0f + fabsf(zn[i])));
    sn_layernorm(yn, zn, L->nm_g, L->nm_c, I, m->eps);
    sn_gemv(out, yn, L->Wc, I, D);
    for (int i = 0; i < D; ++i) out[i] = out[i] + (L->b_gain * s_l[i] + sfb[i] + x[i]);

    if (dbg) {
        float* t = dbg;
        memcpy(t, raw, sizeof(float) * D); t += D;
        memcpy(t, at, sizeof(float) * D); t += D;
        memcpy(t, v, sizeof(float) * R); t += R;
        memcpy(t, gate, sizeof(float) * D); t += D;
        memcpy(t, u, sizeof(float) * D); t += D;
        memcpy(t, s_l, sizeof(float) * D); t += D;
        memcpy(t, zn, sizeof(float) * I); t += I;
        memcpy(t, yn, sizeof(float) * I); t += I;
        memcpy(t, sfb, sizeof(float) * D); t += D;
        memcpy(t, out, sizeof(float) * D);
    }
}

void orc_sn_free(OrcSn* m) {
    if (!m) return;
    if (m->layers) {
        for (int l = 0; l < m->L; ++l) {
            free(m->layers[l].V); free(m->layers[l].U); free(m->layers[l].Wz);
            free(m->layers[l].Wc); free(m->layers[l].Ws);
        }
    }
    free(m->layers); free(m->blob); free(m->head);
    free(m->s); free(m->hist); free(m->sc); free(m->top);
    free(m);
}

/* Parses the layout of experiments/_export_runtime.py:3-17 as read by
 * sunnynet.c:358-454, with size checks the reference leaves out. */
OrcSn* orc_sn_new(const void* blob, int64_t nbytes, int batch) {
    if (!blob || nbytes < 40 || batch <= 0) return NULL;
    int32_t h[10];
    memcpy(h, blob, sizeof h);
    if (h[0] != ORC_SN_MAGIC) return NULL;
    const int V = h[1], D = h[2], I = h[3], R = h[4], K = h[5], L = h[6];
    if (V <= 0 || D <= 0 || I <= 0 || R <= 0 || K <= 0 || L <= 0 || h[7] <= 0) return NULL;
    const size_t per_layer = (size_t)2 * D + (size_t)2 * I + (size_t)K * D +
                             (size_t)D * R + (size_t)R * 2 * D + (size_t)D * I +
                             (size_t)I * D + (size_t)D * D + D + 2;
    const size_t total = (size_t)L * per_layer + 2 + 2 * (size_t)D +
                         (size_t)V * D + (size_t)D * V;
    if ((size_t)nbytes != 40 + total * sizeof(float)) return NULL;

    OrcSn* m = (OrcSn*)calloc(1, sizeof(OrcSn));
    if (!m) return NULL;
    m->vocab = V; m->D = D; m->I = I; m->R = R; m->K = K; m->L = L;
    m->G = h[7]; m->tied = h[8]; m->clamp = h[9]; m->batch = batch;
    m->kh = K > 1 ? K - 1 : 0;
    m->blob = (float*)malloc(total * sizeof(float));
    m->layers = (OrcLayer*)calloc((size_t)L, sizeof(OrcLayer));
    if (!m->blob || !m->layers) { orc_sn_free(m); return NULL; }
    memcpy(m->blob, (const char*)blob + 40, total * sizeof(float));

    const float* p = m->blob;
    for (int l = 0; l < L; ++l) {
        OrcLayer* A = &m->layers[l];
        A->ni_g = p; p += D;
        A->ni_c = p; p += D;
        A->nm_g = p; p += I;
        A->nm_c = p; p += I;
        A->dw = p; p += (size_t)K * D;
        A->V = flip_copy(p, D, R); p += (size_t)D * R;
        A->U = flip_copy(p, R, 2 * D); p += (size_t)R * 2 * D;
        A->Wz = flip_copy(p, D, I); p += (size_t)D * I;
        A->Wc = flip_copy(p, I, D); p += (size_t)I * D;
        A->Ws = flip_copy(p, D, D); p += (size_t)D * D;
        A->delta = p; p += D;
        A->a_tanh = p[0]; A->b_gain = p[1]; p += 2;
        if (!A->V || !A->U || !A->Wz || !A->Wc || !A->Ws) { orc_sn_free(m); return NULL; }
    }
    m->eps = p[0]; m->p_floor = p[1]; p += 2;
    m->no_g = p; p += D;
    m->no_c = p; p += D;
    m->embed = p; p += (size_t)V * D;
    m->head = flip_copy(p, D, V);
    m->s = (float*)calloc((size_t)batch * L * D, sizeof(float));
    m->hist = (float*)calloc((size_t)batch * L * (m->kh ? m->kh : 1) * D, sizeof(float));
    m->sc = (float*)calloc((size_t)9 * D + R + 2 * (size_t)I, sizeof(float));
    m->top = (float*)calloc((size_t)3 * D, sizeof(float));
    if (!m->head || !m->s || !m->hist || !m->sc || !m->top) { orc_sn_free(m); return NULL; }
    return m;
}

void orc_sn_reset(OrcSn* m) {
    if (!m) return;
    memset(m->s, 0, sizeof(float) * (size_t)m->batch * m->L * m->D);
    memset(m->hist, 0, sizeof(float) * (size_t)m->batch * m->L * (m->kh ? m->kh : 1) * m->D);
}

void orc_sn_dims(const OrcSn* m, int32_t* hdr) {
    hdr[0] = m->vocab; hdr[1] = m->D; hdr[2] = m->I; hdr[3] = m->R; hdr[4] = m->K;
    hdr[5] = m->L; hdr[6] = m->G; hdr[7] = m->tied; hdr[8] = m->clamp; hdr[9] = m->batch;
}

/* sunnynet.c:321-334 for sequence b. */
void orc_sn_step_one(OrcSn* m, int b, int32_t token, float* logits) {
    const int D = m->D, L = m->L;
    float* x = m->top;
    float* lout = x + D;
    float* nrm = lout + D;
    memcpy(x, m->embed + (size_t)token * D, sizeof(float) * D);
    for (int l = 0; l < L; ++l) {
        float* s_l = m->s + ((size_t)b * L + l) * D;
        float* h_l = m->hist + ((size_t)b * L + l) * (size_t)m->kh * D;
        sn_layer_step(m, l, s_l, h_l, x, lout, NULL);
        memcpy(x, lout, sizeof(float) * D);
    }
    sn_layernorm(nrm, x, m->no_g, m->no_c, D, m->eps);
    sn_gemv(logits, nrm, m->head, D, m->vocab);
}

void orc_sn_step(OrcSn* m, const int32_t* tokens, float* logits) {
    for (int b = 0; b < m->batch; ++b)
        orc_sn_step_one(m, b, tokens[b], logits + (size_t)b * m->vocab);
}

void orc_sn_get_state(const OrcSn* m, float* s, float* hist) {
    memcpy(s, m->s, sizeof(float) * (size_t)m->batch * m->L * m->D);
    if (m->kh) memcpy(hist, m->hist, sizeof(float) * (size_t)m->batch * m->L * m->kh * m->D);
}

void orc_sn_set_state(OrcSn* m, const float* s, const float* hist) {
    memcpy(m->s, s, sizeof(float) * (size_t)m->batch * m->L * m->D);
    if (m->kh) memcpy(m->hist, hist, sizeof(float) * (size_t)m->batch * m->L * m->kh * m->D);
}

/* sunnynet.c:336-345 for sequence b. */
void orc_sn_dbg_layer(OrcSn* m, int b, int32_t token, int layer, float* dbg) {
    const int D = m->D, L = m->L;
    float* x = m->top;
    float* lout = x + D;
    memcpy(x, m->embed + (size_t)token * D, sizeof(float) * D);
    for (int l = 0; l <= layer && l < L; ++l) {
        float* s_l = m->s + ((size_t)b * L + l) * D;
        float* h_l = m->hist + ((size_t)b * L + l) * (size_t)m->kh * D;
        sn_layer_step(m, l, s_l, h_l, x, lout, l == layer ? dbg : NULL);
        memcpy(x, lout, sizeof(float) * D);
    }
}
