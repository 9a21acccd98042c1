/* CPU oracle for the RWKV-7 matrix-state decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see sn_oracle.h). Restates
 * sunnynet/runtime/rwkv7.c:89-360 (fp32 path) in scalar ISO C with the same
 * operation order. INT4-tagged matrices in a v3 blob are dequantized at load
 * with quant.c's formula and then run through the fp32 path, which is the
 * W4A32 semantics the HIP backend implements.
 */
#include "sn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_RK_MAGIC 0x4B57524B
#define ORC_RK_VERSION 3
#define ORC_R2 0.6065306597126334f   /* 1/sqrt(e), rwkv7.c:33 */
#define ORC_EPS_GROUP 6.4e-4f        /* rwkv7.c:34 */

typedef struct { int in, out; float* w; } OrcMat;   /* fp32 (in,out), owned */

typedef struct {
    int Rw, Ra, Rv, Rg, first;
    const float *ln1w, *ln1b, *ln2w, *ln2b, *lerp;
    OrcMat rw, kw, vw, ow, w1, w2, a1, a2, v1, v2, g1, g2, cmk, cmv;
    const float *w0, *a0, *v0, *kk_w, *ka_w, *rk_w, *lnx_w, *lnx_b, *cmk_lerp;
} OrcRkLayer;

struct OrcRk {
    int L, D, HS, NH, F, vocab, q4, batch;
    float eps;
    unsigned char* buf;            /* owned copy of the tagged payload */
    OrcRkLayer* layers;
    const float *en_w, *en_b, *on_w, *on_b, *embed;
    OrcMat head;
    float* S;                      /* (batch, L, NH, HS, HS) */
    float* shift;                  /* (batch, L, 2, D) */
    float* sc;
    float* top;
};

/* rwkv7.c:89-121: y = Wt^T x with Wt (in,out); each output accumulates
 * fma(x[i], Wt[i][j], acc) sequentially over i. The scalar column tail
 * (out % 8) uses two roundings (rwkv7.c:115-120). */
static void rk_gemv(float* y, const float* x, const OrcMat* M) {
    const int in = M->in, out = M->out, o8 = out & ~7;
    const float* Wt = M->w;
    #pragma omp parallel for schedule(static) if (out >= 1024)
    for (int j = 0; j < out; ++j) {
        float acc = 0.0f;
        if (j < o8) {
            for (int i = 0; i < in; ++i) acc = fmaf(x[i], Wt[(size_t)i * out + j], acc);
        } else {
            for (int i = 0; i < in; ++i) acc = acc + x[i] * Wt[(size_t)i * out + j];
        }
        y[j] = acc;
    }
}

static float sgnf(float x) { return 1.0f / (1.0f + expf(-x)); }

void orc_libm(const float* x, float* e, float* t, int64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        e[i] = expf(x[i]);
        t[i] = tanhf(x[i]);
    }
}

static void rk_layernorm(float* y, const float* x, const float* g,
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

/* rwkv7.c:77-84: ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)). */
static float hsum8(const float* v) {
    const float c0 = v[0] + v[4], c1 = v[1] + v[5], c2 = v[2] + v[6], c3 = v[3] + v[7];
    return (c0 + c1) + (c2 + c3);
}

/* rwkv7.c:143-189 for one head; HS is a multiple of 8. */
static void rk_head(int HS, float* Sh, const float* w, const float* k,
                    const float* v, const float* a, const float* kk,
                    const float* r, float* y, float* buf) {
    float ss[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < HS; j += 8)
        for (int q = 0; q < 8; ++q) ss[q] = fmaf(kk[j + q], kk[j + q], ss[q]);
    float nrm = sqrtf(hsum8(ss));
    if (!(nrm > 1e-12f)) nrm = 1e-12f;
    const float inv = 1.0f / nrm;
    for (int j = 0; j < HS; ++j) buf[j] = kk[j] * inv;
    for (int i = 0; i < HS; ++i) {
        float* row = Sh + (size_t)i * HS;
        float proj[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < HS; j += 8)
            for (int q = 0; q < 8; ++q) proj[q] = fmaf(row[j + q], buf[j + q], proj[q]);
        const float pv = hsum8(proj);
        const float vi = v[i];
        float yacc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < HS; j += 8)
            for (int q = 0; q < 8; ++q) {
                const float kka = buf[j + q] * a[j + q];
                const float vk = vi * k[j + q];
                const float ns = fmaf(row[j + q], w[j + q], vk - pv * kka);
                row[j + q] = ns;
                yacc[q] = fmaf(ns, r[j + q], yacc[q]);
            }
        y[i] = hsum8(yacc);
    }
}

/* rwkv7.c:191-320 for one sequence. */
static void rk_layer(OrcRk* m, const OrcRkLayer* L, float* S, float* shift,
                     float* x, float* vfirst) {
    const int D = m->D, HS = m->HS, NH = m->NH, F = m->F;
    float* xn = m->sc;
    float* dd = xn + D;
    float *xr = dd + D, *xw = xr + D, *xk = xw + D, *xv = xk + D, *xa = xv + D, *xg = xa + D;
    float* r = xg + D;
    float* k = r + D;
    float* v = k + D;
    float* a = v + D;
    float* g = a + D;
    float* kk = g + D;
    float* ww = kk + D;
    float* y = ww + D;
    float* xn2 = y + D;
    float* xk2 = xn2 + D;
    float* lo = xk2 + D;
    float* ck = lo + 256;
    float* cksq = ck + F;
    float* hbuf = cksq + F;

    rk_layernorm(xn, x, L->ln1w, L->ln1b, D, m->eps);
    for (int i = 0; i < D; ++i) dd[i] = shift[i] - xn[i];
    const float* lp = L->lerp;
    for (int i = 0; i < D; ++i) {
        const float d = dd[i];
        xr[i] = xn[i] + lp[i] * d;
        xw[i] = xn[i] + lp[D + i] * d;
        xk[i] = xn[i] + lp[2 * D + i] * d;
        xv[i] = xn[i] + lp[3 * D + i] * d;
        xa[i] = xn[i] + lp[4 * D + i] * d;
        xg[i] = xn[i] + lp[5 * D + i] * d;
    }
    rk_gemv(r, xr, &L->rw);
    rk_gemv(k, xk, &L->kw);
    rk_gemv(v, xv, &L->vw);

    rk_gemv(lo, xw, &L->w1);
    for (int i = 0; i < L->Rw; ++i) lo[i] = tanhf(lo[i]);
    rk_gemv(dd, lo, &L->w2);
    for (int i = 0; i < D; ++i) ww[i] = expf(-sgnf(dd[i] + L->w0[i]) * ORC_R2);

    if (L->first) {
        memcpy(vfirst, v, sizeof(float) * D);
    } else {
        rk_gemv(lo, xv, &L->v1);
        rk_gemv(dd, lo, &L->v2);
        for (int i = 0; i < D; ++i) {
            const float mix = sgnf(dd[i] + L->v0[i]);
            v[i] = v[i] + (vfirst[i] - v[i]) * mix;
        }
    }
    rk_gemv(lo, xa, &L->a1);
    rk_gemv(dd, lo, &L->a2);
    for (int i = 0; i < D; ++i) a[i] = sgnf(dd[i] + L->a0[i]);
    rk_gemv(lo, xg, &L->g1);
    for (int i = 0; i < L->Rg; ++i) lo[i] = sgnf(lo[i]);
    rk_gemv(g, lo, &L->g2);
    for (int i = 0; i < D; ++i) {
        kk[i] = k[i] * L->kk_w[i];
        k[i] = k[i] + k[i] * (a[i] - 1.0f) * L->ka_w[i];
    }
    for (int h = 0; h < NH; ++h)
        rk_head(HS, S + (size_t)h * HS * HS, ww + h * HS, k + h * HS, v + h * HS,
                a + h * HS, kk + h * HS, r + h * HS, y + h * HS, hbuf);
    for (int h = 0; h < NH; ++h) {
        float* yh = y + (size_t)h * HS;
        const float* rh = r + (size_t)h * HS;
        const float* kh = k + (size_t)h * HS;
        const float* vh = v + (size_t)h * HS;
        const int base = h * HS;
        float mean = 0.0f;
        for (int i = 0; i < HS; ++i) mean = mean + yh[i];
        mean = mean / (float)HS;
        float var = 0.0f;
        for (int i = 0; i < HS; ++i) {
            const float t = yh[i] - mean;
            var = var + t * t;
        }
        const float rstd = 1.0f / sqrtf(var / (float)HS + ORC_EPS_GROUP);
        float dot = 0.0f;
        for (int i = 0; i < HS; ++i) dot = dot + rh[i] * kh[i] * L->rk_w[base + i];
        for (int i = 0; i < HS; ++i) {
            const float n = (yh[i] - mean) * rstd * L->lnx_w[base + i] + L->lnx_b[base + i];
            yh[i] = (n + dot * vh[i]) * g[base + i];
        }
    }
    rk_gemv(dd, y, &L->ow);
    for (int i = 0; i < D; ++i) x[i] = x[i] + dd[i];
    memcpy(shift, xn, sizeof(float) * D);

    rk_layernorm(xn2, x, L->ln2w, L->ln2b, D, m->eps);
    for (int i = 0; i < D; ++i)
        xk2[i] = xn2[i] + L->cmk_lerp[i] * (shift[D + i] - xn2[i]);
    rk_gemv(ck, xk2, &L->cmk);
    for (int i = 0; i < F; ++i) {
        const float t = ck[i] > 0.0f ? ck[i] : 0.0f;
        ck[i] = t;
        cksq[i] = t * t;
    }
    rk_gemv(dd, cksq, &L->cmv);
    for (int i = 0; i < D; ++i) x[i] = x[i] + dd[i];
    memcpy(shift + D, xn2, sizeof(float) * D);
}

/* ---- loader: rwkv7.c:376-508 with bounds checks ---- */
typedef struct { const unsigned char* p; const unsigned char* end; int ok; int block; } Cur;

static const float* take_f32(Cur* c, size_t n) {
    if (!c->ok || (size_t)(c->end - c->p) < 4 + n * sizeof(float)) { c->ok = 0; return NULL; }
    int32_t tag;
    memcpy(&tag, c->p, 4);
    if (tag != 0) { c->ok = 0; return NULL; }
    c->p += 4;
    const float* r = (const float*)c->p;
    c->p += n * sizeof(float);
    return r;
}

static void take_mat(Cur* c, OrcMat* M, int in, int out) {
    M->in = in; M->out = out; M->w = NULL;
    if (!c->ok || c->end - c->p < 4) { c->ok = 0; return; }
    int32_t tag;
    memcpy(&tag, c->p, 4);
    c->p += 4;
    M->w = (float*)malloc(sizeof(float) * (size_t)in * out);
    if (!M->w) { c->ok = 0; return; }
    if (tag == 1) {
        const int block = c->block;
        if (in % block) { c->ok = 0; return; }
        const size_t qb = (size_t)out * (size_t)(in / 2);
        const size_t sb = (size_t)out * (size_t)(in / block) * sizeof(float);
        if ((size_t)(c->end - c->p) < qb + sb) { c->ok = 0; return; }
        float* W = (float*)malloc(sizeof(float) * (size_t)in * out);
        float* sc = (float*)malloc(sb);
        if (!W || !sc) { free(W); free(sc); c->ok = 0; return; }
        memcpy(sc, c->p + qb, sb);   /* scales may be unaligned in the stream */
        orc_dequant_i4(c->p, sc, W, out, in, block);
        for (int j = 0; j < out; ++j)
            for (int i = 0; i < in; ++i) M->w[(size_t)i * out + j] = W[(size_t)j * in + i];
        free(W); free(sc);
        c->p += qb + sb;
    } else if (tag == 0) {
        const size_t nb = (size_t)in * out * sizeof(float);
        if ((size_t)(c->end - c->p) < nb) { c->ok = 0; return; }
        memcpy(M->w, c->p, nb);
        c->p += nb;
    } else {
        c->ok = 0;
    }
}

static void free_mat(OrcMat* M) { free(M->w); M->w = NULL; }

void orc_rk_free(OrcRk* m) {
    if (!m) return;
    if (m->layers) {
        for (int l = 0; l < m->L; ++l) {
            OrcRkLayer* A = &m->layers[l];
            OrcMat* ms[14] = {&A->rw, &A->kw, &A->vw, &A->ow, &A->w1, &A->w2, &A->a1,
                              &A->a2, &A->v1, &A->v2, &A->g1, &A->g2, &A->cmk, &A->cmv};
            for (int i = 0; i < 14; ++i) free_mat(ms[i]);
        }
    }
    free_mat(&m->head);
    free(m->layers); free(m->buf); free(m->S); free(m->shift); free(m->sc); free(m->top);
    free(m);
}

OrcRk* orc_rk_new(const void* blob, int64_t nbytes, int batch, int block) {
    if (!blob || nbytes < 44 || batch <= 0 || block <= 0 || (block & 1)) return NULL;
    int32_t h[10];
    memcpy(h, blob, sizeof h);
    if (h[0] != ORC_RK_MAGIC || h[1] != ORC_RK_VERSION) return NULL;
    const int L = h[2], D = h[3], HS = h[4], NH = h[5], F = h[6], vocab = h[8];
    if (L <= 0 || D <= 0 || HS <= 0 || HS % 8 || NH * HS != D || F <= 0 || vocab <= 0)
        return NULL;
    const unsigned char* p = (const unsigned char*)blob + 40;
    const unsigned char* end = (const unsigned char*)blob + nbytes;
    float eps;
    memcpy(&eps, p, 4);
    p += 4;
    if ((size_t)(end - p) < (size_t)16 * L) return NULL;
    int32_t* ranks = (int32_t*)malloc(sizeof(int32_t) * 4 * (size_t)L);
    if (!ranks) return NULL;
    memcpy(ranks, p, sizeof(int32_t) * 4 * (size_t)L);
    p += 16 * (size_t)L;

    OrcRk* m = (OrcRk*)calloc(1, sizeof(OrcRk));
    if (!m) { free(ranks); return NULL; }
    m->L = L; m->D = D; m->HS = HS; m->NH = NH; m->F = F; m->vocab = vocab;
    m->q4 = h[9]; m->batch = batch; m->eps = eps;
    const size_t nrest = (size_t)(end - p);
    m->buf = (unsigned char*)malloc(nrest ? nrest : 1);
    m->layers = (OrcRkLayer*)calloc((size_t)L, sizeof(OrcRkLayer));
    if (!m->buf || !m->layers) { free(ranks); orc_rk_free(m); return NULL; }
    memcpy(m->buf, p, nrest);
    Cur c = {m->buf, m->buf + nrest, 1, block};
    for (int l = 0; l < L; ++l) {
        OrcRkLayer* A = &m->layers[l];
        A->first = (l == 0);
        A->Rw = ranks[4 * l]; A->Ra = ranks[4 * l + 1];
        A->Rv = ranks[4 * l + 2]; A->Rg = ranks[4 * l + 3];
        if (A->Rw <= 0 || A->Ra <= 0 || A->Rv <= 0 || A->Rg <= 0 ||
            A->Rw > 256 || A->Ra > 256 || A->Rv > 256 || A->Rg > 256) c.ok = 0;
        A->ln1w = take_f32(&c, D);
        A->ln1b = take_f32(&c, D);
        A->ln2w = take_f32(&c, D);
        A->ln2b = take_f32(&c, D);
        A->lerp = take_f32(&c, (size_t)6 * D);
        take_mat(&c, &A->rw, D, D);
        take_mat(&c, &A->kw, D, D);
        take_mat(&c, &A->vw, D, D);
        take_mat(&c, &A->ow, D, D);
        take_mat(&c, &A->w1, D, A->Rw);
        take_mat(&c, &A->w2, A->Rw, D);
        take_mat(&c, &A->a1, D, A->Ra);
        take_mat(&c, &A->a2, A->Ra, D);
        take_mat(&c, &A->v1, D, A->Rv);
        take_mat(&c, &A->v2, A->Rv, D);
        take_mat(&c, &A->g1, D, A->Rg);
        take_mat(&c, &A->g2, A->Rg, D);
        A->w0 = take_f32(&c, D);
        A->a0 = take_f32(&c, D);
        A->v0 = take_f32(&c, D);
        A->kk_w = take_f32(&c, D);
        A->ka_w = take_f32(&c, D);
        A->rk_w = take_f32(&c, D);
        A->lnx_w = take_f32(&c, D);
        A->lnx_b = take_f32(&c, D);
        take_mat(&c, &A->cmk, D, F);
        take_mat(&c, &A->cmv, F, D);
        A->cmk_lerp = take_f32(&c, D);
    }
    m->en_w = take_f32(&c, D);
    m->en_b = take_f32(&c, D);
    m->on_w = take_f32(&c, D);
    m->on_b = take_f32(&c, D);
    m->embed = take_f32(&c, (size_t)vocab * D);
    take_mat(&c, &m->head, D, vocab);
    free(ranks);
    if (!c.ok) { orc_rk_free(m); return NULL; }
    m->S = (float*)calloc((size_t)batch * L * NH * HS * HS, sizeof(float));
    m->shift = (float*)calloc((size_t)batch * L * 2 * D, sizeof(float));
    m->sc = (float*)calloc((size_t)18 * D + 256 + 2 * (size_t)F + 8 + HS, sizeof(float));
    m->top = (float*)calloc((size_t)3 * D, sizeof(float));
    if (!m->S || !m->shift || !m->sc || !m->top) { orc_rk_free(m); return NULL; }
    return m;
}

void orc_rk_reset(OrcRk* m) {
    if (!m) return;
    memset(m->S, 0, sizeof(float) * (size_t)m->batch * m->L * m->NH * m->HS * m->HS);
    memset(m->shift, 0, sizeof(float) * (size_t)m->batch * m->L * 2 * m->D);
}

void orc_rk_dims(const OrcRk* m, int32_t* hdr) {
    hdr[0] = m->L; hdr[1] = m->D; hdr[2] = m->HS; hdr[3] = m->NH;
    hdr[4] = m->F; hdr[5] = m->vocab; hdr[6] = m->q4; hdr[7] = m->batch;
}

/* rwkv7.c:349-360 for sequence b. */
void orc_rk_step_one(OrcRk* m, int b, int32_t token, float* logits) {
    const int D = m->D, L = m->L;
    const size_t sl = (size_t)m->NH * m->HS * m->HS;
    float* x = m->top;
    float* nrm = x + D;
    float* vfirst = nrm + D;
    memcpy(x, m->embed + (size_t)token * D, sizeof(float) * D);
    rk_layernorm(x, x, m->en_w, m->en_b, D, m->eps);
    for (int l = 0; l < L; ++l)
        rk_layer(m, &m->layers[l], m->S + ((size_t)b * L + l) * sl,
                 m->shift + ((size_t)b * L + l) * 2 * D, x, vfirst);
    rk_layernorm(nrm, x, m->on_w, m->on_b, D, m->eps);
    rk_gemv(logits, nrm, &m->head);
}

void orc_rk_step(OrcRk* m, const int32_t* tokens, float* logits) {
    for (int b = 0; b < m->batch; ++b)
        orc_rk_step_one(m, b, tokens[b], logits + (size_t)b * m->vocab);
}

void orc_rk_get_state(const OrcRk* m, float* S, float* shift) {
    memcpy(S, m->S, sizeof(float) * (size_t)m->batch * m->L * m->NH * m->HS * m->HS);
    memcpy(shift, m->shift, sizeof(float) * (size_t)m->batch * m->L * 2 * m->D);
}

void orc_rk_set_state(OrcRk* m, const float* S, const float* shift) {
    memcpy(m->S, S, sizeof(float) * (size_t)m->batch * m->L * m->NH * m->HS * m->HS);
    memcpy(m->shift, shift, sizeof(float) * (size_t)m->batch * m->L * 2 * m->D);
}
