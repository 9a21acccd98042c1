// Persistent decode step for a batch of sequences: every layer of one step in
// one cooperative launch (the batched path of snhip_step_batch_dev /
// snhip_decode_greedy_dev from 3 sequences up).
//
// The math is the decode step of sunnynet/runtime/sunnynet.c:212-334 for each
// sequence. Per layer the grid walks through five phases:
//
//   P0  at = LN_in(x) + conv(history) per sequence row; history shifted
//   P1  v = V at and sfb = W_eff s (V's rows then W_eff's, one storage)
//   P2  q = U v per channel group, competitive + decay gate, new state s'
//   P3  z = wedge(W_z u)
//   P4  x' = W_c LN_mid(z) + b s' + sfb + x   (LayerNorm in the tile prologue)
//
// and after the last layer the final LayerNorm of every row (the head's
// input). Products are 16 x 16 output tiles (16 sequence rows x 16 weight
// rows): the workgroup's 8 waves split K into 64-wide chunks, lane (r, q)
// holds 16 consecutive k of X row m0 + r and weight row n0 + r, and
// v_mfma_f32_16x16x4f32 number j multiplies component j of both, so a chunk's
// 16 MFMAs cover its 64 k once; the waves' tiles are summed through LDS in wave
// order. A workgroup takes tiles wg, wg + G, ...; the weights of its first tile
// in the next product are loaded once its tiles of the current one are done
// (they depend on nothing the waits order), and those of its next tile while
// it multiplies the current one.
//
// Dataflow instead of grid barriers. Every row of P0 and every tile of P1-P4
// has a flag word per layer; once the writer's stores (agent-coherent, sc1)
// have completed, its thread 0 stores the launch's epoch there (agent scope),
// and a tile waits only for the flags of what it reads:
//
//   P0 row b       the x' tiles of b's row block (layer l - 1)
//   P1 V tile      the 16 rows of at of its row block (W_eff tiles: nothing;
//                  s is the previous step's)
//   P2 tile        the V tiles of its row block (all of v)
//   P3 tile        the P2 tiles of its row block (all of u)
//   P4 tile        the P3 tiles (all of z) and the W_eff tiles of its row
//                  block: after those every reader of the old s rows it
//                  overwrites is done (P2's readers precede P3)
//
// and the final LayerNorm of row b the last layer's x' tiles of its block.
// Every wait is on an earlier phase (or layer), so with every workgroup
// resident the launch always drains. Every phase writes its outputs to a
// buffer no other phase of the launch writes (per-layer slabs of at, v, sfb,
// u, z, s', x), and every reader of a row waits for all of the row's writers,
// so no XCD holds a line of it from earlier in the launch and plain cached
// loads return the new values; the kernel boundary orders launch against
// launch. Flags are zeroed with the handle and epochs grow by one per launch;
// every poll is bounded (time-out -> error word -> every workgroup leaves at
// its next wait).
#include "decode.h"

namespace snhip {
namespace {

constexpr int NT = 512, NW = NT / 64, CH = 64, NCM = kBatchMaxK / (NW * CH), PERM = kBatchMaxRow / NT;
constexpr int kTaps = 4;
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;

__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }

// The same value, opaque to the optimizer: applied to the thread index at
// every tile so per-lane addresses are formed where they are used instead of
// being hoisted out of the layer loop (they would stay live and spill).
__device__ __forceinline__ int opq(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Store visible to every XCD once the wave's stores have completed.
__device__ __forceinline__ void st_ag(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Global-memory pointers. Pointers read from the LDS layer table are generic
// to the compiler, and generic (flat) loads also count against the LDS wait
// counter: the next LDS access would wait for a weight prefetch.
template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> glb(const T* p) { return (gptr<T>)p; }

struct Mat { const float* w; const uint8_t* q; const float* sc; int N, K; };

// Weight fragment of one 64-wide chunk: fp32 16 values, or INT4 16 codes
// (16 bytes holding two halves or quarters of a group) and the group's scale.
template <int BLK> struct WF;
template <> struct WF<0> { f4 b[4]; };
template <int BLK> struct WF { u4 q; float sc; };
struct XF { f4 a[4]; };

struct Tile { int n0, m0; };

// Tile t of a product with mb row blocks and nt weight tiles: when the weight
// tiles come in eights, the mb tiles that share one weight tile are t, t + 8,
// ... (the same workgroup residue mod 8, so the same XCD under round-robin
// dispatch) and read it from one L2.
__device__ __forceinline__ Tile tile_of(int t, int mb, int nt) {
    if (mb > 1 && (nt & 7) == 0) {
        const int x = t & 7, sl = t >> 3;
        return Tile{((sl / mb) * 8 + x) * 16, (sl % mb) * 16};
    }
    return Tile{(t / mb) * 16, (t % mb) * 16};
}

// Chunks of a product with nch chunks that wave wv multiplies: c = wv + NW i
// for i < NC. A chunk past the end (a product shorter than NW NC chunks)
// reads chunk 0 and contributes zero (its X values are cleared), so loads and
// MFMAs stay straight-line.
template <int BLK, int NC, bool FULL>
__device__ __forceinline__ void load_w(WF<BLK> (&f)[NCM], const Mat& W, int n0, int wv, int lane) {
    const int r = lane & 15, q = lane >> 4;
    const int nr = min(n0 + r, W.N - 1);
    const int nch = W.K / CH;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = FULL || wv + NW * i < nch ? wv + NW * i : 0;
        const int k0 = c * CH + 16 * q;
        if constexpr (BLK == 0) {
            const gptr<float> p = glb(W.w) + (size_t)nr * W.K + k0;
#pragma unroll
            for (int j = 0; j < 4; ++j) f[i].b[j] = *(gptr<f4>)(p + 4 * j);
        } else {
            // BLK 32: k0 opens the low (q even) or high (q odd) nibbles of
            // group k0 / 32's 16 bytes. BLK 64: quarter q of group k0 / 64 is
            // the low (q < 2) or high nibbles of bytes 16 (q & 1) .. + 15.
            const int grp = k0 / BLK;
            const size_t qo = (size_t)grp * (BLK / 2) + (BLK == 64 ? 16 * (q & 1) : 0);
            f[i].q = *(gptr<u4>)(glb(W.q) + (size_t)nr * (W.K / 2) + qo);
            f[i].sc = glb(W.sc)[(size_t)nr * (W.K / BLK) + grp];
        }
    }
}

// X rows m0 .. m0 + 15 (rows past B read row B - 1; their results are not
// stored). FULL: the product has exactly NW NC chunks (no chunk to clear).
template <int NC, bool FULL>
__device__ __forceinline__ void load_x(XF (&x)[NCM], const float* X, long ldx, int m0, int B, int K,
                                       int wv, int lane) {
    const int r = lane & 15, q = lane >> 4;
    const gptr<float> xr = glb(X) + (size_t)min(m0 + r, B - 1) * ldx;
    const int nch = K / CH;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const bool ok = FULL || wv + NW * i < nch;
        const int c = ok ? wv + NW * i : 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[i].a[j] = *(gptr<f4>)(xr + c * CH + 16 * q + 4 * j);
        if (!FULL) {
            // multiply, not select: keeps the loads in one block
            const float mk = ok ? 1.0f : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) x[i].a[j] *= mk;
        }
    }
    // every X load is issued before the first MFMA (one memory round trip)
    __builtin_amdgcn_sched_barrier(0);
}

template <int BLK, int NC>
__device__ __forceinline__ void mma(f4 (&acc)[4], const XF (&x)[NCM], const WF<BLK> (&w)[NCM], int lane) {
    const int q = lane >> 4;
    const int nshift = BLK == 32 ? 4 * (q & 1) : (BLK == 64 ? 4 * (q >> 1) : 0);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float a = x[i].a[j >> 2][j & 3];
            float b;
            if constexpr (BLK == 0) {
                b = w[i].b[j >> 2][j & 3];
            } else {
                // (q - 8) * scale: sn_dequant_i4's arithmetic (quant.c:82-83)
                b = (float)((int)((w[i].q[j >> 2] >> (8 * (j & 3) + nshift)) & 0xFu) - 8) * w[i].sc;
            }
            acc[j & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j & 3], 0, 0, 0);
        }
    }
}

// A pointer or value read from LDS, made wave-uniform (scalar registers).
template <class T>
__device__ __forceinline__ T* uni(T* p) {
    const unsigned long long v = (unsigned long long)p;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (T*)(((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ float uni(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// Sum of the waves' partial tiles in wave order into tile[16 * row + col].
__device__ __forceinline__ void tile_sum(const f4 (&acc)[4], float* red, float* tile, int wv, int lane,
                                         int tid) {
    const f4 t = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    const int r = lane & 15, q = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) red[wv * 256 + (4 * q + v) * 16 + r] = t[v];
    __syncthreads();
    if (tid < 256) {
        float s = red[tid];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[w * 256 + tid];
        tile[tid] = s;
    }
    __syncthreads();
}

// 512-thread block sum; red holds NW floats.
__device__ __forceinline__ float block_sum(float v, float* red, int wv, int lane) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if (lane == 0) red[wv] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) s += red[w];
    return s;
}

// Two-pass LayerNorm statistics (sunnynet.c:198-210 form) of one row of n
// values, element k * NT + tid in xv[k].
__device__ __forceinline__ void row_stats(const float (&xv)[PERM], int n, float eps, float* red, int tid,
                                          int wv, int lane, float& mean, float& rstd) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < PERM; ++k)
        if (k * NT + tid < n) sum += xv[k];
    mean = block_sum(sum, red, wv, lane) / (float)n;
    float vs = 0.0f;
#pragma unroll
    for (int k = 0; k < PERM; ++k)
        if (k * NT + tid < n) {
            const float d = xv[k] - mean;
            vs += d * d;
        }
    rstd = 1.0f / sqrtf(block_sum(vs, red, wv, lane) / (float)n + eps);
}

// Keeps the loads issued so far ahead of what follows (a compiler fence: the
// optimizer would otherwise sink a prefetch past the barrier wait to its use).
__device__ __forceinline__ void issued() { asm volatile("" ::: "memory"); }

// The writer's half: every wave's stores have completed, then thread 0
// publishes the epoch in flag f.
__device__ __forceinline__ void publish(unsigned* f, unsigned ep) {
    __builtin_amdgcn_s_waitcnt(0);          // this wave's stores have completed
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(f, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The writer's half for every tile this workgroup took in a product (tiles
// wg, wg + G, ... < T): one wait for all of their stores, then one flag each.
__device__ __forceinline__ void publish_tiles(unsigned* f, int wg, int G, int T, int mb, int N, unsigned ep) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int t = wg + (int)threadIdx.x * G;
    if (t < T) {
        const Tile tl = tile_of(t, mb, N);
        __hip_atomic_store(f + (size_t)(tl.m0 >> 4) * N + (tl.n0 >> 4), ep, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The reader's half: until each of the n flags f[0 .. n) holds `want`; true
// if the launch is abandoned (a wait timed out, here or in another
// workgroup).
__device__ __forceinline__ bool await(const unsigned* f, int n, unsigned want, unsigned* err, unsigned limit,
                                      int* sdead) {
    int dead = 0;
    for (int i = threadIdx.x; i < n && !dead; i += NT) {
        unsigned k = 0;
        while (__hip_atomic_load(const_cast<unsigned*>(f + i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != want) {
            if (++k > limit) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                dead = 1;
                break;
            }
            if ((k & 63) == 0 && __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                dead = 1;
                break;
            }
        }
    }
    if (dead) *sdead = 1;
    __syncthreads();
    return *sdead != 0;
}

#ifdef SNHIP_BATCH_PROF
// Profiling builds: wall-clock marks of thread 0 of workgroups 0, G / 2 and
// G - 1 for every phase (start, first tile done, products done, barrier entry).
__device__ unsigned long long g_bprof[3][5 * kPersistMaxL + 1][4];
#define BPROF(ph, k)                                                                          \
    do {                                                                                      \
        if (threadIdx.x == 0 && (wg == 0 || wg == G / 2 || wg == G - 1))                      \
            g_bprof[wg == 0 ? 0 : (wg == G - 1 ? 2 : 1)][ph][k] = wall_clock64();              \
    } while (0)
// Mark k of phase ph once this wave's loads have arrived (profiling only).
#define BPROF_LOADED(ph, k)                                                                   \
    do {                                                                                      \
        __builtin_amdgcn_s_waitcnt(0);                                                        \
        BPROF(ph, k);                                                                         \
    } while (0)
#else
#define BPROF(ph, k) do {} while (0)
#define BPROF_LOADED(ph, k) do {} while (0)
#endif

// NCD, NCR, NCI: chunks per wave of the products over dim, rank and inner.
template <int BLK, int NCD, int NCR, int NCI, bool FULL>
__global__ __launch_bounds__(NT) void k_decode_batch(BatchArgs a) {
    __shared__ float red[NW * 256];
    __shared__ float tile[256];
    __shared__ float lnp[2][NW * 16];          // LN_mid partial sums per wave and row
    __shared__ float gc[2 * kBatchMaxK];       // LN_mid gains and biases of the layer
    __shared__ float rred[NW];
    __shared__ int sdead;
    __shared__ PLayer ltab[kPersistMaxL];

    int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    auto fresh = [&]() {
        tid = opq(tid);
        lane = tid & 63;
    };
    const int wg = blockIdx.x, G = gridDim.x;
    const int B = a.B, D = a.D, I = a.I, R = a.R, L = a.L;
    const int mb = (B + 15) / 16;
    const size_t sbs = (size_t)L * D;                    // state row stride
    const size_t hbs = (size_t)L * a.kh * D;             // history row stride
    const unsigned ep = a.epoch, want = a.epoch + a.stall;
    // Layer 0's input row b: the embedding row of token b (NaN for an id
    // outside the vocabulary, as k_embed writes), later layers' the residual.
    auto in_row = [&](int l, int b, bool& ok) -> const float* {
        if (l > 0) {
            ok = true;
            return a.xs + ((size_t)(l - 1) * B + b) * D;
        }
        const int t = a.tok[b];
        ok = t >= 0 && t < a.vocab;
        return a.embed + (size_t)(ok ? t : 0) * D;
    };

    if (tid == 0) sdead = 0;
    for (int i = tid; i < L * (int)sizeof(PLayer) / 4; i += NT)
        reinterpret_cast<unsigned*>(ltab)[i] = reinterpret_cast<const unsigned*>(a.layers)[i];
    __syncthreads();

    auto mat = [&](const PMat& P, int N, int K) { return Mat{uni(P.w), uni(P.q), uni(P.sc), N, K}; };
    // Weight tiles and tiles of each product: (weight rows / 16) x mb.
    const int N1 = (R + D) / 16, N2 = (2 * D) / 16, N3 = I / 16, N4 = D / 16;
    const int T1 = N1 * mb, T2 = N2 * mb, T3 = N3 * mb, T4 = N4 * mb;
    // Flags of layer l, phase ph: P0 one per row, P1-P4 one per tile, by
    // (row block, weight tile).
    const size_t nfl = batch_flag_words(1, B, D, I, R);
    auto fl = [&](int l, int ph) -> unsigned* {
        unsigned* f = a.flags + (size_t)l * nfl;
        if (ph == 0) return f;
        f += B;
        if (ph == 1) return f;
        f += (size_t)mb * N1;
        if (ph == 2) return f;
        f += (size_t)mb * N2;
        if (ph == 3) return f;
        return f + (size_t)mb * N3;
    };
    auto wait = [&](const unsigned* f, int n) { return await(f, n, want, a.err, a.spin_limit, &sdead); };

    WF<BLK> wa[NCM];
    if (wg < T1) load_w<BLK, NCD, FULL>(wa, mat(ltab[0].VW, R + D, D), tile_of(wg, mb, N1).n0, wv, lane);

    for (int l = 0; l < L; ++l) {
        const PLayer* P = ltab + l;
        float* atl = a.at + (size_t)l * B * D;
        float* vl = a.v + (size_t)l * B * R;
        float* sfbl = a.sfb + (size_t)l * B * D;
        float* ul = a.u + (size_t)l * B * D;
        float* zl = a.z + (size_t)l * B * I;
        float* snl = a.sn + (size_t)l * B * D;
        float* xo = a.xs + (size_t)l * B * D;
        float* s_l = a.s + (size_t)l * D;

        // ---- P0: LN_in + conv of the rows this workgroup owns (sunnynet.c:216-237)
        BPROF(5 * l, 0);
        for (int b = wg; b < B; b += G) {
            fresh();
            // The row's history and the layer's gains and taps do not depend
            // on the wait: issued ahead of it.
            const gptr<float> ng = glb(uni(P->ni_g));
            const gptr<float> nc = glb(uni(P->ni_c));
            const gptr<float> dw = glb(uni(P->dw));
            float* hb = a.hist + (size_t)b * hbs + (size_t)l * a.kh * D;
            float xv[PERM], gv[PERM], cv[PERM], h[kTaps - 1][PERM], dv[kTaps][PERM], rv[PERM];
#pragma unroll
            for (int k = 0; k < PERM; ++k) {
                const int i = min(k * NT + tid, D - 1);
                gv[k] = ng[i];
                cv[k] = nc[i];
#pragma unroll
                for (int t = 0; t < kTaps - 1; ++t) h[t][k] = hb[(size_t)t * D + i];
#pragma unroll
                for (int t = 0; t < kTaps; ++t) dv[t][k] = dw[(size_t)t * D + i];
            }
            issued();
            if (l > 0 && wait(fl(l - 1, 4) + (size_t)(b >> 4) * N4, N4)) return;
            bool xok;
            const float* xr = in_row(l, b, xok);
#pragma unroll
            for (int k = 0; k < PERM; ++k) xv[k] = xok ? xr[min(k * NT + tid, D - 1)] : __builtin_nanf("");
            float mean, rstd;
            row_stats(xv, D, a.eps, rred, tid, wv, lane, mean, rstd);
#pragma unroll
            for (int k = 0; k < PERM; ++k) {
                const int i = k * NT + tid;
                const float raw = (xv[k] - mean) * rstd * gv[k] + cv[k];
                // acc = raw w[K-1] + hist[0] w[K-2] + hist[1] w[K-3] + hist[2] w[K-4]
                float acc = raw * dv[kTaps - 1][k];
#pragma unroll
                for (int t = 0; t < kTaps - 1; ++t) acc = acc + h[t][k] * dv[kTaps - 2 - t][k];
                if (i < D) st_ag(atl + (size_t)b * D + i, raw + acc);
                rv[k] = raw;
            }
            publish(fl(l, 0) + b, ep);
            // The history shift after the flag: P1 reads only `at`, and the
            // history is this workgroup's own until the next step.
#pragma unroll
            for (int k = 0; k < PERM; ++k) {
                const int i = k * NT + tid;
                if (i >= D) continue;
#pragma unroll
                for (int t = kTaps - 2; t >= 1; --t) hb[(size_t)t * D + i] = h[t - 1][k];
                hb[i] = rv[k];
            }
        }
        BPROF(5 * l, 2);
        BPROF(5 * l, 3);

        // ---- P1: v = V at (rows 0..R) and sfb = W_eff s_old (rows R..R+D)
        {
            const Mat W = mat(P->VW, R + D, D);
            BPROF(5 * l + 1, 0);
            int done_m = -1;                        // row block whose inputs are in
            for (int t = wg; t < T1; t += G) {
                fresh();
                const Tile tl = tile_of(t, mb, N1);
                XF x[NCM];
                const bool vrow = tl.n0 < R;            // V rows read at, W_eff rows s
                if (vrow && tl.m0 != done_m) {         // (a row block waited for once)
                    if (wait(fl(l, 0) + tl.m0, min(16, B - tl.m0))) return;
                    done_m = tl.m0;
                }
                load_x<NCD, FULL>(x, vrow ? atl : s_l, vrow ? (long)D : (long)sbs, tl.m0, B, D, wv, lane);
                if (t == wg) BPROF_LOADED(5 * l + 1, 1);
                f4 acc[4] = {};
                mma<BLK, NCD>(acc, x, wa, lane);
                if (t + G < T1) load_w<BLK, NCD, FULL>(wa, W, tile_of(t + G, mb, N1).n0, wv, lane);
                tile_sum(acc, red, tile, wv, lane, tid);
                if (t == wg) BPROF(5 * l + 1, 2);
                if (tid < 256) {
                    const int m = tl.m0 + (tid >> 4), n = tl.n0 + (tid & 15);
                    if (m < B) {
                        if (n < R) st_ag(vl + (size_t)m * R + n, tile[tid]);
                        else st_ag(sfbl + (size_t)m * D + (n - R), tile[tid]);
                    }
                }
            }
        }
        BPROF(5 * l + 1, 3);
        publish_tiles(fl(l, 1), wg, G, T1, mb, N1, ep);
        fresh();
        if (wg < T2) load_w<BLK, NCR, FULL>(wa, mat(P->U, 2 * D, R), tile_of(wg, mb, N2).n0, wv, lane);
        issued();

        // ---- P2: q = U v for channel group n0 / 16 (rows 0-7 values, 8-15
        // gates), competitive + decay gate, s' (sunnynet.c:248-266)
        {
            const Mat W = mat(P->U, 2 * D, R);
            const gptr<float> delta = glb(uni(P->delta));
            BPROF(5 * l + 2, 0);
            int done_m = -1;                        // row block whose inputs are in
            for (int t = wg; t < T2; t += G) {
                fresh();
                const Tile tl = tile_of(t, mb, N2);
                // epilogue operands first: thread o < 128 takes row o >> 3, channel o & 7
                const int em = tl.m0 + ((tid & 127) >> 3), ei = tl.n0 / 2 + (tid & 7);
                const bool eon = tid < 128 && em < B;
                const float e_dl = delta[ei];
                const float e_s = s_l[(size_t)min(em, B - 1) * sbs + ei];
                if (tl.m0 != done_m) {
                    if (wait(fl(l, 1) + (size_t)(tl.m0 >> 4) * N1, R / 16)) return;
                    done_m = tl.m0;
                }
                XF x[NCM];
                load_x<NCR, FULL>(x, vl, R, tl.m0, B, R, wv, lane);
                if (t == wg) BPROF_LOADED(5 * l + 2, 1);
                f4 acc[4] = {};
                mma<BLK, NCR>(acc, x, wa, lane);
                if (t + G < T2) load_w<BLK, NCR, FULL>(wa, W, tile_of(t + G, mb, N2).n0, wv, lane);
                tile_sum(acc, red, tile, wv, lane, tid);
                if (t == wg) BPROF(5 * l + 2, 2);
                if (eon) {
                    const int off = tid & 7;
                    const float* qr = tile + (tid >> 3) * 16;
                    const float gi = qr[8 + off];
                    const float uu = qr[off] * (sgm(gi - qr[8 + ((off + 1) & 7)]) * sgm(gi - qr[8 + ((off + 2) & 7)]));
                    float p = 1.0f - e_dl * (1.0f - sgm(gi));
                    if (a.clamp && p < a.p_floor) p = a.p_floor;
                    st_ag(snl + (size_t)em * D + ei, p * e_s + (1.0f - p) * uu);
                    st_ag(ul + (size_t)em * D + ei, uu);
                }
            }
        }
        BPROF(5 * l + 2, 3);
        publish_tiles(fl(l, 2), wg, G, T2, mb, N2, ep);
        fresh();
        if (wg < T3) load_w<BLK, NCD, FULL>(wa, mat(P->Wz, I, D), tile_of(wg, mb, N3).n0, wv, lane);
        issued();

        // ---- P3: z = wedge(W_z u) (sunnynet.c:268-271)
        // (the LN_mid gains of P4 are loaded here and staged in LDS before
        // the barrier, off P4's path)
        float gcv[2][NCM];
        {
            const gptr<float> mg = glb(uni(P->nm_g));
            const gptr<float> mc = glb(uni(P->nm_c));
#pragma unroll
            for (int k = 0; k < NCM; ++k) {
                const int i = min(k * NT + tid, I - 1);
                gcv[0][k] = mg[i];
                gcv[1][k] = mc[i];
            }
        }
        {
            const Mat W = mat(P->Wz, I, D);
            const float at = uni(P->a_tanh);
            BPROF(5 * l + 3, 0);
            int done_m = -1;                        // row block whose inputs are in
            for (int t = wg; t < T3; t += G) {
                fresh();
                const Tile tl = tile_of(t, mb, N3);
                if (tl.m0 != done_m) {
                    if (wait(fl(l, 2) + (size_t)(tl.m0 >> 4) * N2, N2)) return;
                    done_m = tl.m0;
                }
                XF x[NCM];
                load_x<NCD, FULL>(x, ul, D, tl.m0, B, D, wv, lane);
                if (t == wg) BPROF_LOADED(5 * l + 3, 1);
                f4 acc[4] = {};
                mma<BLK, NCD>(acc, x, wa, lane);
                if (t + G < T3) load_w<BLK, NCD, FULL>(wa, W, tile_of(t + G, mb, N3).n0, wv, lane);
                tile_sum(acc, red, tile, wv, lane, tid);
                if (t == wg) BPROF(5 * l + 3, 2);
                if (tid < 256) {
                    const int m = tl.m0 + (tid >> 4), n = tl.n0 + (tid & 15);
                    const float y = tile[tid];
                    if (m < B) st_ag(zl + (size_t)m * I + n, y * (1.0f + 0.5f * at / (1.0f + fabsf(y))));
                }
            }
        }
#pragma unroll
        for (int k = 0; k < NCM; ++k)
            if (k * NT + tid < I) {
                gc[k * NT + tid] = gcv[0][k];
                gc[kBatchMaxK + k * NT + tid] = gcv[1][k];
            }
        BPROF(5 * l + 3, 3);
        publish_tiles(fl(l, 3), wg, G, T3, mb, N3, ep);
        fresh();
        if (wg < T4) load_w<BLK, NCI, FULL>(wa, mat(P->Wc, D, I), tile_of(wg, mb, N4).n0, wv, lane);
        issued();

        // ---- P4: x' = W_c LN_mid(z) + b s' + sfb + x (sunnynet.c:273-276)
        {
            const Mat W = mat(P->Wc, D, I);
            const float bg = uni(P->b_gain);
            const int nch = I / CH;
            BPROF(5 * l + 4, 0);
            int done_m = -1;                        // row block whose inputs are in
            for (int t = wg; t < T4; t += G) {
                fresh();
                const Tile tl = tile_of(t, mb, N4);
                if (tl.m0 != done_m) {
                    if (wait(fl(l, 3) + (size_t)(tl.m0 >> 4) * N3, N3) ||
                        wait(fl(l, 1) + (size_t)(tl.m0 >> 4) * N1 + R / 16, D / 16))
                        return;
                    done_m = tl.m0;
                }
                const int em = tl.m0 + ((tid & 255) >> 4), en = tl.n0 + (tid & 15);
                const bool eon = tid < 256 && em < B;
                const size_t eo = (size_t)min(em, B - 1) * D + en;
                bool xok;
                const float* xr = in_row(l, min(em, B - 1), xok);
                const float e_sn = snl[eo], e_sfb = sfbl[eo], e_x = xok ? xr[en] : __builtin_nanf("");
                XF x[NCM];
                load_x<NCI, FULL>(x, zl, I, tl.m0, B, I, wv, lane);
                if (t == wg) BPROF_LOADED(5 * l + 4, 1);
                // LayerNorm of the tile's 16 rows: lane (r, q) holds 16 values
                // of row r per chunk; sums over q by shuffles, over waves in LDS.
                const int r = lane & 15, q = lane >> 4;
                float ps = 0.0f;
#pragma unroll
                for (int i = 0; i < NCI; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) ps += (x[i].a[j][0] + x[i].a[j][1]) + (x[i].a[j][2] + x[i].a[j][3]);
                ps += __shfl_xor(ps, 16, 64);
                ps += __shfl_xor(ps, 32, 64);
                if (lane < 16) lnp[0][wv * 16 + r] = ps;
                __syncthreads();
                float sum = lnp[0][r];
#pragma unroll
                for (int w = 1; w < NW; ++w) sum += lnp[0][w * 16 + r];
                const float mean = sum / (float)I;
                float pv = 0.0f;
#pragma unroll
                for (int i = 0; i < NCI; ++i) {
                    const float mk = FULL || wv + NW * i < nch ? 1.0f : 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float d = x[i].a[j][e] - mean;
                            pv += mk * (d * d);
                        }
                }
                pv += __shfl_xor(pv, 16, 64);
                pv += __shfl_xor(pv, 32, 64);
                if (lane < 16) lnp[1][wv * 16 + r] = pv;
                __syncthreads();
                float vsum = lnp[1][r];
#pragma unroll
                for (int w = 1; w < NW; ++w) vsum += lnp[1][w * 16 + r];
                const float rstd = 1.0f / sqrtf(vsum / (float)I + a.eps);
#pragma unroll
                for (int i = 0; i < NCI; ++i) {
                    const bool ok = FULL || wv + NW * i < nch;
                    const int c = ok ? wv + NW * i : 0;
                    const float mk = ok ? 1.0f : 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int k = c * CH + 16 * q + 4 * j + e;
                            x[i].a[j][e] = ((x[i].a[j][e] - mean) * rstd * gc[k] + gc[kBatchMaxK + k]) * mk;
                        }
                }
                f4 acc[4] = {};
                mma<BLK, NCI>(acc, x, wa, lane);
                if (t + G < T4) load_w<BLK, NCI, FULL>(wa, W, tile_of(t + G, mb, N4).n0, wv, lane);
                tile_sum(acc, red, tile, wv, lane, tid);
                if (t == wg) BPROF(5 * l + 4, 2);
                if (eon) {
                    st_ag(xo + (size_t)em * D + en, tile[tid] + (bg * e_sn + e_sfb + e_x));
                    st_ag(s_l + (size_t)em * sbs + en, e_sn);
                }
            }
        }
        BPROF(5 * l + 4, 3);
        publish_tiles(fl(l, 4), wg, G, T4, mb, N4, ep);
        fresh();
        if (l + 1 < L && wg < T1)
            load_w<BLK, NCD, FULL>(wa, mat(ltab[l + 1].VW, R + D, D), tile_of(wg, mb, N1).n0, wv, lane);
        issued();
    }

    // ---- final LayerNorm of every row (sunnynet.c:330-332): the head's input
    BPROF(5 * L, 0);
    const float* xl = a.xs + (size_t)(L - 1) * B * D;
    for (int b = wg; b < B; b += G) {
        fresh();
        if (wait(fl(L - 1, 4) + (size_t)(b >> 4) * N4, N4)) return;
        float xv[PERM], gv[PERM], cv[PERM];
#pragma unroll
        for (int k = 0; k < PERM; ++k) {
            const int i = min(k * NT + tid, D - 1);
            xv[k] = xl[(size_t)b * D + i];
            gv[k] = a.no_g[i];
            cv[k] = a.no_c[i];
        }
        float mean, rstd;
        row_stats(xv, D, a.eps, rred, tid, wv, lane, mean, rstd);
#pragma unroll
        for (int k = 0; k < PERM; ++k) {
            const int i = k * NT + tid;
            if (i < D) a.nrm[(size_t)b * D + i] = (xv[k] - mean) * rstd * gv[k] + cv[k];
        }
    }
}

#ifdef SNHIP_BATCH_PROF
}  // namespace
extern "C" int snhip_batch_prof(unsigned long long* out, int n) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_bprof), sizeof(unsigned long long) * n) == hipSuccess;
}
namespace {
#endif

// Chunks per wave of a product of depth k (0 if deeper than the kernel takes).
int chunks(int k) { return (k / CH + NW - 1) / NW; }

// The compiled shapes: SunnyNet-100M's dim / rank / inner of 1024 / 512 /
// 1536 (whole chunks for every wave), and any model up to 512 wide.
const void* kernel_for(int blk, int D, int I, int R) {
    const int cd = chunks(D), cr = chunks(R), ci = chunks(I);
    const bool full = D == cd * NW * CH && R == cr * NW * CH && I == ci * NW * CH;
#define SNHIP_KB(NCD, NCR, NCI, FULL)                                                   \
    if (cd == NCD && cr == NCR && ci == NCI && full == FULL) {                          \
        if (blk == 32) return (const void*)k_decode_batch<32, NCD, NCR, NCI, FULL>;     \
        if (blk == 64) return (const void*)k_decode_batch<64, NCD, NCR, NCI, FULL>;     \
        return (const void*)k_decode_batch<0, NCD, NCR, NCI, FULL>;                     \
    }
    SNHIP_KB(2, 1, 3, true)
    SNHIP_KB(1, 1, 1, false)
#undef SNHIP_KB
    return nullptr;
}

}  // namespace

bool batch_shape_ok(int D, int I, int R, int K, int L) {
    auto deep_ok = [](int k) { return k > 0 && k % CH == 0 && k <= kBatchMaxK; };
    return deep_ok(D) && deep_ok(I) && deep_ok(R) && D <= kBatchMaxRow && K == kTaps && L >= 1 &&
           L <= kPersistMaxL && kernel_for(0, D, I, R) != nullptr;
}

int batch_grid(int blk, int D, int I, int R) {
    int dev = 0, coop = 0, ncu = 0, occ = 0;
    const void* k = kernel_for(blk, D, I, R);
    if (!k || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, NT, 0) != hipSuccess || occ < 1) return 0;
    return (ncu / 8) * 8;
}

snhip_status launch_decode_batch(const BatchArgs& a, int G, int blk, hipStream_t st) {
    const void* k = kernel_for(blk, a.D, a.I, a.R);
    if (!k || !batch_shape_ok(a.D, a.I, a.R, a.K, a.L) || a.B < 1 || G < 8 || G % 8 || a.kh != kTaps - 1) {
        set_last_error("batched persistent decode: unsupported shape or arguments");
        return SNHIP_E_INVAL;
    }
    BatchArgs args = a;
    void* kargs[] = {&args};
    SNHIP_CHECK(launch_persistent(k, dim3(G), dim3(NT), kargs, st));
    return SNHIP_OK;
}

}  // namespace snhip
