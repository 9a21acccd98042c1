// Persistent decode of several sequences in one cooperative launch: the
// single-sequence kernel's phase walk (A, B, C, D per layer, the head H and
// the token reduction T; see persist.hip) with up to NS sequences carried
// through every phase together. Every weight row a workgroup owns is loaded
// and dequantized once per phase and multiplied against each sequence's
// input vector, so a batch of 2..8 sequences streams the INT4 weights once per
// step, as one sequence does.
//
// Included by persist_kernel.h inside the 512-thread namespace (its helpers:
// exchange words, DPP sums, Geo / Pool / pool_load, argmax keys).
//
// Layouts (ns <= NS sequences, q the sequence):
//   exchange word of element i of a phase's output vector: i NS + q
//   new-state words sx: ((l 2 + step parity) D + i) NS + q
//   argmax keys of the head: ((q G + wg) 2 + h)
//   LN_in history ring of workgroup wg: ((l KH + slot) D + i) NS + q
//   handle state s (B, L, D) and history (B, L, KH, D), as the batched paths
//   staged LDS vectors: sequence q at q XSQ (the INT4 staged layout)
// so a thread's NS words of one element are contiguous.

constexpr int XSQ = kMaxK + kStagePad * 64;  // LDS floats per sequence of a staged input vector
constexpr int XSD = kMaxD + kStagePad * 64;  // and of a staged old state
constexpr int kMsOwn = 32;                   // owned channels per workgroup, at most
constexpr int kMsRows = 64;                  // rows a workgroup multiplies in a layer phase, at most
constexpr int kMsMaxGrid = 256;              // workgroups, at most (argmax keys: one per thread)

// Block sums of NS values per thread, one barrier (red holds NS NWV floats).
template <int NS>
__device__ __forceinline__ void bsum_ms(float (&v)[NS], float* red, int ns) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        if (q >= ns) break;
        const float s = wsum(v[q]);
        if (lane == 0) red[q * NWV + w] = s;
    }
    barrier_lds();
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        if (q >= ns) break;
        float r[NWV];
#pragma unroll
        for (int i = 0; i < NWV; ++i) r[i] = red[q * NWV + i];
#pragma unroll
        for (int h = NWV / 2; h > 0; h >>= 1)
#pragma unroll
            for (int i = 0; i < h; ++i) r[i] = r[i] + r[i + h];
        v[q] = r[0];
    }
}

// Two-pass LayerNorm statistics (sunnynet.c:198-210) of each sequence's n
// values (element k NT + tid of sequence q in xv[k][q]); red holds 2 NS NWV.
template <int N, int NS>
__device__ __forceinline__ void ln_stats_ms(const float (&xv)[N][NS], int n, float eps, float* red, int ns,
                                            float (&mean)[NS], float (&rstd)[NS]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (k * NT + tid < n) s += xv[k][q];
        mean[q] = s;
    }
    bsum_ms<NS>(mean, red, ns);
#pragma unroll
    for (int q = 0; q < NS; ++q) mean[q] = mean[q] * (1.0f / (float)n);
    float vs[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (k * NT + tid < n) {
                const float d = xv[k][q] - mean[q];
                s += d * d;
            }
        vs[q] = s;
    }
    bsum_ms<NS>(vs, red + NS * NWV, ns);
#pragma unroll
    for (int q = 0; q < NS; ++q) rstd[q] = rsqrtf(vs[q] * (1.0f / (float)n) + eps);
}

// Batch b of J (INT4 units, as compute_i4) for every sequence: the lane's
// group is dequantized once, then multiplied against each sequence's staged
// input (its quads read from LDS), in the single-sequence kernel's order of
// partial sums. epi(q, j, row, value, writer).
template <int BLK, int NS, class Epi>
__device__ __forceinline__ void compute_i4_ms(const Job& J, int b, const Pool<BLK>& P, int lane, int ns,
                                              Epi&& epi) {
    constexpr int MU = Pool<BLK>::MU;
    constexpr int NW = BLK / 8;                  // 32-bit words of codes per group
    const Geo& g = J.g;
    const int seg = 1 << g.lseg;
    const int lrow = lane >> g.lseg, lg = lane & (seg - 1);
    const bool lane_ok = lg < g.ng;
    const int lgc = min(lg, g.ng - 1);
    const int nvu = min(MU, g.nwu - b * MU);
    float acc[MU][NS];
#pragma unroll
    for (int s = 0; s < MU; ++s) {
#pragma unroll
        for (int q = 0; q < NS; ++q) acc[s][q] = 0.0f;
        if (s >= nvu) continue;
        // (q - 8) * scale as one rounding: fma(q, scale, -8 scale), with
        // -8 scale exact (quant.c:82-83 dequantization, bit-identical).
        const float sc = P.wsc[s], m8 = -8.0f * sc;
        float wd[BLK];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const uint4& qq = P.wq[s][w >> 2];
            const int wi = w & 3;
            const uint32_t word = wi == 0 ? qq.x : wi == 1 ? qq.y : wi == 2 ? qq.z : qq.w;
            // byte 4w + e: element 4w + e (low nibble), BLK/2 + 4w + e (high)
            const uint32_t lo = opqu(word & 0x0F0F0F0Fu), hi = opqu((word >> 4) & 0x0F0F0F0Fu);
            wd[4 * w + 0] = fmaf((float)(lo & 0xFFu), sc, m8);
            wd[4 * w + 1] = fmaf((float)((lo >> 8) & 0xFFu), sc, m8);
            wd[4 * w + 2] = fmaf((float)((lo >> 16) & 0xFFu), sc, m8);
            wd[4 * w + 3] = fmaf((float)(lo >> 24), sc, m8);
            wd[BLK / 2 + 4 * w + 0] = fmaf((float)(hi & 0xFFu), sc, m8);
            wd[BLK / 2 + 4 * w + 1] = fmaf((float)((hi >> 8) & 0xFFu), sc, m8);
            wd[BLK / 2 + 4 * w + 2] = fmaf((float)((hi >> 16) & 0xFFu), sc, m8);
            wd[BLK / 2 + 4 * w + 3] = fmaf((float)(hi >> 24), sc, m8);
        }
#pragma unroll
        for (int q = 0; q < NS; ++q) {
            if (q >= ns) break;
            const l_f32* xq = J.x + q * (g.xsel ? XSD : XSQ);
            float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float4 xl = lds4(xq + 4 * (w * (g.ng + kStagePad) + lgc));
                const float4 xh = lds4(xq + 4 * ((w + NW) * (g.ng + kStagePad) + lgc));
                a4[0] = fmaf(wd[4 * w + 0], xl.x, a4[0]);
                a4[1] = fmaf(wd[4 * w + 1], xl.y, a4[1]);
                a4[2] = fmaf(wd[4 * w + 2], xl.z, a4[2]);
                a4[3] = fmaf(wd[4 * w + 3], xl.w, a4[3]);
                a4[0] = fmaf(wd[BLK / 2 + 4 * w + 0], xh.x, a4[0]);
                a4[1] = fmaf(wd[BLK / 2 + 4 * w + 1], xh.y, a4[1]);
                a4[2] = fmaf(wd[BLK / 2 + 4 * w + 2], xh.z, a4[2]);
                a4[3] = fmaf(wd[BLK / 2 + 4 * w + 3], xh.w, a4[3]);
            }
            acc[s][q] = lane_ok ? (a4[0] + a4[1]) + (a4[2] + a4[3]) : 0.0f;
            // one sequence's quads in flight at a time (hoisting every
            // sequence's loads above the first FMA would spill)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (seg >= 16) {
        // the 16-lane rows by DPP, then across rows with lane swaps (the
        // values stay in vector registers: 4 NS MU scalar reads would not fit)
#pragma unroll
        for (int s = 0; s < MU; ++s)
#pragma unroll
            for (int q = 0; q < NS; ++q)
                if (s < nvu && q < ns) acc[s][q] = row_sum(acc[s][q]);
        if (seg > 16) {
#pragma unroll
            for (int s = 0; s < MU; ++s)
#pragma unroll
                for (int q = 0; q < NS; ++q) {
                    if (s >= nvu || q >= ns) continue;
                    float v = acc[s][q] + __shfl_xor(acc[s][q], 16, 64);
                    if (seg == 64) v = v + __shfl_xor(v, 32, 64);
                    acc[s][q] = v;
                }
        }
    } else {
        for (int o = seg >> 1; o > 0; o >>= 1)
#pragma unroll
            for (int s = 0; s < MU; ++s)
#pragma unroll
                for (int q = 0; q < NS; ++q)
                    if (s < nvu && q < ns) acc[s][q] += __shfl_xor(acc[s][q], o, 64);
    }
#pragma unroll
    for (int s = 0; s < MU; ++s) {
        const int jl = (g.wl + g.nwp * (b * MU + s)) * g.rpp + lrow;
        if (s >= nvu || jl >= g.cnt) continue;
        const int j = g.base + jl, row = job_row(g, j);
#pragma unroll
        for (int q = 0; q < NS; ++q)
            if (q < ns) epi(q, j, row, acc[s][q], lg == 0);
    }
}

// Every batch of J for every sequence (batch 0 already in p0; later batches
// stream through two pools local to the job, as run_job's INT4 path).
template <int BLK, int NS, class Epi>
__device__ __forceinline__ void run_job_ms(const Job& J, const Pool<BLK>& p0, int lane, int ns, Epi&& epi) {
    const int nb = J.g.nb;
    if (nb == 0) return;
    if (nb == 1) {
        compute_i4_ms<BLK, NS>(J, 0, p0, lane, ns, epi);
        return;
    }
    Pool<BLK> q0, q1;
    pool_load<BLK>(J, 1, q1, lane);
    compute_i4_ms<BLK, NS>(J, 0, p0, lane, ns, epi);
    for (int b = 1; b < nb; b += 2) {
        pool_load<BLK>(J, b + 1, q0, lane);
        compute_i4_ms<BLK, NS>(J, b, q1, lane, ns, epi);
        pool_load<BLK>(J, b + 2, q1, lane);
        if (b + 1 < nb) compute_i4_ms<BLK, NS>(J, b + 1, q0, lane, ns, epi);
    }
}

template <int BLK, int NS>
__global__ __launch_bounds__(NT) void k_decode_persist_ms(PersistArgs a) {
    static_assert(is_i4(BLK), "the multi-sequence kernel multiplies INT4 rows");
    // staged input vectors of the current products (sequence q at q XSQ), the
    // old states (W_eff's input in phase A; the state update in phase B)
    __shared__ __align__(16) float xin[NS * XSQ];
    __shared__ __align__(16) float xs2[NS * XSD];
    __shared__ float xres[NS][kMsOwn];            // x of the layer, owned channels
    __shared__ float res[NS][kMsRows];            // products of the current phase, by job row
    __shared__ float sown[NS][kMsOwn];            // s' of the owned channels
    __shared__ float sfbl[NS][kMsOwn];            // W_eff s_old of the owned channels
    __shared__ float red[2 * NS * NWV];
    __shared__ u64 kred[NS][NWV];
    __shared__ int sflag;
    __shared__ PLayer ltab[kPersistMaxL];
    __shared__ Geo geo[5][NWV];

    int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    auto fresh = [&]() {
        tid = opq(tid);
        lane = tid & 63;
    };
    const int G = gridDim.x, wg = blockIdx.x;
    const int D = a.D, I = a.I, R = a.R, L = a.L, ns = a.ns;
    const size_t sst = (size_t)L * D, hst = (size_t)L * KH * D;   // handle state strides
    const int cpw = D / G, c0 = wg * cpw;                     // owned channels
    const int grp0 = c0 >> 3, ngrp = cpw >= 8 ? cpw >> 3 : 1; // owned channel groups
    const PollCtl pc{a.err, a.spin_limit};
    for (int i = tid; i < L * (int)sizeof(PLayer) / 4; i += NT)
        ((uint32_t*)ltab)[i] = ((const uint32_t*)a.layers)[i];
    const PLayer* lt = ltab;
    u64* ex0 = a.ex;
    auto exs = [&](unsigned e) -> u64* { return ex0 + (size_t)(e & 1u) * kPersistMsExWords; };

    if (tid == 0) sflag = 0;
    barrier_lds();
    auto agree = [&](bool ok) -> bool {
        if (!ok) sflag = 1;
        barrier_lds();
        return sflag == 0;
    };

    const int nV = R > wg ? (R - wg + G - 1) / G : 0;
    const int nZ = I > wg ? (I - wg + G - 1) / G : 0;
    const int nH = a.vocab > wg ? (a.vocab - wg + G - 1) / G : 0;
    const l_f32* lx = (const l_f32*)xin;
    const l_f32* ls = (const l_f32*)xs2;
    const int NP = 4 * L + 1;
    if (lane == 0) {
        geo[0][wv] = make_geo<BLK>(D, nV, nV + cpw, wg, G, R + c0, wv);
        geo[1][wv] = make_geo<BLK>(R, 16 * ngrp, 16 * ngrp, 16 * grp0, 1, 0, wv);
        geo[2][wv] = make_geo<BLK>(D, nZ, nZ, wg, G, 0, wv);
        geo[3][wv] = make_geo<BLK>(I, cpw, cpw, c0, 1, 0, wv);
        geo[4][wv] = make_geo<BLK>(D, nH, nH, wg, G, 0, wv);
    }
    barrier_lds();
    auto job = [&](int p) -> Job {
        const int t = p < 4 * L ? (p & 3) : 4;
        Job J;
        J.g = geo[t][wv];
        J.x = J.g.xsel ? ls : lx;
        PMat W = a.head;
        if (t < 4) {
            const PLayer* Ly = lt + (p >> 2);
            W = t == 0 ? Ly->VW : t == 1 ? Ly->U : t == 2 ? Ly->Wz : Ly->Wc;
        }
        J.w = W.w; J.h = W.h; J.q = W.q; J.sc = W.sc;
        return J;
    };

    Pool<BLK> p0;
    prefetch_job<BLK>(job(0), p0, lane);

    unsigned ep = 0;
    const unsigned stall = a.stall;
    int tok[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) tok[q] = q < ns ? a.tok_in[q] : 0;
    float* ring_wg = a.ring + (size_t)wg * L * KH * D * NS;
    constexpr int WMAX = 2 * PD;      // exchange elements per thread (A: x and s)
    static_assert(WMAX >= PK, "gather words");

    for (int step = 0; step < a.n_steps; ++step) {
        const bool last = step + 1 == a.n_steps;
        auto tok_ok = [&](int q) { return tok[q] >= 0 && tok[q] < a.vocab; };
        u64 best[NS];
#pragma unroll
        for (int q = 0; q < NS; ++q) best[q] = 0ull;
        for (int p = 0; p < NP; ++p) {
            fresh();
            const int t = p < 4 * L ? (p & 3) : 4;        // 0 A, 1 B, 2 C, 3 D, 4 H
            const int l = min(p >> 2, L - 1);
            const PLayer* Ly = lt + l;
            const int n0 = t == 1 ? R : t == 3 ? I : D;
            const unsigned e0 = ep + stall, e1 = (unsigned)step + stall;
            const u64* s0 = exs(ep);
            const u64* s1 = a.sx + ((size_t)l * 2 + ((step - 1) & 1)) * D * NS;
            const bool plain0 = t == 0 && l == 0;          // x = the tokens' embedding rows
            const bool plain1 = step == 0;                 // s = the handle's state
            const bool ln = t == 0 || t >= 3;
            const float* gp = t == 0 ? Ly->ni_g : t == 3 ? Ly->nm_g : a.no_g;
            const float* cp = t == 0 ? Ly->ni_c : t == 3 ? Ly->nm_c : a.no_c;
            u64 w[WMAX][NS];
            float gv[PK], cv[PK], dw3[PD], ach[PD][NS], dl[PD];
            float* ring_l = ring_wg + (size_t)l * KH * D * NS;
            // element index of word slot k (A: x for k < PD, s for k >= PD)
            auto elem = [&](int k) -> int {
                const bool s_word = t == 0 && k >= PD;
                return (s_word ? k - PD : k) * NT + tid;
            };
            auto slot_in = [&](int k) -> bool {
                if (t == 0) return elem(k) < D;
                return k < PK && elem(k) < n0;
            };
            auto addr = [&](int k, int q) -> const u64* {
                if (t == 0 && k >= PD) return s1 + (size_t)min(elem(k), D - 1) * NS + q;
                return s0 + (size_t)min(elem(k), n0 - 1) * NS + q;
            };
            auto want = [&](int k) { return t == 0 && k >= PD ? e1 : e0; };
#pragma unroll
            for (int k = 0; k < WMAX; ++k) {
                const bool s_word = t == 0 && k >= PD;
                const int i = min(elem(k), (s_word ? D : n0) - 1);
#pragma unroll
                for (int q = 0; q < NS; ++q) {
                    if (!slot_in(k) || q >= ns) w[k][q] = ll_ready(0.0f, want(k));
                    else if (s_word && plain1) w[k][q] = ll_ready(ldg(a.s + q * sst + (size_t)l * D + i), want(k));
                    else if (!s_word && plain0)
                        w[k][q] = ll_ready(ldg(a.embed + (size_t)(tok_ok(q) ? tok[q] : 0) * D + i), want(k));
                    else w[k][q] = ll_get(addr(k, q));
                }
            }
            if (ln) {
#pragma unroll
                for (int k = 0; k < PK; ++k) {
                    const int i = min(k * NT + tid, n0 - 1);
                    gv[k] = ldg(gp + i);
                    cv[k] = ldg(cp + i);
                }
            }
            if (t == 0) {
                // The history's part of the conv (sunnynet.c:227-233) does not
                // depend on the polled x: hist[0] w[K-2] + hist[1] w[K-3] + ...
                // from this workgroup's ring (or the handle's history before
                // the launch), formed while the words are in flight.
#pragma unroll
                for (int k = 0; k < PD; ++k) {
                    const int i = min(k * NT + tid, D - 1);
                    float dv[KT];
#pragma unroll
                    for (int u = 0; u < KT; ++u) dv[u] = ldg(Ly->dw + (size_t)u * D + i);
                    dw3[k] = dv[KT - 1];
#pragma unroll
                    for (int q = 0; q < NS; ++q) {
                        float hsum = 0.0f;
#pragma unroll
                        for (int u = 0; u < KH; ++u) {
                            const int age = step - 1 - u;
                            const float h = q >= ns ? 0.0f
                                          : age >= 0 ? ring_l[((size_t)(age % KH) * D + i) * NS + q]
                                                     : ldg(a.hist + q * hst + ((size_t)l * KH + (u - step)) * D + i);
                            hsum = u == 0 ? h * dv[KT - 2] : hsum + h * dv[KT - 2 - u];
                        }
                        ach[k][q] = hsum;
                    }
                }
            }
            if (t == 1) {
#pragma unroll
                for (int k = 0; k < PD; ++k) dl[k] = ldg(Ly->delta + min(c0 + k * NT + tid, D - 1));
            }
            // Re-polls the words that do not carry their epoch yet (all
            // sequences of a slot at once).
            bool polled = true;
            {
                unsigned spins = 0;
                while (true) {
                    bool all = true;
#pragma unroll
                    for (int k = 0; k < WMAX; ++k)
#pragma unroll
                        for (int q = 0; q < NS; ++q) all = all && ll_ok(w[k][q], want(k));
                    if (all) break;
                    if ((++spins & 255) == 0) {
                        if (__hip_atomic_load(pc.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                            polled = false;
                            break;
                        }
                        if (spins > pc.limit) {
                            __hip_atomic_store(pc.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            polled = false;
                            break;
                        }
                    }
#pragma unroll
                    for (int k = 0; k < WMAX; ++k)
#pragma unroll
                        for (int q = 0; q < NS; ++q)
                            if (!ll_ok(w[k][q], want(k))) w[k][q] = ll_get(addr(k, q));
                }
            }
            float xv[PK][NS];
#pragma unroll
            for (int k = 0; k < PK; ++k) {
                const bool in = k * NT + tid < n0 && (t != 0 || k < PD);
#pragma unroll
                for (int q = 0; q < NS; ++q)
                    xv[k][q] = !in ? 0.0f : (plain0 && !tok_ok(q)) ? __builtin_nanf("") : ll_f(w[k][q]);
            }
            if (!agree(polled)) return;
            float mean[NS], rstd[NS];
#pragma unroll
            for (int q = 0; q < NS; ++q) mean[q] = rstd[q] = 0.0f;
            if (ln) ln_stats_ms<PK, NS>(xv, n0, a.eps, red, ns, mean, rstd);
#pragma unroll
            for (int k = 0; k < PK; ++k) {
                const int i = k * NT + tid;
                if (i >= n0 || (t == 0 && k >= PD)) continue;
#pragma unroll
                for (int q = 0; q < NS; ++q) {
                    if (q >= ns) break;
                    float y = ln ? (xv[k][q] - mean[q]) * rstd[q] * gv[k] + cv[k] : xv[k][q];
                    if (k < PD && t == 0) {
                        const float acc = y * dw3[k] + ach[k][q];
                        ring_l[((size_t)(step % KH) * D + i) * NS + q] = y;
                        xs2[q * XSD + sidx<BLK>(i, D)] = ll_f(w[PD + k][q]);
                        if (i >= c0 && i < c0 + cpw) xres[q][i - c0] = xv[k][q];
                        y = y + acc;
                    }
                    xin[q * XSQ + sidx<BLK>(i, n0)] = y;
                }
            }
            barrier_lds();
            // ---- the products; every phase but H leaves them in res by job row
            const bool head = t == 4;
            float* lgp = head && last ? a.logits : nullptr;
            run_job_ms<BLK, NS>(job(p), p0, lane, ns, [&](int q, int j, int row, float v, bool wr) {
                if (!wr) return;
                if (!head) {
                    res[q][j] = v;
                } else {
                    if (lgp) lgp[(size_t)q * a.vocab + row] = v;
                    best[q] = max(best[q], argmax_key(v, row));
                }
            });
            barrier_lds();
            // ---- the phase's outputs
            const unsigned epv = ++ep;
            u64* out = exs(epv);
            if (t == 0) {
                for (int e = tid; e < (nV + cpw) * NS; e += NT) {
                    const int j = e / NS, q = e - j * NS;
                    if (q >= ns) continue;
                    if (j < nV) ll_putf(out + (size_t)(wg + j * G) * NS + q, res[q][j], epv);
                    else sfbl[q][j - nV] = res[q][j];
                }
            } else if (t == 1) {
                // sunnynet.c:248-262: competitive gate within the group of 8,
                // decay gate, state update
                u64* sout = a.sx + ((size_t)l * 2 + (step & 1)) * D * NS;
#pragma unroll
                for (int k = 0; k < PD; ++k) {
                    const int c = k * NT + tid;
                    if (c >= cpw) continue;
                    const int i = c0 + c, jj = i & 7, base = ((i >> 3) - grp0) * 16;
#pragma unroll
                    for (int q = 0; q < NS; ++q) {
                        if (q >= ns) break;
                        const float* rq = res[q];
                        const float gi = rq[base + 8 + jj];
                        const float uu = rq[base + jj] * (sgm(gi - rq[base + 8 + ((jj + 1) & 7)]) *
                                                          sgm(gi - rq[base + 8 + ((jj + 2) & 7)]));
                        float pg = 1.0f - dl[k] * (1.0f - sgm(gi));
                        if (a.clamp && pg < a.p_floor) pg = a.p_floor;
                        const float sn = pg * xs2[q * XSD + sidx<BLK>(i, D)] + (1.0f - pg) * uu;
                        ll_putf(out + (size_t)i * NS + q, uu, epv);
                        ll_putf(sout + (size_t)i * NS + q, sn, (unsigned)step + 1);
                        sown[q][c] = sn;
                    }
                }
            } else if (t == 2) {
                const float at = Ly->a_tanh;
                for (int e = tid; e < nZ * NS; e += NT) {
                    const int j = e / NS, q = e - j * NS;
                    if (q >= ns) continue;
                    const float v = res[q][j];
                    ll_putf(out + (size_t)(wg + j * G) * NS + q, v * (1.0f + 0.5f * at / (1.0f + fabsf(v))), epv);
                }
            } else if (t == 3) {
                const float bg = Ly->b_gain;
                for (int e = tid; e < cpw * NS; e += NT) {
                    const int c = e / NS, q = e - c * NS;
                    if (q >= ns) continue;
                    ll_putf(out + (size_t)(c0 + c) * NS + q, res[q][c] + (bg * sown[q][c] + sfbl[q][c] + xres[q][c]),
                            epv);
                }
            } else if (a.greedy) {
#pragma unroll
                for (int q = 0; q < NS; ++q) {
                    if (q >= ns) break;
                    const u64 bq = kmax_wave(best[q]);
                    if (lane == 0) kred[q][wv] = bq;
                }
                barrier_lds();
                if (tid < 2 * ns) {
                    const int q = tid >> 1, h = tid & 1;
                    u64 kk = kred[q][0];
#pragma unroll
                    for (int i = 1; i < NWV; ++i) kk = max(kk, kred[q][i]);
                    ll_put(out + ((size_t)q * G + wg) * 2 + h, h == 0 ? (uint32_t)(kk >> 32) : (uint32_t)kk, epv);
                }
            }
            // ---- the next phase's first weights (the next step's first phase after H)
            prefetch_job<BLK>(job(p + 1 < NP ? p + 1 : 0), p0, lane);
        }
        if (!a.greedy) break;
        fresh();
        // ---------------- T: every workgroup reduces each sequence's keys
        // (every sequence's words issued at once, then re-polled together)
        {
            const unsigned epx = ep + stall;
            const u64* ksrc = exs(ep);
            u64 w2[NS][2];
            auto kaddr = [&](int q, int k) {
                return ksrc + ((size_t)q * G + min(tid, G - 1)) * 2 + k;
            };
#pragma unroll
            for (int q = 0; q < NS; ++q)
#pragma unroll
                for (int k = 0; k < 2; ++k)
                    w2[q][k] = q < ns && tid < G ? ll_get(kaddr(q, k)) : ll_ready(0.0f, epx);
            bool ok = true;
            unsigned spins = 0;
            while (true) {
                bool all = true;
#pragma unroll
                for (int q = 0; q < NS; ++q)
#pragma unroll
                    for (int k = 0; k < 2; ++k) all = all && ll_ok(w2[q][k], epx);
                if (all) break;
                if ((++spins & 255) == 0) {
                    if (__hip_atomic_load(pc.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                        ok = false;
                        break;
                    }
                    if (spins > pc.limit) {
                        __hip_atomic_store(pc.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        ok = false;
                        break;
                    }
                }
#pragma unroll
                for (int q = 0; q < NS; ++q)
#pragma unroll
                    for (int k = 0; k < 2; ++k)
                        if (!ll_ok(w2[q][k], epx)) w2[q][k] = ll_get(kaddr(q, k));
            }
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                if (q >= ns) break;
                u64 kk = tid < G ? ((u64)(uint32_t)w2[q][0] << 32) | (uint32_t)w2[q][1] : 0ull;
                kk = kmax_wave(kk);
                if (lane == 0) kred[q][wv] = kk;
            }
            if (!agree(ok)) return;
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                if (q >= ns) break;
                u64 kk = kred[q][0];
#pragma unroll
                for (int i = 1; i < NWV; ++i) kk = max(kk, kred[q][i]);
                tok[q] = (int)(0xFFFFFFFFu - (uint32_t)(kk & 0xFFFFFFFFull));
                if (wg == 0 && tid == 0) a.out_tok[(size_t)step * ns + q] = tok[q];
            }
            barrier_lds();
        }
    }

    // Owners write back each sequence's state and history (newest first) of
    // their channels, for every layer. A ring entry is read by the thread that
    // wrote it in phase A (element k NT + tid).
    const int T = a.n_steps;
    for (int l = 0; l < L; ++l) {
        const float* ring_l = ring_wg + (size_t)l * KH * D * NS;
        const u64* sl = a.sx + ((size_t)l * 2 + ((T - 1) & 1)) * D * NS;
#pragma unroll
        for (int k = 0; k < PD; ++k) {
            const int i = k * NT + tid;
            if (i >= D || i < c0 || i >= c0 + cpw) continue;
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                if (q >= ns) break;
                a.s[q * sst + (size_t)l * D + i] = ll_f(ll_get(sl + (size_t)i * NS + q));
#pragma unroll
                for (int j = KH - 1; j >= 0; --j) {
                    const int age = T - 1 - j;
                    float* hj = a.hist + q * hst + ((size_t)l * KH + j) * D + i;
                    *hj = age >= 0 ? ring_l[((size_t)(age % KH) * D + i) * NS + q]
                                   : a.hist[q * hst + ((size_t)l * KH + (j - T)) * D + i];
                }
            }
        }
    }
}
