// Body of the persistent single-sequence decode kernel, included by
// persist.hip once per workgroup size: SNHIP_PERSIST_NT threads per
// workgroup, in namespace snhip::SNHIP_PERSIST_NS. See persist.hip.
namespace snhip {
namespace SNHIP_PERSIST_NS {


constexpr int NT = SNHIP_PERSIST_NT;         // threads per workgroup
constexpr int NWV = NT / 64;
constexpr int kMaxD = kPersistMaxD;          // dim
constexpr int kMaxK = kPersistMaxK;          // inner, rank
constexpr int PD = (kMaxD + NT - 1) / NT;   // values per thread of a dim-wide vector
constexpr int PK = (kMaxK + NT - 1) / NT;   // of an inner- or rank-wide vector
constexpr int CAPF = 4;                      // fp32: float4 per lane in one batch
constexpr int KPT = (kPersistMaxGrid + NT - 1) / NT;   // argmax keys per thread
constexpr int KT = kPersistTaps;             // conv taps
constexpr int KH = KT - 1;                   // history entries
constexpr int kStagePad = 2;                 // INT4 staged layout: pad groups per quad row

typedef unsigned long long u64;

// Read-only data through global-address-space pointers: global_load (counted
// by vmcnt only); through a generic pointer the compiler emits flat loads,
// which also count against lgkmcnt and would make the first LDS wait after a
// prefetch wait for every prefetched weight.
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const float g_f32;
typedef __attribute__((address_space(1))) const f32x4v g_f32x4;
typedef __attribute__((address_space(1))) const u32x4v g_u32x4;
__device__ __forceinline__ float ldg(const float* p) { return *(g_f32*)p; }
__device__ __forceinline__ float4 ldg4(const float* p) {
    const f32x4v v = *(g_f32x4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldgq(const uint8_t* p) {
    const u32x4v v = *(g_u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) const u32x2v g_u32x2;
// Four fp16 weights (8 bytes) and their exact fp32 values.
__device__ __forceinline__ uint2 ldgh4(const uint16_t* p) {
    const u32x2v v = *(g_u32x2*)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ float4 h4f(uint2 h) {
    return make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(h.x & 0xFFFFu)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(h.x >> 16)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(h.y & 0xFFFFu)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(h.y >> 16)));
}
typedef __attribute__((address_space(3))) float l_f32;
typedef __attribute__((address_space(3))) const f32x4v l_f32x4;
__device__ __forceinline__ float4 lds4(const l_f32* p) {
    const f32x4v v = *(l_f32x4*)p;
    return make_float4(v.x, v.y, v.z, v.w);
}

// ---- exchange words
__device__ __forceinline__ void ll_put(u64* p, uint32_t bits, unsigned ep) {
    __hip_atomic_store(p, ((u64)ep << 32) | (u64)bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_putf(u64* p, float v, unsigned ep) { ll_put(p, __float_as_uint(v), ep); }
__device__ __forceinline__ u64 ll_get(const u64* p) {
    return __hip_atomic_load(const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool ll_ok(u64 w, unsigned ep) { return (uint32_t)(w >> 32) == ep; }
__device__ __forceinline__ float ll_f(u64 w) { return __uint_as_float((uint32_t)w); }
__device__ __forceinline__ u64 ll_ready(float v, unsigned ep) { return ((u64)ep << 32) | __float_as_uint(v); }

struct PollCtl {
    unsigned* err;
    unsigned limit;
};

// Re-polls the words of w that do not carry their epoch yet (word k from
// addr(k), expected epoch want(k)) until all do. False on time-out (this
// thread then sets the error word) or when another workgroup reported one.
template <int W, class Addr, class Want>
__device__ __forceinline__ bool ll_spin(u64 (&w)[W], Addr&& addr, Want&& want, const PollCtl& pc) {
    unsigned spins = 0;
    while (true) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < W; ++k) all = all && ll_ok(w[k], want(k));
        if (all) return true;
        if ((++spins & 255) == 0) {
            if (__hip_atomic_load(pc.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
            if (spins > pc.limit) {
                __hip_atomic_store(pc.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return false;
            }
        }
#pragma unroll
        for (int k = 0; k < W; ++k)
            if (!ll_ok(w[k], want(k))) w[k] = ll_get(addr(k));
    }
}

__device__ __forceinline__ float sgm(float x) { return 1.0f / (1.0f + expf(-x)); }

// The same value, opaque to the optimizer. Applied to the thread index at
// every phase so per-lane addresses are formed inside the phase instead of
// being hoisted out of the step loop (hundreds would stay live and spill).
__device__ __forceinline__ int opq(int v) {
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint32_t opqu(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// ---- wave / block reductions
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Sum over the lane's 16-lane row, in every lane of the row (rotations by 8,
// 4, 2, 1: pairs are symmetric, so every lane ends with the same value).
__device__ __forceinline__ float row_sum(float v) {
    v += dppf<0x128>(v);
    v += dppf<0x124>(v);
    v += dppf<0x122>(v);
    v += dppf<0x121>(v);
    return v;
}
__device__ __forceinline__ float lane_val(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wsum(float v) {
    v = row_sum(v);
    return (lane_val(v, 0) + lane_val(v, 16)) + (lane_val(v, 32) + lane_val(v, 48));
}
__device__ __forceinline__ u64 kmax_wave(u64 k) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const u64 other = ((u64)(uint32_t)__shfl_xor((int)(k >> 32), o, 64) << 32) |
                          (uint32_t)__shfl_xor((int)(k & 0xFFFFFFFFull), o, 64);
        k = max(k, other);
    }
    return k;
}
// Orderable key of (value, index): larger value wins, then the smaller index
// (torch.argmax's first maximal index, sunnynet/cli.py:41).
__device__ __forceinline__ u64 argmax_key(float v, int idx) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((u64)ord << 32) | (u64)(0xFFFFFFFFu - (uint32_t)idx);
}

// Block sum (wave-uniform result in every thread) through the NWV floats at
// red: one barrier. Consecutive sums use different red buffers, and any two
// uses of one buffer are separated by other barriers.
__device__ __forceinline__ float bsum(float v, float* red) {
    v = wsum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) red[w] = v;
    barrier_lds();
    float r[NWV];
#pragma unroll
    for (int i = 0; i < NWV; ++i) r[i] = red[i];
#pragma unroll
    for (int h = NWV / 2; h > 0; h >>= 1)
#pragma unroll
        for (int i = 0; i < h; ++i) r[i] = r[i] + r[i + h];
    return r[0];
}

// Two-pass LayerNorm statistics (sunnynet.c:198-210) over n values, element
// k * NT + tid in xv[k] (0 beyond n); red holds 2 NWV floats.
template <int N>
__device__ __forceinline__ void ln_stats(const float (&xv)[N], int n, float eps, float* red, float& mean,
                                         float& rstd) {
    const int tid = threadIdx.x;
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (k * NT + tid < n) sum += xv[k];
    mean = bsum(sum, red) * (1.0f / (float)n);
    float vs = 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (k * NT + tid < n) {
            const float d = xv[k] - mean;
            vs += d * d;
        }
    rstd = rsqrtf(bsum(vs, red + NWV) * (1.0f / (float)n) + eps);
}

// ---- jobs: the rows of one matrix a workgroup multiplies in one phase
//
// Rows j < n1 are r0 + j s0 and multiply x0; rows n1 <= j < n are r1 + (j - n1)
// and multiply x1 (LDS vectors in the staged layout). With two parts, waves
// 0 .. NWV/2-1 take the first and the others the second, so each wave
// multiplies one vector and keeps its slice of it in registers for the whole
// job. fp32: lane l holds float4 i of a row at k = 256 i + 4 l; the wave's
// rows form a flat list of items (row, i), nk4 = ceil(K / 256) items per row,
// and a batch is CAPF consecutive items (a row may straddle two batches: its
// per-lane partial sum carries over). INT4: a row is split over seg lanes
// (the next power of two >= its ng groups), one group of codes per lane; a
// unit is rpp = 64 / seg rows, a batch MU units.
//
// Everything but the weight pointers is the same in every layer, so each
// wave computes its share of each phase type once per launch (Geo, kept in
// LDS) and a phase only reads it back: the scalar unit, shared by the 16
// waves of a CU, is otherwise the bottleneck of a phase.
struct Geo {
    int K, n1, r0, s0, r1;   // job rows -> weight rows
    int base, cnt, wl, nwp;  // this wave's rows: base + wl + nwp m (cnt rows in its part)
    int nb;                  // batches of this wave
    int ng, lseg, rpp;       // INT4: groups per row, log2 lanes per row, rows per unit
    int nk4;                 // fp32: float4 items per row
    int xsel;                // multiplies x1 (1) or x0 (0)
    int nwu;                 // INT4: units of this wave
};
static_assert(sizeof(Geo) == 64, "Geo is read as four 16-byte words");

struct Job {
    const float* w;
    const uint16_t* h;
    const uint8_t* q;
    const float* sc;
    const l_f32* x;
    Geo g;
};

template <int BLK>
__device__ __forceinline__ Geo make_geo(int K, int n1, int n, int r0, int s0, int r1, int wv);

__device__ __forceinline__ int job_row(const Geo& g, int j) { return j < g.n1 ? g.r0 + j * g.s0 : g.r1 + (j - g.n1); }

// Weight formats of the template argument BLK: 0 fp32, 16 fp16 (both rows of
// K contiguous values), 32 / 64 INT4 groups.
constexpr bool is_i4(int blk) { return blk == 32 || blk == 64; }

template <int BLK>
struct Pool {
    static constexpr int QW = is_i4(BLK) ? BLK / 32 : 1;    // uint4 per INT4 group
    static constexpr int MU = 2;                            // INT4 units per batch
    float4 wf[BLK == 0 ? CAPF : 1];
    uint2 wh[BLK == 16 ? CAPF : 1];
    uint4 wq[is_i4(BLK) ? MU : 1][QW];
    float wsc[is_i4(BLK) ? MU : 1];
};

// The lane's slice of the job's input vector: fp32 nothing (read per item);
// INT4 the quads of its group (low and high halves), zero past the row.
template <int BLK>
struct XCache {
    float4 q[is_i4(BLK) ? BLK / 4 : 1];
};

template <int BLK>
__device__ __forceinline__ Geo make_geo(int K, int n1, int n, int r0, int s0, int r1, int wv) {
    Geo g;
    g.K = K; g.n1 = n1; g.r0 = r0; g.s0 = s0; g.r1 = r1;
    const bool two = n1 > 0 && n1 < n;
    const bool hi = two && wv >= NWV / 2;
    g.nwp = two ? NWV / 2 : NWV;
    g.wl = hi ? wv - NWV / 2 : wv;
    g.base = hi ? n1 : 0;
    g.cnt = two ? (hi ? n - n1 : n1) : n;
    g.xsel = hi ? 1 : 0;
    g.nwu = 0;
    const int nw = g.cnt > g.wl ? (g.cnt - g.wl + g.nwp - 1) / g.nwp : 0;   // the wave's rows
    if constexpr (!is_i4(BLK)) {
        g.nk4 = (K + 255) >> 8;
        g.ng = 0; g.lseg = 6; g.rpp = 1;
        g.nb = (nw * g.nk4 + CAPF - 1) / CAPF;
    } else {
        g.nk4 = 0;
        g.ng = K / BLK;
        g.lseg = g.ng <= 1 ? 0 : 32 - __clz(g.ng - 1);
        g.rpp = 64 >> g.lseg;
        const int nu = (g.cnt + g.rpp - 1) / g.rpp;
        g.nwu = nu > g.wl ? (nu - g.wl + g.nwp - 1) / g.nwp : 0;
        g.nb = (g.nwu + Pool<BLK>::MU - 1) / Pool<BLK>::MU;
    }
    return g;
}

// fp32: item m = b CAPF + s of a wave's list is float4 i of its row mr (one
// division per batch; the slots step through the list).
__device__ __forceinline__ void first_item(const Geo& g, int b, int& mr, int& i) {
    const int m = b * CAPF;
    mr = m / g.nk4;
    i = m - mr * g.nk4;
}
__device__ __forceinline__ void next_item(const Geo& g, int& mr, int& i) {
    if (++i == g.nk4) {
        i = 0;
        ++mr;
    }
}

// Batch b of J into P. Straight-line: every slot issues its loads (empty ones
// read element 0 of the matrix), so wait counts stay exact.
template <int BLK>
__device__ __forceinline__ void pool_load(const Job& J, int b, Pool<BLK>& P, int lane) {
    const Geo& g = J.g;
    if constexpr (!is_i4(BLK)) {
        int mr, i;
        first_item(g, b, mr, i);
#pragma unroll
        for (int s = 0; s < CAPF; ++s) {
            if (s > 0) next_item(g, mr, i);
            const int jl = g.wl + g.nwp * mr;
            const int k = i * 256 + lane * 4;
            const bool ok = jl < g.cnt && k < g.K;
            const int row = job_row(g, g.base + jl);
            const size_t off = ok ? (size_t)(uint32_t)(row * g.K + k) : 0;
            if constexpr (BLK == 16) P.wh[s] = ldgh4(J.h + off);
            else P.wf[s] = ldg4(J.w + off);
        }
    } else {
        constexpr int MU = Pool<BLK>::MU;
        const int lrow = lane >> g.lseg, lg = lane & ((1 << g.lseg) - 1);
#pragma unroll
        for (int s = 0; s < MU; ++s) {
            const int jl = (g.wl + g.nwp * (b * MU + s)) * g.rpp + lrow;
            const bool ok = jl < g.cnt && lg < g.ng;
            const int row = job_row(g, g.base + jl);
            const uint32_t qo = (uint32_t)(row * (g.K / 2) + lg * (BLK / 2));
            const uint32_t so = (uint32_t)(row * g.ng + lg);
#pragma unroll
            for (int qq = 0; qq < Pool<BLK>::QW; ++qq) P.wq[s][qq] = ldgq(J.q + (ok ? qo + 16 * qq : 0));
            P.wsc[s] = ldg(J.sc + (ok ? so : 0));
        }
    }
}

template <int BLK>
__device__ __forceinline__ void xcache_load(const Job& J, XCache<BLK>& X, int lane) {
    if constexpr (is_i4(BLK)) {
        const Geo& g = J.g;
        const int lg = min(lane & ((1 << g.lseg) - 1), g.ng - 1);
#pragma unroll
        for (int q = 0; q < BLK / 4; ++q) X.q[q] = lds4(J.x + 4 * (q * (g.ng + kStagePad) + lg));
    }
}

// epi(j, row, value, writer): `writer` is true on exactly one lane per row.
// Every slot's loads are valid addresses; only rows of the job reach epi.
template <int BLK, class Epi>
__device__ __forceinline__ void compute_f32(const Job& J, int b, const Pool<BLK>& P, int lane, float& pacc,
                                            Epi&& epi) {
    const Geo& g = J.g;
    float4 xs[CAPF];
    int mr0, i0;
    first_item(g, b, mr0, i0);
    {
        int mr = mr0, i = i0;
#pragma unroll
        for (int s = 0; s < CAPF; ++s) {
            if (s > 0) next_item(g, mr, i);
            xs[s] = lds4(J.x + min(i * 256 + lane * 4, g.K - 4));
        }
    }
    int mr = mr0, i = i0;
#pragma unroll
    for (int s = 0; s < CAPF; ++s) {
        if (s > 0) next_item(g, mr, i);
        const int jl = g.wl + g.nwp * mr;
        if (i * 256 + lane * 4 < g.K) {
            const float4 w4 = BLK == 16 ? h4f(P.wh[s]) : P.wf[s];
            pacc = pacc + (fmaf(w4.x, xs[s].x, w4.y * xs[s].y) + fmaf(w4.z, xs[s].z, w4.w * xs[s].w));
        }
        if (i == g.nk4 - 1) {
            const float v = wsum(pacc);
            pacc = 0.0f;
            if (jl < g.cnt) epi(g.base + jl, job_row(g, g.base + jl), v, lane == 0);
        }
    }
}

template <int BLK, class Epi>
__device__ __forceinline__ void compute_i4(const Job& J, int b, const Pool<BLK>& P, const XCache<BLK>& X, int lane,
                                           Epi&& epi) {
    constexpr int MU = Pool<BLK>::MU;
    constexpr int NW = BLK / 8;                  // 32-bit words of codes per group
    const Geo& g = J.g;
    const int seg = 1 << g.lseg;
    const int lrow = lane >> g.lseg, lg = lane & (seg - 1);
    const bool lane_ok = lg < g.ng;
    // Units of this batch that hold rows (the rest are skipped, uniformly).
    const int nvu = min(MU, g.nwu - b * MU);
    float acc[MU];
#pragma unroll
    for (int s = 0; s < MU; ++s) {
        acc[s] = 0.0f;
        if (s >= nvu) continue;
        // (q - 8) * scale as one rounding: fma(q, scale, -8 scale), with
        // -8 scale exact (quant.c:82-83 dequantization, bit-identical).
        const float sc = P.wsc[s], m8 = -8.0f * sc;
        // Four independent partial sums (one per byte of a code word) keep
        // the FMA dependency chains short.
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const uint4& qq = P.wq[s][w >> 2];
            const int wi = w & 3;
            const uint32_t word = wi == 0 ? qq.x : wi == 1 ? qq.y : wi == 2 ? qq.z : qq.w;
            // Byte 4w + e holds element 4w + e (low nibble) and 4w + e + BLK/2
            // (high nibble). The nibble words are opaque to the optimizer, so
            // each code converts with one v_cvt_f32_ubyte<e> (known-bits
            // folding would otherwise emit a bit-field extract first).
            const uint32_t lo = opqu(word & 0x0F0F0F0Fu), hi = opqu((word >> 4) & 0x0F0F0F0Fu);
            const float4 xl = X.q[w], xh = X.q[w + NW];
            a[0] = fmaf(fmaf((float)(lo & 0xFFu), sc, m8), xl.x, a[0]);
            a[1] = fmaf(fmaf((float)((lo >> 8) & 0xFFu), sc, m8), xl.y, a[1]);
            a[2] = fmaf(fmaf((float)((lo >> 16) & 0xFFu), sc, m8), xl.z, a[2]);
            a[3] = fmaf(fmaf((float)(lo >> 24), sc, m8), xl.w, a[3]);
            a[0] = fmaf(fmaf((float)(hi & 0xFFu), sc, m8), xh.x, a[0]);
            a[1] = fmaf(fmaf((float)((hi >> 8) & 0xFFu), sc, m8), xh.y, a[1]);
            a[2] = fmaf(fmaf((float)((hi >> 16) & 0xFFu), sc, m8), xh.z, a[2]);
            a[3] = fmaf(fmaf((float)(hi >> 24), sc, m8), xh.w, a[3]);
        }
        acc[s] = lane_ok ? (a[0] + a[1]) + (a[2] + a[3]) : 0.0f;
    }
    if (seg >= 16) {
#pragma unroll
        for (int s = 0; s < MU; ++s)
            if (s < nvu) acc[s] = row_sum(acc[s]);
        if (seg > 16) {
#pragma unroll
            for (int s = 0; s < MU; ++s) {
                if (s >= nvu) continue;
                const float r0 = lane_val(acc[s], 0), r1 = lane_val(acc[s], 16);
                const float r2 = lane_val(acc[s], 32), r3 = lane_val(acc[s], 48);
                acc[s] = seg == 64 ? (r0 + r1) + (r2 + r3) : (lane < 32 ? r0 + r1 : r2 + r3);
            }
        }
    } else {
        for (int o = seg >> 1; o > 0; o >>= 1)
#pragma unroll
            for (int s = 0; s < MU; ++s)
                if (s < nvu) acc[s] += __shfl_xor(acc[s], o, 64);
    }
#pragma unroll
    for (int s = 0; s < MU; ++s) {
        const int jl = (g.wl + g.nwp * (b * MU + s)) * g.rpp + lrow;
        if (s < nvu && jl < g.cnt) epi(g.base + jl, job_row(g, g.base + jl), acc[s], lg == 0);
    }
}

template <int BLK, class Epi>
__device__ __forceinline__ void compute(const Job& J, int b, const Pool<BLK>& P, const XCache<BLK>& X, int lane,
                                        float& pacc, Epi&& epi) {
    if constexpr (!is_i4(BLK)) compute_f32<BLK>(J, b, P, lane, pacc, epi);
    else compute_i4<BLK>(J, b, P, X, lane, epi);
}

// Runs every batch of J (batch 0 is already in p0): batches alternate between
// two pools, and each is issued before the previous one is multiplied. INT4
// keeps p0 read-only and streams the later batches through two pools local
// to the job, so no path leaves p0 different (a pool rewritten on one path
// costs register copies, and a wait for their loads, where the paths join:
// 188.6 -> 184.0 us per 100M step); fp32 rotates p0 and p1 (the local pools
// measured 224.4 -> 236.3 us there). The loads of a batch past the last read
// element 0 of the matrix (unused), so every path of the loop issues the
// same loads and the wait counts stay exact. A wave with no rows does
// nothing.
#ifdef SNHIP_PERSIST_PROF
__device__ unsigned long long g_jprof[64 * 4];
#define JPROF(i) do { if (probe && lane == 0) g_jprof[(i) * 16 + wv] = wall_clock64(); } while (0)
#else
#define JPROF(i) do { } while (0)
#endif
template <int BLK, class Epi>
__device__ __forceinline__ void run_job(const Job& J, Pool<BLK>& p0, Pool<BLK>& p1, int wv, int lane, Epi&& epi,
                                        bool probe = false) {
    JPROF(0);
    const int nb = J.g.nb;
    if (nb == 0) return;
    XCache<BLK> X;
    xcache_load<BLK>(J, X, lane);
    JPROF(1);
    float pacc = 0.0f;
    if (nb == 1) {
        // One batch (the common case in the layer phases): nothing else to
        // issue, and its own copy of the product code waits for p0 alone.
        JPROF(2);
        compute<BLK>(J, 0, p0, X, lane, pacc, epi);
        JPROF(3);
        return;
    }
    if constexpr (is_i4(BLK)) {
        Pool<BLK> q0, q1;
        pool_load<BLK>(J, 1, q1, lane);
        compute<BLK>(J, 0, p0, X, lane, pacc, epi);
        for (int b = 1; b < nb; b += 2) {
            pool_load<BLK>(J, b + 1, q0, lane);
            compute<BLK>(J, b, q1, X, lane, pacc, epi);
            pool_load<BLK>(J, b + 2, q1, lane);
            if (b + 1 < nb) compute<BLK>(J, b + 1, q0, X, lane, pacc, epi);
        }
    } else {
        for (int b = 0; b < nb; b += 2) {
            pool_load<BLK>(J, b + 1, p1, lane);
            compute<BLK>(J, b, p0, X, lane, pacc, epi);
            pool_load<BLK>(J, b + 2, p0, lane);
            if (b + 1 < nb) compute<BLK>(J, b + 1, p1, X, lane, pacc, epi);
        }
    }
}

// Batch 0 of the next job into p0 (nothing for a wave with no rows in it).
template <int BLK>
__device__ __forceinline__ void prefetch_job(const Job& J, Pool<BLK>& p0, int lane) {
    if (J.g.nb > 0) pool_load<BLK>(J, 0, p0, lane);
}

// Index of element i of a K-long vector in the staged LDS layout: fp32 plain;
// INT4 quad-major, so lane g of a row reads its group's quads q at
// (q (ng + 2) + g) * 4 (consecutive lanes, consecutive 16 bytes). The stride
// of ng + 2 groups puts the 64 floats a wave stages (8 quads of 2 groups)
// on 64 different banks; with a stride of ng they shared 8.
template <int BLK>
__device__ __forceinline__ int sidx(int i, int K) {
    if constexpr (!is_i4(BLK)) return i;
    else return ((((i % BLK) >> 2) * (K / BLK + kStagePad) + i / BLK) << 2) + (i & 3);
}

#ifdef SNHIP_PERSIST_PROF
// Phase timestamps of workgroup 0 (wall clock), for profiling builds only.
__device__ unsigned long long g_prof[2048];
__device__ unsigned long long g_clk[4];
#define PROF(idx) do { if (wg == 0 && lane == 0 && step == 3) g_prof[(idx) * 4 + wv] = wall_clock64(); \
    if (wg == 0 && tid == 0 && step == 3 && (idx) == 1) { g_clk[0] = wall_clock64(); g_clk[1] = clock64(); } \
    if (wg == 0 && tid == 0 && step == 3 && (idx) == 8 * 48 + 1) { g_clk[2] = wall_clock64(); g_clk[3] = clock64(); } } while (0)
#else
#define PROF(idx) do { } while (0)
#endif

// One code path serves every phase (the instruction cache holds the whole
// step loop): phase p of a step is A, B, C, D of layer p / 4 for p < 4 L, then
// the head H; per-phase differences are uniform branches on the phase type.
template <int BLK>
__global__ __launch_bounds__(NT) void k_decode_persist(PersistArgs a) {
    // input vector of the current products, and the old state s (W_eff's
    // input in phase A), in the staged layout (INT4: K + kStagePad BLK floats)
    __shared__ __align__(16) float xin[kMaxK + kStagePad * 64];
    __shared__ __align__(16) float xs2[kMaxD + kStagePad * 64];
    __shared__ float xres[kMaxD];                 // x of the layer (residual)
    __shared__ float res[kMaxK + kMaxD];          // products of the current phase, by job row
    __shared__ float sown[kMaxD];                 // s' of the owned channels
    __shared__ float sfbl[kMaxD];                 // W_eff s_old of the owned channels
    __shared__ float red[2 * NWV];
    __shared__ u64 kred[NWV];
    __shared__ int sflag;
    __shared__ PLayer ltab[kPersistMaxL];          // the layer table (LDS reads, no scalar misses)
    __shared__ Geo geo[5][NWV];                   // each wave's share of each phase type

    int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    auto fresh = [&]() {
        tid = opq(tid);
        lane = tid & 63;
    };
    const int D = a.D, I = a.I, R = a.R, L = a.L;
    // Independent sequences run on equal slices of the grid: this workgroup
    // is workgroup wg of sequence sq's G (one sequence: sq = 0, G = the grid).
    const int NI = a.ni > 1 ? a.ni : 1;
    const int G = gridDim.x / NI, sq = blockIdx.x / G, wg = blockIdx.x - sq * G;
    if (NI > 1) {
        a.s += (size_t)sq * L * D;
        a.hist += (size_t)sq * L * KH * D;
        a.ex += (size_t)sq * 2 * kPersistExWords;
        a.sx += (size_t)sq * L * 2 * D;
        a.tok_in += sq;
        if (a.out_tok) a.out_tok += sq;
        if (a.logits) a.logits += (size_t)sq * a.vocab;
    }
    const int cpw = D / G, c0 = wg * cpw;                     // owned channels
    const int grp0 = c0 >> 3, ngrp = cpw >= 8 ? cpw >> 3 : 1; // owned channel groups
    const PollCtl pc{a.err, a.spin_limit};
    for (int i = tid; i < L * (int)sizeof(PLayer) / 4; i += NT)
        ((uint32_t*)ltab)[i] = ((const uint32_t*)a.layers)[i];
    const PLayer* lt = ltab;
    u64* ex0 = a.ex;
    auto exs = [&](unsigned e) -> u64* { return ex0 + (size_t)(e & 1u) * kPersistExWords; };

    if (tid == 0) sflag = 0;
    barrier_lds();
    // Leaves the kernel (in every thread of the workgroup) when any thread's
    // poll failed.
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
    // The rows this workgroup multiplies in phase p (A: its V rows, then the
    // W_eff rows of its channels; B: the U rows of its channel groups; C: its
    // W_z rows; D: the W_c rows of its channels; H: its head rows): this
    // wave's geometry of each phase type, once per launch.
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

    Pool<BLK> p0, p1;   // p1: fp32 jobs of more than one batch
    prefetch_job<BLK>(job(0), p0, lane);

    unsigned ep = 0;                  // epoch of the last exchange produced
    const unsigned stall = a.stall;   // > 0 only to test the time-out path
    int tok = a.tok_in[0];
    float* ring_wg = a.ring + (size_t)blockIdx.x * L * KH * D;
    constexpr int WMAX = 2 * PD;      // exchange words per thread (A: x and s)
    static_assert(WMAX >= PK, "gather words");

    for (int step = 0; step < a.n_steps; ++step) {
        const bool last = step + 1 == a.n_steps;
        const bool tok_ok = tok >= 0 && tok < a.vocab;
        const float* erow = a.embed + (size_t)(tok_ok ? tok : 0) * D;
        u64 best = 0ull;
        for (int p = 0; p < NP; ++p) {
            fresh();
            const int t = p < 4 * L ? (p & 3) : 4;        // 0 A, 1 B, 2 C, 3 D, 4 H
            const int l = min(p >> 2, L - 1);
            const PLayer* Ly = lt + l;
            // ---- the phase's input: the vector it multiplies (A: x, B: v,
            // C: u, D: z, H: x), for A also the old state s (words PD..)
            const int n0 = t == 1 ? R : t == 3 ? I : D;
            const unsigned e0 = ep + stall, e1 = (unsigned)step + stall;
            const u64* s0 = exs(ep);
            const u64* s1 = a.sx + ((size_t)l * 2 + ((step - 1) & 1)) * D;
            const bool plain0 = t == 0 && l == 0;          // x = the token's embedding row
            const bool plain1 = step == 0;                 // s = the handle's state
            const bool ln = t == 0 || t >= 3;
            const float* gp = t == 0 ? Ly->ni_g : t == 3 ? Ly->nm_g : a.no_g;
            const float* cp = t == 0 ? Ly->ni_c : t == 3 ? Ly->nm_c : a.no_c;
            u64 w[WMAX];
            float gv[PK], cv[PK], dv[KT][PD], hv[KH][PD], dl[PD];
            float* ring_l = ring_wg + (size_t)l * KH * D;
            auto word_in = [&](int k) -> bool {            // word k holds an element
                if (t == 0) return (k % PD) * NT + tid < D;
                return k < PK && k * NT + tid < n0;
            };
            auto addr = [&](int k) -> const u64* {
                if (t == 0 && k >= PD) return s1 + min((k - PD) * NT + tid, D - 1);
                return s0 + min(k * NT + tid, n0 - 1);
            };
            auto want = [&](int k) { return t == 0 && k >= PD ? e1 : e0; };
#pragma unroll
            for (int k = 0; k < WMAX; ++k) {
                const bool s_word = t == 0 && k >= PD;
                const int i = min((s_word ? k - PD : k) * NT + tid, (s_word ? D : n0) - 1);
                if (!word_in(k)) w[k] = ll_ready(0.0f, want(k));
                else if (s_word ? plain1 : plain0)
                    w[k] = ll_ready(ldg((s_word ? a.s + (size_t)l * D : erow) + i), want(k));
                else w[k] = ll_get(addr(k));
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
#pragma unroll
                for (int k = 0; k < PD; ++k) {
                    const int i = min(k * NT + tid, D - 1);
#pragma unroll
                    for (int u = 0; u < KT; ++u) dv[u][k] = ldg(Ly->dw + (size_t)u * D + i);
#pragma unroll
                    for (int u = 0; u < KH; ++u) {
                        // raw of step - 1 - u: this workgroup's ring, or the
                        // handle's history (newest first) before the launch
                        const int age = step - 1 - u;
                        hv[u][k] = age >= 0 ? ring_l[(size_t)(age % KH) * D + i]
                                            : ldg(a.hist + ((size_t)l * KH + (u - step)) * D + i);
                    }
                }
            }
            if (t == 1) {
#pragma unroll
                for (int k = 0; k < PD; ++k) dl[k] = ldg(Ly->delta + min(c0 + k * NT + tid, D - 1));
            }
            PROF(p * 8 + 0);
            const bool polled = ll_spin(w, addr, want, pc);
            PROF(p * 8 + 1);
            float xv[PK];
#pragma unroll
            for (int k = 0; k < PK; ++k) {
                const bool in = k * NT + tid < n0 && (t != 0 || k < PD);
                xv[k] = !in ? 0.0f : (plain0 && !tok_ok) ? __builtin_nanf("") : ll_f(w[k]);
            }
            if (!agree(polled)) return;
            float mean = 0.0f, rstd = 0.0f;
            if (ln) ln_stats(xv, n0, a.eps, red, mean, rstd);
            PROF(p * 8 + 2);
#pragma unroll
            for (int k = 0; k < PK; ++k) {
                const int i = k * NT + tid;
                if (i >= n0 || (t == 0 && k >= PD)) continue;
                float y = ln ? (xv[k] - mean) * rstd * gv[k] + cv[k] : xv[k];
                if (k < PD && t == 0) {
                    // sunnynet.c:227-233: acc = raw w[K-1] + hist[0] w[K-2] + ...
                    float acc = y * dv[KT - 1][k];
#pragma unroll
                    for (int u = 0; u < KH; ++u) acc = acc + hv[u][k] * dv[KT - 2 - u][k];
                    ring_l[(size_t)(step % KH) * D + i] = y;
                    xs2[sidx<BLK>(i, D)] = ll_f(w[PD + k]);
                    xres[i] = xv[k];
                    y = y + acc;
                }
                xin[sidx<BLK>(i, n0)] = y;
            }
            barrier_lds();
            PROF(p * 8 + 3);
            // ---- the products; every phase but H leaves them in res by job row
            const bool head = t == 4;
            float* lgp = head && last ? a.logits : nullptr;
            run_job<BLK>(job(p), p0, p1, wv, lane, [&](int j, int row, float v, bool wr) {
                if (!wr) return;
                if (!head) {
                    res[j] = v;
                } else {
                    if (lgp) lgp[row] = v;
                    best = max(best, argmax_key(v, row));
                }
            }, wg == 0 && step == 3 && p == 4);
            PROF(p * 8 + 4);
            barrier_lds();
            PROF(p * 8 + 5);
            // ---- the phase's outputs
            const unsigned epv = ++ep;
            u64* out = exs(epv);
            if (t == 0) {
                for (int j = tid; j < nV + cpw; j += NT) {
                    if (j < nV) ll_putf(out + wg + j * G, res[j], epv);
                    else sfbl[j - nV] = res[j];
                }
            } else if (t == 1) {
                // sunnynet.c:248-262: competitive gate within the group of 8,
                // decay gate, state update
                u64* sout = a.sx + ((size_t)l * 2 + (step & 1)) * D;
#pragma unroll
                for (int k = 0; k < PD; ++k) {
                    const int c = k * NT + tid;
                    if (c >= cpw) continue;
                    const int i = c0 + c, jj = i & 7, base = ((i >> 3) - grp0) * 16;
                    const float gi = res[base + 8 + jj];
                    const float uu = res[base + jj] * (sgm(gi - res[base + 8 + ((jj + 1) & 7)]) *
                                                       sgm(gi - res[base + 8 + ((jj + 2) & 7)]));
                    float pg = 1.0f - dl[k] * (1.0f - sgm(gi));
                    if (a.clamp && pg < a.p_floor) pg = a.p_floor;
                    const float sn = pg * xs2[sidx<BLK>(i, D)] + (1.0f - pg) * uu;
                    ll_putf(out + i, uu, epv);
                    ll_putf(sout + i, sn, (unsigned)step + 1);
                    sown[c] = sn;
                }
            } else if (t == 2) {
                const float at = Ly->a_tanh;
                for (int j = tid; j < nZ; j += NT) {
                    const float v = res[j];
                    ll_putf(out + wg + j * G, v * (1.0f + 0.5f * at / (1.0f + fabsf(v))), epv);
                }
            } else if (t == 3) {
                const float bg = Ly->b_gain;
                for (int c = tid; c < cpw; c += NT)
                    ll_putf(out + c0 + c, res[c] + (bg * sown[c] + sfbl[c] + xres[c0 + c]), epv);
            } else if (a.greedy) {
                best = kmax_wave(best);
                if (lane == 0) kred[wv] = best;
                barrier_lds();
                if (tid < 2) {
                    u64 kk = kred[0];
#pragma unroll
                    for (int i = 1; i < NWV; ++i) kk = max(kk, kred[i]);
                    ll_put(out + 2 * wg + tid, tid == 0 ? (uint32_t)(kk >> 32) : (uint32_t)kk, epv);
                }
            }
            PROF(p * 8 + 6);
            // ---- the next phase's first weights (the next step's first phase
            // after H)
            prefetch_job<BLK>(job(p + 1 < NP ? p + 1 : 0), p0, lane);
            PROF(p * 8 + 7);
        }
        if (!a.greedy) break;
        fresh();
        // ---------------- T: every workgroup reduces the keys to the same token
        {
            const unsigned epx = ep + stall;
            const u64* ksrc = exs(ep);
            u64 w[2 * KPT];
            auto addr = [&](int k) { return ksrc + 2 * min((k >> 1) * NT + tid, G - 1) + (k & 1); };
#pragma unroll
            for (int k = 0; k < 2 * KPT; ++k)
                w[k] = (k >> 1) * NT + tid < G ? ll_get(addr(k)) : ll_ready(0.0f, epx);
            if (!agree(ll_spin(w, addr, [&](int) { return epx; }, pc))) return;
            u64 kk = 0ull;
#pragma unroll
            for (int q = 0; q < KPT; ++q)
                if (q * NT + tid < G) kk = max(kk, ((u64)(uint32_t)w[2 * q] << 32) | (uint32_t)w[2 * q + 1]);
            kk = kmax_wave(kk);
            if (lane == 0) kred[wv] = kk;
            barrier_lds();
            kk = kred[0];
#pragma unroll
            for (int i = 1; i < NWV; ++i) kk = max(kk, kred[i]);
            tok = (int)(0xFFFFFFFFu - (uint32_t)(kk & 0xFFFFFFFFull));
            if (wg == 0 && tid == 0) a.out_tok[(size_t)step * NI] = tok;
            barrier_lds();
        }
    }

    // Owners write back the state and the history (newest first) of their
    // channels, for every layer. The ring entries are this thread's own
    // stores; a history entry older than the launch comes from the handle's
    // history, read before the entry it would overwrite.
    const int T = a.n_steps;
    for (int l = 0; l < L; ++l) {
        const float* ring_l = ring_wg + (size_t)l * KH * D;
        const u64* sl = a.sx + ((size_t)l * 2 + ((T - 1) & 1)) * D;
#pragma unroll
        for (int k = 0; k < PD; ++k) {
            const int i = k * NT + tid;
            if (i >= D || i < c0 || i >= c0 + cpw) continue;
            a.s[(size_t)l * D + i] = ll_f(ll_get(sl + i));
#pragma unroll
            for (int j = KH - 1; j >= 0; --j) {
                const int age = T - 1 - j;
                float* hj = a.hist + ((size_t)l * KH + j) * D + i;
                *hj = age >= 0 ? ring_l[(size_t)(age % KH) * D + i] : a.hist[((size_t)l * KH + (j - T)) * D + i];
            }
        }
    }
}

const void* kernel_for(int blk) {
    return blk == 0 ? (const void*)k_decode_persist<0>
         : blk == 16 ? (const void*)k_decode_persist<16>
         : blk == 32 ? (const void*)k_decode_persist<32>
                     : (const void*)k_decode_persist<64>;
}

}  // namespace SNHIP_PERSIST_NS
}  // namespace snhip
