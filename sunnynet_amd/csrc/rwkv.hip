// RWKV-7 decode on gfx950 (include/snhip_rwkv7.h).
//
// The math is the reference's C runtime, sunnynet/runtime/rwkv7.c:143-360:
//   x = LN_0(E[token]); per layer:
//     xn = LN_1(x); d = shift_0 - xn; x_{r,w,k,v,a,g} = xn + lerp_* d
//     r, k, v = W_r x_r, W_k x_k, W_v x_v
//     w = exp(-sig(W_2 tanh(W_1 x_w) + w_0) / sqrt(e))
//     v = v + (v_first - v) sig(V_2 V_1 x_v + v_0)   (layer 0: v_first = v)
//     a = sig(A_2 A_1 x_a + a_0);  g = G_2 sig(G_1 x_g)
//     kk = k kk_w;  k = k + k (a - 1) ka_w
//     per head: S = S diag(w) - (S kk^) (kk^ a)^T + v k^T;  y = S r
//               y = (GroupNorm(y) + (r . k rk_w) v) g
//     x += W_o y;  shift_0 = xn
//     xn2 = LN_2(x);  x += W_cv relu(W_ck (xn2 + cmk_lerp (shift_1 - xn2)))^2;  shift_1 = xn2
//   logits = W_head LN_out(x)
//
// One step is a short sequence of kernels on the handle's stream (captured
// into a HIP graph and replayed); every kernel processes all B sequences and
// follows the reference's rounding order (rkseq.hip): row LayerNorms with the
// token-shift mixes, matrix products as sequential fmaf chains on the matrix
// cores (with the LoRA tanh / sigmoid, relu^2 and residual epilogues), and one
// kernel per head for the decay, mixes, normalized kk, the 64 x 64 state
// update and read-out, group norm, bonus and gate. A step therefore gives the
// reference's logits bit for bit on the same weights. Single-sequence steps
// may instead run as one cooperative launch (rkpersist.hip).
// Weights live row-major (out, in), fp32 or INT4.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "common.h"
#include "gemv.h"
#include "rkpersist.h"
#include "rkseq.h"
#include "snhip.h"
#include "snhip_rwkv7.h"

namespace snhip {
namespace {

constexpr int kRkMagic = 0x4B57524B;   // rwkv7.c:36
constexpr int kRkVersion = 3;
constexpr int kRkBlobBlock = 64;       // INT4 group of the v3 blob (rwkv7.c:40)
constexpr float kR2 = 0.6065306597126334f;   // 1/sqrt(e), rwkv7.c:38
constexpr float kEpsGroup = 6.4e-4f;          // rwkv7.c:39
constexpr int kHS = 64;                        // head size this backend runs
constexpr int kMaxRank = 256;                  // rwkv7.c: LoRA scratch of 256
constexpr int kMaxDim = 4096;                  // row kernels hold one row in LDS

// (in, out) row-major -> (out, in) row-major, 32x32 tiles through LDS.
__global__ void k_rk_transpose(const float* __restrict__ src, float* __restrict__ dst, int in, int out) {
    __shared__ float tile[32][33];
    const int bo = blockIdx.x * 32, bi = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int r = ty; r < 32; r += 8) {
        const int i = bi + r, o = bo + tx;
        if (i < in && o < out) tile[r][tx] = src[(size_t)i * out + o];
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int o = bo + r, i = bi + tx;
        if (o < out && i < in) dst[(size_t)o * in + i] = tile[tx][r];
    }
}

// Per-block partial maxima of logits rows (GEMM head): grid (nblk, B).
__global__ __launch_bounds__(256) void k_rk_argmax_partial(const float* __restrict__ logits, int V,
                                                           unsigned long long* __restrict__ part) {
    __shared__ unsigned long long red[256];
    const int b = blockIdx.y, nblk = gridDim.x;
    const int chunk = (V + nblk - 1) / nblk;
    const int lo = blockIdx.x * chunk, hi = min(V, lo + chunk);
    unsigned long long k = 0ull;
    for (int i = lo + (int)threadIdx.x; i < hi; i += 256) k = max(k, argmax_key(logits[(size_t)b * V + i], i));
    red[threadIdx.x] = k;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    if (threadIdx.x == 0) part[(size_t)b * nblk + blockIdx.x] = red[0];
}

// Greedy token of each sequence from the per-block maxima (first maximal
// index); writes it to tok (the next step's input) and to out at the device
// step counter; the last block to finish advances the counter.
__global__ __launch_bounds__(256) void k_rk_finalize(const unsigned long long* __restrict__ part,
                                                     int nblk, int B, int32_t* __restrict__ tok,
                                                     int32_t* __restrict__ out,
                                                     int32_t* __restrict__ counter,
                                                     int32_t* __restrict__ done, int cap) {
    __shared__ unsigned long long red[256];
    const int b = blockIdx.x;
    unsigned long long k = 0ull;
    for (int i = threadIdx.x; i < nblk; i += 256) k = max(k, part[(size_t)b * nblk + i]);
    red[threadIdx.x] = k;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int32_t tk = (int32_t)(0xFFFFFFFFu - (uint32_t)(red[0] & 0xFFFFFFFFull));
        const int step = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        tok[b] = tk;
        if ((long)step * B + b < (long)cap) out[(size_t)step * B + b] = tk;
        __threadfence();
        if (atomicAdd(done, 1) == B - 1) {
            *done = 0;
            __hip_atomic_store(counter, step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// A weight matrix, row-major (M, Kd): fp32 w, or INT4 q + sc with group block.
struct RMat {
    int M = 0, Kd = 0;
    float* w = nullptr;
    uint8_t* q = nullptr;
    float* sc = nullptr;
    int block = 0;
    float* w4 = nullptr;   // the tiled fp32 form the per-kernel steps multiply (or null)
};

struct RkLayer {
    const float *ln1w, *ln1b, *ln2w, *ln2b, *lerp, *w0, *a0, *v0, *kk, *ka, *rk, *lnxw, *lnxb, *cmk_lerp;
    int Rw, Ra, Rv, Rg;
    RMat r, k, v, o, w1, w2, a1, a2, v1, v2, g1, g2, cmk, cmv;
};

}  // namespace
}  // namespace snhip

struct SnHipRwkv7 {
    int L = 0, D = 0, HS = 0, NH = 0, F = 0, vocab = 0, max_batch = 1, wfmt = 0, block = 32;
    float eps = 0.f;
    std::vector<snhip::RkLayer> layers;
    const float *en_w = nullptr, *en_b = nullptr, *on_w = nullptr, *on_b = nullptr, *embed = nullptr;
    snhip::RMat head;
    float *S = nullptr, *shift = nullptr;
    float *x = nullptr, *X6 = nullptr, *r = nullptr, *k = nullptr, *v = nullptr, *lo = nullptr,
          *dw = nullptr, *da = nullptr, *dv = nullptr, *g = nullptr, *y = nullptr, *vfirst = nullptr,
          *xk2 = nullptr, *ck = nullptr, *nrm = nullptr, *logits = nullptr;
    int32_t* tok = nullptr;
    unsigned long long* best = nullptr;
    int32_t *counter = nullptr, *done = nullptr, *tok_hist = nullptr;
    int hist_cap = 0;
    std::vector<void*> allocs;
    hipStream_t stream = nullptr, work = nullptr;
    hipEvent_t ev_in = nullptr, ev_out = nullptr;
    std::map<std::tuple<int, const void*, int>, hipGraphExec_t> graphs;
    bool use_graphs = true;
    bool fuse_ups = true;   // LoRA up-projections inside the heads kernel (SNHIP_RKQ_FUSE_UPS=0: apart)
    // One-sequence steps as one cooperative launch each (rkpersist.hip);
    // p_grid = 0 when off (SNHIP_RK_PERSIST=0, or a shape it does not take).
    int p_grid = 0;
    bool p_exact = false;                 // the kernel is k_rk_exact (else k_rk_persist)
    // Steps of B = 2..p_mi_max sequences: the same kernel on a slice of
    // p_mi_grid[B] workgroups per sequence, one launch for all; the words
    // hold p_mi_max sequences' slabs, p_seq_words apart.
    int p_mi_max = 0;
    int p_mi_grid[snhip::kRkPMiMax + 1] = {};
    size_t p_seq_words = 0;
    snhip::RkPArgs p_args{};
    unsigned p_epoch = 0;                 // the last epoch a persistent launch used
    unsigned long long* p_words = nullptr;   // exchange slabs and key words (zeroed: epoch 0)
    size_t p_nwords = 0;
    unsigned* p_err = nullptr;
    unsigned p_spin = 1u << 22;
    // A persistent step timed out after some layers had written S and shift in
    // place: every stepping call fails until snhip_rk_reset or set_state.
    int poisoned = 0;
    int ready = 0;
};

namespace snhip {
namespace {

template <typename T>
T* ralloc(SnHipRwkv7* m, size_t n) {
    void* p = nullptr;
    if (hipMalloc(&p, n * sizeof(T) > 0 ? n * sizeof(T) : 4) != hipSuccess) return nullptr;
    m->allocs.push_back(p);
    return static_cast<T*>(p);
}

void free_rk(SnHipRwkv7* m) {
    if (!m) return;
    for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
    if (m->ev_in) (void)hipEventDestroy(m->ev_in);
    if (m->ev_out) (void)hipEventDestroy(m->ev_out);
    if (m->work) (void)hipStreamDestroy(m->work);
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

// Tag-prefixed tensor stream of the v3 blob (rwkv7.c:380-420).
struct Cur {
    const uint8_t* p;
    const uint8_t* end;
    bool ok;
};

const float* take_vec(Cur& c, size_t n) {
    if (!c.ok || (size_t)(c.end - c.p) < 4 + n * sizeof(float)) { c.ok = false; return nullptr; }
    int32_t tag;
    memcpy(&tag, c.p, 4);
    if (tag != 0) { c.ok = false; return nullptr; }
    c.p += 4;
    const float* r = reinterpret_cast<const float*>(c.p);
    c.p += n * sizeof(float);
    return r;
}

bool upload(SnHipRwkv7* m, const float*& dst, const float* src, size_t n) {
    float* d = ralloc<float>(m, n);
    if (!d || hipMemcpy(d, src, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) return false;
    dst = d;
    return true;
}

// A matrix y = M x with `in` inputs and `out` outputs, into (out, in) rows:
// tag 0 (fp32 M^T) is transposed on the device and, for INT4, quantized when
// block divides in; tag 1 (INT4, group 64) stays INT4 or is dequantized.
bool take_mat(SnHipRwkv7* m, Cur& c, RMat& M, int in, int out, float* tmp0, float* tmp1) {
    M.M = out;
    M.Kd = in;
    if (!c.ok || (size_t)(c.end - c.p) < 4) { c.ok = false; return false; }
    int32_t tag;
    memcpy(&tag, c.p, 4);
    c.p += 4;
    const size_t n = (size_t)in * out;
    if (tag == 0) {
        if ((size_t)(c.end - c.p) < n * sizeof(float)) { c.ok = false; return false; }
        if (hipMemcpy(tmp0, c.p, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) return false;
        c.p += n * sizeof(float);
        hipLaunchKernelGGL(k_rk_transpose, dim3((out + 31) / 32, (in + 31) / 32), dim3(256), 0, nullptr,
                           tmp0, tmp1, in, out);
        if (hipGetLastError() != hipSuccess) return false;
        if (m->wfmt == SNHIP_WEIGHTS_INT4 && in % m->block == 0) {
            M.block = m->block;
            M.q = ralloc<uint8_t>(m, n / 2);
            M.sc = ralloc<float>(m, n / M.block);
            if (!M.q || !M.sc) return false;
            if (launch_quant_i4(tmp1, M.q, M.sc, out, in, M.block, nullptr) != SNHIP_OK) return false;
        } else {
            M.w = ralloc<float>(m, n);
            if (!M.w || hipMemcpy(M.w, tmp1, n * sizeof(float), hipMemcpyDeviceToDevice) != hipSuccess)
                return false;
        }
    } else if (tag == 1) {
        if (in % kRkBlobBlock) { c.ok = false; return false; }
        const size_t qb = n / 2, sb = n / kRkBlobBlock * sizeof(float);
        if ((size_t)(c.end - c.p) < qb + sb) { c.ok = false; return false; }
        uint8_t* q = ralloc<uint8_t>(m, qb);
        float* sc = ralloc<float>(m, n / kRkBlobBlock);
        if (!q || !sc) return false;
        // (scales may sit unaligned in the stream; hipMemcpy takes bytes)
        if (hipMemcpy(q, c.p, qb, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(sc, c.p + qb, sb, hipMemcpyHostToDevice) != hipSuccess)
            return false;
        c.p += qb + sb;
        if (m->wfmt != SNHIP_WEIGHTS_F32) {
            M.q = q; M.sc = sc; M.block = kRkBlobBlock;
        } else {
            M.w = ralloc<float>(m, n);
            if (!M.w || launch_dequant_i4(q, sc, M.w, out, in, kRkBlobBlock, nullptr) != SNHIP_OK)
                return false;
        }
    } else {
        c.ok = false;
        return false;
    }
    return hipDeviceSynchronize() == hipSuccess;
}

RkPMat pmat(const RMat& M) { return RkPMat{M.w, M.q, M.sc, M.M, M.Kd, M.q ? M.block : 0}; }

// The one-launch step for one sequence (or one per grid slice), when the
// device and the shape allow it: its layer table, exchange slabs and key
// words. Two kernels share them:
// * k_rk_exact (rkexact.hip), the default (SNHIP_RK_EXACT=0 turns it off):
//   every rounding in the reference's order, so its logits equal
//   sn_rk_step's bit for bit; its layer table points at fp32 (output, input)
//   copies of the layer matrices (INT4 rows dequantized to the values the
//   reference multiplies: 361 MB at 12 x 768, F = 3072), since a sequential
//   chain per output runs fastest on four-value fp32 reads;
// * k_rk_persist (rkpersist.hip), opt-in (SNHIP_RK_PERSIST=1): products and
//   LayerNorms summed in parallel, which RWKV-7 amplifies: on the 12-layer
//   INT4 model its logits were up to 1.26e-4 from sn_rk_step over 256 first
//   steps from the zero state (32 of them past 2e-5) and up to 2.7e-5 over a
//   512-token prompt and 128 greedy steps.
// The grid is at most one workgroup per CU (SNHIP_RK_PERSIST_WG caps it; it
// is rounded down to a multiple of 8), and at most the rows of the first
// product (r, k, v and the LoRA middles) and of the channel-mix key, so that
// every workgroup that takes rows of them has some: the kernels rely on that
// to know when every workgroup has read the shift vectors they then
// overwrite (k_rk_exact also checks its own row split: rke_grid_ok).
void setup_rk_persist(SnHipRwkv7* m) {
    const bool fast = env_unsigned("SNHIP_RK_PERSIST", 0, 0) != 0;
    const bool exact = !fast && env_unsigned("SNHIP_RK_EXACT", 1, 0) != 0;
    if (!fast && !exact) return;
    m->p_spin = env_unsigned("SNHIP_PERSIST_SPIN", m->p_spin, 1);
    std::vector<int> rk(4 * (size_t)m->L);
    for (int l = 0; l < m->L; ++l) {
        const RkLayer& A = m->layers[l];
        rk[4 * l] = A.Rw; rk[4 * l + 1] = A.Ra; rk[4 * l + 2] = A.Rv; rk[4 * l + 3] = A.Rg;
    }
    const auto* rk4 = reinterpret_cast<const int(*)[4]>(rk.data());
    if (!(exact ? rke_shape_ok(m->D, m->F, m->HS, m->NH, rk4, m->L)
                : rkp_shape_ok(m->D, m->F, m->HS, m->NH, rk4, m->L)))
        return;
    int G = exact ? rke_grid(m->NH) : rkp_grid(m->NH);
    if (const char* e = getenv("SNHIP_RK_PERSIST_WG")) G = std::min(G, atoi(e));
    int p1rows = 1 << 30, p1max = 0;   // the first product's rows: fewest and most over the layers
    for (int l = 0; l < m->L; ++l) {
        const int n = 3 * m->D + rk[4 * l] + rk[4 * l + 1] + rk[4 * l + 3];
        p1rows = std::min(p1rows, n);
        p1max = std::max(p1max, n + (l > 0 ? rk[4 * l + 2] : 0));
    }
    G = std::min(G, std::min(p1rows, m->F)) / 8 * 8;
    if (G < 8 || G < m->NH || (exact && !rke_grid_ok(G, m->D, m->F, p1max))) return;
    // exact: each layer matrix as fp32 (output, input) rows
    auto rows_f32 = [&](const RMat& M, bool& ok) -> RkPMat {
        if (!M.q) return RkPMat{M.w, nullptr, nullptr, M.M, M.Kd, 0};
        float* w = ralloc<float>(m, (size_t)M.M * M.Kd);
        if (!w || launch_dequant_i4(M.q, M.sc, w, M.M, M.Kd, M.block, nullptr) != SNHIP_OK) ok = false;
        return RkPMat{w, nullptr, nullptr, M.M, M.Kd, 0};
    };
    bool ok = true;
    auto mat = [&](const RMat& M) -> RkPMat { return exact ? rows_f32(M, ok) : pmat(M); };
    std::vector<RkPLayer> tab(m->L);
    for (int l = 0; l < m->L; ++l) {
        const RkLayer& A = m->layers[l];
        RkPLayer& P = tab[l];
        P.r = mat(A.r); P.k = mat(A.k); P.v = mat(A.v); P.w1 = mat(A.w1); P.a1 = mat(A.a1);
        P.g1 = mat(A.g1); P.v1 = l > 0 ? mat(A.v1) : pmat(A.v1); P.w2 = mat(A.w2); P.a2 = mat(A.a2);
        P.g2 = mat(A.g2); P.v2 = l > 0 ? mat(A.v2) : pmat(A.v2); P.o = mat(A.o); P.cmk = mat(A.cmk);
        P.cmv = mat(A.cmv);
        P.ln1w = A.ln1w; P.ln1b = A.ln1b; P.ln2w = A.ln2w; P.ln2b = A.ln2b; P.lerp = A.lerp; P.w0 = A.w0;
        P.a0 = A.a0; P.v0 = A.v0; P.kk = A.kk; P.ka = A.ka; P.rk = A.rk; P.lnxw = A.lnxw; P.lnxb = A.lnxb;
        P.cmk_lerp = A.cmk_lerp;
    }
    if (!ok) return;
    // Slices for B = 2..p_mi_max (SNHIP_RK_PERSIST_MI=n, default 8): the
    // largest multiple of 8 workgroups, at least the head count, that B
    // slices fit in the one-sequence grid. Each sequence's results equal its
    // one-sequence launch's bit for bit (neither kernel's arithmetic depends
    // on the grid size).
    m->p_mi_max = 0;
    const int lim = std::min(std::min(m->max_batch, kRkPMiMax),
                             (int)std::min(env_unsigned("SNHIP_RK_PERSIST_MI", 8, 0), (unsigned)kRkPMiMax));
    for (int b = 2; b <= lim; ++b) {
        const int g = G / b / 8 * 8;
        if (g < 8 || g < m->NH || (exact && !rke_grid_ok(g, m->D, m->F, p1max))) break;
        m->p_mi_grid[b] = g;
        m->p_mi_max = b;
    }
    RkPLayer* dtab = ralloc<RkPLayer>(m, tab.size());
    m->p_seq_words = (size_t)m->L * rkp_slab(m->D, m->F) + 2 * (size_t)G;
    m->p_nwords = m->p_seq_words * std::max(1, m->p_mi_max);
    m->p_words = ralloc<unsigned long long>(m, m->p_nwords);
    m->p_err = ralloc<unsigned>(m, 1);
    if (!dtab || !m->p_words || !m->p_err ||
        hipMemcpy(dtab, tab.data(), tab.size() * sizeof(RkPLayer), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(m->p_words, 0, m->p_nwords * sizeof(unsigned long long)) != hipSuccess)
        return;
    unsigned long long* xch = m->p_words;
    unsigned long long* keys = xch + (size_t)m->L * rkp_slab(m->D, m->F);
    RkPArgs& a = m->p_args;
    a.layers = dtab; a.L = m->L; a.D = m->D; a.F = m->F; a.NH = m->NH; a.vocab = m->vocab; a.eps = m->eps;
    a.embed = m->embed; a.en_w = m->en_w; a.en_b = m->en_b; a.on_w = m->on_w; a.on_b = m->on_b;
    a.head = pmat(m->head);
    a.S = m->S; a.shift = m->shift; a.vfirst = m->vfirst; a.xch = xch; a.keys = keys;
    a.tok = m->tok; a.counter = m->counter;
    a.err = m->p_err; a.spin_limit = m->p_spin; a.stall = 0;
    a.words = m->p_seq_words;
    m->p_grid = G;
    m->p_exact = exact;
}

// The tiled fp32 form of every layer matrix (rkseq.h: block -1), for the
// per-kernel steps: their products then run one independent wave per 64
// rows and 4-16 sequences, streaming 1 KiB weight blocks, with no producer
// waves and no barrier per 64 inputs. Made when some batch size up to
// max_batch steps per kernel (SNHIP_RKQ_W4=0: never); each is 4 bytes per
// weight (plus 64 KiB of padding). The vocabulary head keeps its own format.
void setup_rkq_w4(SnHipRwkv7* m) {
    if (env_unsigned("SNHIP_RKQ_W4", 1, 0) == 0) return;
    const int one_launch = m->p_grid > 0 ? std::max(1, m->p_mi_max) : 0;
    if (m->max_batch <= one_launch) return;
    bool ok = true;
    auto make = [&](RMat& M) {
        if (!ok || M.M <= 0 || M.Kd <= 0 || M.Kd % 4 || (!M.q && !M.w) ||
            rkq_tiled_floats(M.M, M.Kd) * sizeof(float) >= ((size_t)1 << 31))   // the kernel's 32-bit offsets
            return;
        float* w4 = ralloc<float>(m, rkq_tiled_floats(M.M, M.Kd));
        if (!w4 || launch_rkq_block4(M.w, M.q, M.sc, M.q ? M.block : 0, M.M, M.Kd, w4, nullptr) != SNHIP_OK) {
            ok = false;
            return;
        }
        M.w4 = w4;
    };
    for (int l = 0; l < m->L; ++l) {
        RkLayer& A = m->layers[l];
        for (RMat* M : {&A.r, &A.k, &A.v, &A.o, &A.w1, &A.w2, &A.a1, &A.a2, &A.v1, &A.v2, &A.g1, &A.g2,
                        &A.cmk, &A.cmv})
            make(*M);
    }
    if (hipDeviceSynchronize() != hipSuccess) ok = false;
    if (!ok) {
        // all or nothing: the products then keep the stored format
        for (int l = 0; l < m->L; ++l) {
            RkLayer& A = m->layers[l];
            for (RMat* M : {&A.r, &A.k, &A.v, &A.o, &A.w1, &A.w2, &A.a1, &A.a2, &A.v1, &A.v2, &A.g1, &A.g2,
                            &A.cmk, &A.cmv})
                M->w4 = nullptr;
        }
    }
}

// Do steps of B sequences run as B slices of the persistent kernel?
bool uses_mi(const SnHipRwkv7* m, int B) { return m->p_grid > 0 && B >= 2 && B <= m->p_mi_max; }

// reps persistent steps of sequences [0, B) (B = 1, or 2..p_mi_max on a grid
// slice each): greedy, one launch of up to kRkPStepsPerLaunch steps at a
// time, otherwise one launch per step; every step has its own epoch. The
// call waits for them and reports a time-out of an exchange wait as an error.
// The kernel updates S and shift in place layer by layer, so a time-out
// leaves them part-stepped: the handle is then refused for stepping until its
// state is reset or set.
constexpr int kRkPStepsPerLaunch = 1024;
snhip_status run_persist(SnHipRwkv7* m, int B, float* logits_out, bool greedy, int reps) {
    RkPArgs a = m->p_args;
    a.stall = env_unsigned("SNHIP_PERSIST_STALL", 0, 0);
    a.logits = logits_out;
    a.greedy = greedy ? 1 : 0;
    a.tok_hist = m->tok_hist;
    a.hist_cap = m->hist_cap;
    a.ni = B;
    const int grid = B == 1 ? m->p_grid : B * m->p_mi_grid[B];
    SNHIP_CHECK(hipMemsetAsync(m->p_err, 0, sizeof(unsigned), m->work));
    for (int i = 0; i < reps;) {
        const int n = greedy ? std::min(reps - i, kRkPStepsPerLaunch) : 1;
        if (m->p_epoch > 0xFFFFFFFFu - (unsigned)n) {
            // epochs start over from clean words
            SNHIP_CHECK(hipMemsetAsync(m->p_words, 0, m->p_nwords * sizeof(unsigned long long), m->work));
            m->p_epoch = 0;
        }
        a.epoch = m->p_epoch + 1;
        a.nsteps = n;
        a.hist0 = i;
        m->p_epoch += (unsigned)n;
        const snhip_status rc = m->p_exact ? launch_rk_exact(a, grid, m->work) : launch_rk_persist(a, grid, m->work);
        if (rc != SNHIP_OK) return rc;
        i += n;
    }
    unsigned err = 0;
    SNHIP_CHECK(hipMemcpyAsync(&err, m->p_err, sizeof(unsigned), hipMemcpyDeviceToHost, m->work));
    SNHIP_CHECK(hipStreamSynchronize(m->work));
    if (err) {
        m->poisoned = 1;
        set_last_error("RWKV-7 persistent step: an exchange wait timed out");
        return SNHIP_E_DEVICE;
    }
    return SNHIP_OK;
}

snhip_status check_usable(const SnHipRwkv7* m) {
    if (m->poisoned) {
        set_last_error("the sequence state was left part-stepped by a timed-out step; "
                       "call snhip_rk_reset or snhip_rk_set_state_dev first");
        return SNHIP_E_DEVICE;
    }
    return SNHIP_OK;
}

SnHipRwkv7* load_rk(const char* path, int max_batch, int wfmt, int block) {
    if (!path || max_batch <= 0 || max_batch > 1024) { set_last_error("invalid arguments"); return nullptr; }
    if (wfmt != SNHIP_WEIGHTS_F32 && wfmt != SNHIP_WEIGHTS_INT4 && wfmt != SNHIP_WEIGHTS_STORED) {
        set_last_error("unknown weight format");
        return nullptr;
    }
    if (wfmt == SNHIP_WEIGHTS_INT4 && block != 32 && block != 64) { set_last_error("INT4 block must be 32 or 64"); return nullptr; }
    FILE* f = fopen(path, "rb");
    if (!f) { set_last_error(std::string("cannot open ") + path); return nullptr; }
    std::vector<uint8_t> buf;
    {
        fseek(f, 0, SEEK_END);
        const long sz = ftell(f);
        fseek(f, 0, SEEK_SET);
        if (sz < 44) { fclose(f); set_last_error("blob too short"); return nullptr; }
        buf.resize((size_t)sz);
        const size_t got = fread(buf.data(), 1, buf.size(), f);
        fclose(f);
        if (got != buf.size()) { set_last_error("blob read failed"); return nullptr; }
    }
    int32_t h[10];
    memcpy(h, buf.data(), sizeof h);
    if (h[0] != kRkMagic || h[1] != kRkVersion) { set_last_error("bad RWKV-7 blob header (magic/version)"); return nullptr; }
    const int L = h[2], D = h[3], HS = h[4], NH = h[5], F = h[6], V = h[8];
    if (L <= 0 || D <= 0 || HS != kHS || NH * HS != D || F <= 0 || V <= 0 || D > kMaxDim ||
        D % 32 || F % 4) {
        set_last_error("unsupported RWKV-7 shape (head size must be 64, dim <= 4096)");
        return nullptr;
    }
    const uint8_t* p = buf.data() + 40;
    float eps;
    memcpy(&eps, p, 4);
    p += 4;
    if ((size_t)(buf.data() + buf.size() - p) < (size_t)16 * L) { set_last_error("blob is truncated"); return nullptr; }
    std::vector<int32_t> ranks(4 * (size_t)L);
    memcpy(ranks.data(), p, ranks.size() * sizeof(int32_t));
    p += ranks.size() * sizeof(int32_t);

    SnHipRwkv7* m = new SnHipRwkv7();
    m->L = L; m->D = D; m->HS = HS; m->NH = NH; m->F = F; m->vocab = V; m->eps = eps;
    m->max_batch = max_batch; m->wfmt = wfmt; m->block = block;
    const size_t big = std::max((size_t)D * V, std::max((size_t)D * F, (size_t)D * D));
    float* tmp0 = ralloc<float>(m, big);
    float* tmp1 = ralloc<float>(m, big);
    if (!tmp0 || !tmp1) { free_rk(m); set_last_error("out of device memory"); return nullptr; }
    Cur c{p, buf.data() + buf.size(), true};
    bool ok = true;
    m->layers.resize(L);
    for (int l = 0; l < L && ok && c.ok; ++l) {
        RkLayer& A = m->layers[l];
        A.Rw = ranks[4 * l]; A.Ra = ranks[4 * l + 1]; A.Rv = ranks[4 * l + 2]; A.Rg = ranks[4 * l + 3];
        if (A.Rw <= 0 || A.Ra <= 0 || A.Rv <= 0 || A.Rg <= 0 || A.Rw > kMaxRank || A.Ra > kMaxRank ||
            A.Rv > kMaxRank || A.Rg > kMaxRank || A.Rw % 4 || A.Ra % 4 || A.Rv % 4 || A.Rg % 4) {
            c.ok = false;
            break;
        }
        const float* t;
        ok = ok && (t = take_vec(c, D)) && upload(m, A.ln1w, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.ln1b, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.ln2w, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.ln2b, t, D);
        ok = ok && (t = take_vec(c, (size_t)6 * D)) && upload(m, A.lerp, t, (size_t)6 * D);
        ok = ok && take_mat(m, c, A.r, D, D, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.k, D, D, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.v, D, D, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.o, D, D, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.w1, D, A.Rw, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.w2, A.Rw, D, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.a1, D, A.Ra, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.a2, A.Ra, D, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.v1, D, A.Rv, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.v2, A.Rv, D, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.g1, D, A.Rg, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.g2, A.Rg, D, tmp0, tmp1);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.w0, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.a0, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.v0, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.kk, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.ka, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.rk, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.lnxw, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.lnxb, t, D);
        ok = ok && take_mat(m, c, A.cmk, D, F, tmp0, tmp1);
        ok = ok && take_mat(m, c, A.cmv, F, D, tmp0, tmp1);
        ok = ok && (t = take_vec(c, D)) && upload(m, A.cmk_lerp, t, D);
    }
    if (ok && c.ok) {
        const float* t;
        ok = ok && (t = take_vec(c, D)) && upload(m, m->en_w, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, m->en_b, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, m->on_w, t, D);
        ok = ok && (t = take_vec(c, D)) && upload(m, m->on_b, t, D);
        ok = ok && (t = take_vec(c, (size_t)V * D)) && upload(m, m->embed, t, (size_t)V * D);
        ok = ok && take_mat(m, c, m->head, D, V, tmp0, tmp1);
    }
    if (!ok || !c.ok) {
        if (last_error().empty() || !c.ok) set_last_error("RWKV-7 blob is malformed or truncated");
        free_rk(m);
        return nullptr;
    }
    for (auto it = m->allocs.begin(); it != m->allocs.end();) {
        if (*it == tmp0 || *it == tmp1) { (void)hipFree(*it); it = m->allocs.erase(it); }
        else ++it;
    }
    const size_t B = max_batch;
    m->S = ralloc<float>(m, B * L * NH * HS * HS);
    m->shift = ralloc<float>(m, B * L * 2 * D);
    m->x = ralloc<float>(m, B * D);
    m->X6 = ralloc<float>(m, B * 6 * D);
    m->r = ralloc<float>(m, B * D);
    m->k = ralloc<float>(m, B * D);
    m->v = ralloc<float>(m, B * D);
    m->lo = ralloc<float>(m, B * 4 * kMaxRank);
    m->dw = ralloc<float>(m, B * D);
    m->da = ralloc<float>(m, B * D);
    m->dv = ralloc<float>(m, B * D);
    m->g = ralloc<float>(m, B * D);
    m->y = ralloc<float>(m, B * D);
    m->vfirst = ralloc<float>(m, B * D);
    m->xk2 = ralloc<float>(m, B * D);
    m->ck = ralloc<float>(m, B * F);
    m->nrm = ralloc<float>(m, B * D);
    m->logits = ralloc<float>(m, B * V);
    m->tok = ralloc<int32_t>(m, B);
    m->best = ralloc<unsigned long long>(m, B * 4096);
    m->counter = ralloc<int32_t>(m, 1);
    m->done = ralloc<int32_t>(m, 1);
    if (!m->S || !m->shift || !m->x || !m->X6 || !m->r || !m->k || !m->v || !m->lo || !m->dw ||
        !m->da || !m->dv || !m->g || !m->y || !m->vfirst || !m->xk2 || !m->ck || !m->nrm ||
        !m->logits || !m->tok || !m->best || !m->counter || !m->done ||
        hipMemset(m->S, 0, B * L * NH * HS * HS * sizeof(float)) != hipSuccess ||
        hipMemset(m->shift, 0, B * L * 2 * D * sizeof(float)) != hipSuccess ||
        hipMemset(m->counter, 0, sizeof(int32_t)) != hipSuccess ||
        hipMemset(m->done, 0, sizeof(int32_t)) != hipSuccess ||
        hipStreamCreateWithFlags(&m->work, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_in, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&m->ev_out, hipEventDisableTiming) != hipSuccess) {
        set_last_error("device setup failed");
        free_rk(m);
        return nullptr;
    }
    if (const char* e = getenv("SNHIP_NO_GRAPH")) m->use_graphs = !(e[0] == '1');
    m->fuse_ups = env_unsigned("SNHIP_RKQ_FUSE_UPS", 1, 0) != 0;
    setup_rk_persist(m);
    setup_rkq_w4(m);
    m->ready = 1;
    return m;
}

// Matrix products of one dependency level, grouped by weight format into
// launches of up to kRkqMaxJobs jobs.
struct MMList {
    int B;
    RkqJob jobs[kRkqMaxJobs];
    int blk[kRkqMaxJobs];
    int n = 0;

    snhip_status add(const RMat& W, const float* X, int ldx, float* Y, int ldy, int epi) {
        if (n == kRkqMaxJobs) return SNHIP_E_INVAL;
        RkqJob j{};
        j.X = X; j.ldx = ldx;
        j.w = W.w4 ? W.w4 : W.w; j.q = W.w4 ? nullptr : W.q; j.sc = W.w4 ? nullptr : W.sc;
        j.M = W.M; j.Kd = W.Kd;
        j.Y = Y; j.ldy = ldy;
        j.epi = epi;
        jobs[n] = j;
        blk[n] = W.w4 ? -1 : W.q ? W.block : 0;
        ++n;
        return SNHIP_OK;
    }

    snhip_status flush(hipStream_t st) {
        bool used[kRkqMaxJobs] = {false};
        for (int i = 0; i < n; ++i) {
            if (used[i]) continue;
            RkqJob batch[kRkqMaxJobs];
            int nb = 0;
            for (int j = i; j < n; ++j)
                if (!used[j] && blk[j] == blk[i]) { batch[nb++] = jobs[j]; used[j] = true; }
            const snhip_status rc = launch_rkq_mm(batch, nb, B, blk[i], st);
            if (rc != SNHIP_OK) return rc;
        }
        n = 0;
        return SNHIP_OK;
    }
};

// dbg (device, 9 D floats): run layers 0..dbg_layer only and leave sequence
// 0's intermediates of that layer there in the reference's order (rwkv7.c:308-319).
snhip_status enqueue_step(SnHipRwkv7* m, int B, float* logits_out, bool greedy, hipStream_t st,
                          int dbg_layer = -1, float* dbg = nullptr) {
    const int D = m->D, F = m->F, NH = m->NH, L = m->L, HS = m->HS;
    const size_t s_bstride = (size_t)L * NH * HS * HS, sh_bstride = (size_t)L * 2 * D;
    const int ldl = 4 * kMaxRank;
    float* lw = m->lo;
    float* la = m->lo + kMaxRank;
    float* lv = m->lo + 2 * kMaxRank;
    float* lg = m->lo + 3 * kMaxRank;
    snhip_status rc;
    RkqLnArgs ln{};
    ln.D = D; ln.vocab = m->vocab; ln.eps = m->eps; ln.shift_bstride = sh_bstride;
    ln.mode = RKQ_LN_EMBED;
    ln.tok = m->tok; ln.embed = m->embed; ln.g = m->en_w; ln.c = m->en_b; ln.out = m->x;
    if ((rc = launch_rkq_ln(ln, B, st)) != SNHIP_OK) return rc;
    MMList mm{B};
    const int nl = dbg ? dbg_layer + 1 : L;
    for (int l = 0; l < nl; ++l) {
        const RkLayer& A = m->layers[l];
        float* dl = dbg && l == dbg_layer ? dbg : nullptr;
        float* sh = m->shift + (size_t)l * 2 * D;
        ln.mode = RKQ_LN_MIX1;
        ln.x = m->x; ln.g = A.ln1w; ln.c = A.ln1b; ln.lerp = A.lerp; ln.shift = sh; ln.out = m->X6;
        if ((rc = launch_rkq_ln(ln, B, st)) != SNHIP_OK) return rc;
        const float* xr = m->X6;
        const float* xw = m->X6 + D;
        const float* xk = m->X6 + 2 * D;
        const float* xv = m->X6 + 3 * D;
        const float* xa = m->X6 + 4 * D;
        const float* xg = m->X6 + 5 * D;
        const int ld6 = 6 * D;
        if ((rc = mm.add(A.r, xr, ld6, m->r, D, RKQ_STORE)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.k, xk, ld6, m->k, D, RKQ_STORE)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.v, xv, ld6, m->v, D, RKQ_STORE)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.w1, xw, ld6, lw, ldl, RKQ_TANH)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.a1, xa, ld6, la, ldl, RKQ_STORE)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.g1, xg, ld6, lg, ldl, RKQ_SIGMOID)) != SNHIP_OK) return rc;
        if (l > 0 && (rc = mm.add(A.v1, xv, ld6, lv, ldl, RKQ_STORE)) != SNHIP_OK) return rc;
        if ((rc = mm.flush(st)) != SNHIP_OK) return rc;
        // The LoRA up-projections run inside the heads kernel when they are
        // INT4 of one group size with ranks up to 128 (SNHIP_RKQ_FUSE_UPS=0:
        // never): it computes each channel's four short chains from the
        // codes, and the step saves a launch per layer.
        const bool fuse = m->fuse_ups && A.w2.q && A.a2.q && A.g2.q && (l == 0 || A.v2.q) &&
                          (A.w2.block == 32 || A.w2.block == 64) && A.a2.block == A.w2.block &&
                          A.g2.block == A.w2.block && (l == 0 || A.v2.block == A.w2.block) &&
                          A.w2.Kd <= 128 && A.a2.Kd <= 128 && A.g2.Kd <= 128 && (l == 0 || A.v2.Kd <= 128) &&
                          A.w2.Kd % A.w2.block == 0 && A.a2.Kd % A.w2.block == 0 &&
                          A.g2.Kd % A.w2.block == 0 && (l == 0 || A.v2.Kd % A.w2.block == 0) &&
                          A.w2.M == D && A.a2.M == D && A.g2.M == D && (l == 0 || A.v2.M == D);
        if (!fuse) {
            if ((rc = mm.add(A.w2, lw, ldl, m->dw, D, RKQ_STORE)) != SNHIP_OK) return rc;
            if ((rc = mm.add(A.a2, la, ldl, m->da, D, RKQ_STORE)) != SNHIP_OK) return rc;
            if ((rc = mm.add(A.g2, lg, ldl, m->g, D, RKQ_STORE)) != SNHIP_OK) return rc;
            if (l > 0 && (rc = mm.add(A.v2, lv, ldl, m->dv, D, RKQ_STORE)) != SNHIP_OK) return rc;
            if ((rc = mm.flush(st)) != SNHIP_OK) return rc;
        }
        RkqHeadArgs H{};
        if (fuse) {
            const RMat* up[4] = {&A.w2, &A.a2, &A.g2, l > 0 ? &A.v2 : &A.w2};
            const float* ux[4] = {lw, la, lg, l > 0 ? lv : lw};
            const int uk[4] = {A.w2.Kd, A.a2.Kd, A.g2.Kd, l > 0 ? A.v2.Kd : 0};
            for (int i = 0; i < 4; ++i) {
                H.up_q[i] = up[i]->q;
                H.up_sc[i] = up[i]->sc;
                H.up_x[i] = ux[i];
                H.up_k[i] = uk[i];
            }
            H.up_blk = A.w2.block;
            H.up_ldx = ldl;
            H.g_out = m->g;
        }
        H.r = m->r; H.k = m->k; H.v = m->v; H.dw = m->dw; H.da = m->da; H.dv = m->dv; H.g = m->g;
        H.vfirst = m->vfirst;
        H.w0 = A.w0; H.a0 = A.a0; H.v0 = A.v0; H.kk_w = A.kk; H.ka_w = A.ka; H.rk_w = A.rk;
        H.lnx_w = A.lnxw; H.lnx_b = A.lnxb;
        H.S = m->S + (size_t)l * NH * HS * HS;
        H.s_bstride = s_bstride;
        H.y = m->y;
        H.D = D; H.NH = NH;
        H.first = l == 0;
        H.dbg = dl;
        if ((rc = launch_rkq_heads(H, B, st)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.o, m->y, D, m->x, D, RKQ_ADD)) != SNHIP_OK) return rc;
        if ((rc = mm.flush(st)) != SNHIP_OK) return rc;
        ln.mode = RKQ_LN_MIX2;
        ln.x = m->x; ln.g = A.ln2w; ln.c = A.ln2b; ln.lerp = A.cmk_lerp; ln.shift = sh + D; ln.out = m->xk2;
        if ((rc = launch_rkq_ln(ln, B, st)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.cmk, m->xk2, D, m->ck, F, RKQ_RELU2)) != SNHIP_OK) return rc;
        if ((rc = mm.flush(st)) != SNHIP_OK) return rc;
        if ((rc = mm.add(A.cmv, m->ck, F, m->x, D, RKQ_ADD)) != SNHIP_OK) return rc;
        if ((rc = mm.flush(st)) != SNHIP_OK) return rc;
        if (dl) {
            // xn (the LayerNorm output, kept as shift_0), r, g, y and the layer's x
            const size_t n = (size_t)D * sizeof(float);
            SNHIP_CHECK(hipMemcpyAsync(dl, sh, n, hipMemcpyDeviceToDevice, st));
            SNHIP_CHECK(hipMemcpyAsync(dl + D, m->r, n, hipMemcpyDeviceToDevice, st));
            SNHIP_CHECK(hipMemcpyAsync(dl + 5 * D, m->g, n, hipMemcpyDeviceToDevice, st));
            SNHIP_CHECK(hipMemcpyAsync(dl + 7 * D, m->y, n, hipMemcpyDeviceToDevice, st));
            SNHIP_CHECK(hipMemcpyAsync(dl + 8 * D, m->x, n, hipMemcpyDeviceToDevice, st));
            return SNHIP_OK;
        }
    }
    ln.mode = RKQ_LN_PLAIN;
    ln.x = m->x; ln.g = m->on_w; ln.c = m->on_b; ln.out = m->nrm;
    if ((rc = launch_rkq_ln(ln, B, st)) != SNHIP_OK) return rc;
    if ((rc = mm.add(m->head, m->nrm, D, logits_out, m->vocab, RKQ_STORE)) != SNHIP_OK) return rc;
    if ((rc = mm.flush(st)) != SNHIP_OK) return rc;
    if (greedy) {
        const int nblk = 64;
        hipLaunchKernelGGL(k_rk_argmax_partial, dim3(nblk, B), dim3(256), 0, st, logits_out,
                           m->vocab, m->best);
        hipLaunchKernelGGL(k_rk_finalize, dim3(B), dim3(256), 0, st, m->best, nblk, B, m->tok,
                           m->tok_hist, m->counter, m->done, m->hist_cap);
    }
    SNHIP_CHECK(hipGetLastError());
    return SNHIP_OK;
}

// reps steps on the internal stream, ordered after the caller's stream;
// captured once per (B, logits, greedy) into a graph and replayed.
snhip_status run_steps(SnHipRwkv7* m, int B, float* logits_out, bool greedy, int reps) {
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    SNHIP_CHECK(hipEventRecord(m->ev_in, m->stream));
    SNHIP_CHECK(hipStreamWaitEvent(m->work, m->ev_in, 0));
    if ((B == 1 && m->p_grid > 0) || uses_mi(m, B)) {
        const snhip_status rc = run_persist(m, B, logits_out, greedy, reps);
        if (rc != SNHIP_OK) return rc;
    } else if (!m->use_graphs) {
        for (int i = 0; i < reps; ++i) {
            const snhip_status rc = enqueue_step(m, B, logits_out, greedy, m->work);
            if (rc != SNHIP_OK) return rc;
        }
    } else {
        const auto key = std::make_tuple(B, (const void*)logits_out, greedy ? 1 : 0);
        auto it = m->graphs.find(key);
        if (it == m->graphs.end()) {
            if (m->graphs.size() >= 16) {
                for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
                m->graphs.clear();
            }
            hipGraph_t g = nullptr;
            SNHIP_CHECK(hipStreamBeginCapture(m->work, hipStreamCaptureModeThreadLocal));
            const snhip_status rc = enqueue_step(m, B, logits_out, greedy, m->work);
            const hipError_t ec = hipStreamEndCapture(m->work, &g);
            if (rc != SNHIP_OK) { if (g) (void)hipGraphDestroy(g); return rc; }
            SNHIP_CHECK(ec);
            hipGraphExec_t ex = nullptr;
            const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            SNHIP_CHECK(ei);
            it = m->graphs.emplace(key, ex).first;
        }
        for (int i = 0; i < reps; ++i) SNHIP_CHECK(hipGraphLaunch(it->second, m->work));
    }
    SNHIP_CHECK(hipEventRecord(m->ev_out, m->work));
    SNHIP_CHECK(hipStreamWaitEvent(m->stream, m->ev_out, 0));
    return SNHIP_OK;
}

bool tokens_ok(const SnHipRwkv7* m, const int32_t* t, int n) {
    for (int i = 0; i < n; ++i)
        if (t[i] < 0 || t[i] >= m->vocab) return false;
    return true;
}

snhip_status step_host(SnHipRwkv7* m, const int32_t* tokens, int B, float* logits) {
    if (!m || !tokens || !logits || B <= 0 || B > m->max_batch) return SNHIP_E_INVAL;
    if (!tokens_ok(m, tokens, B)) return SNHIP_E_INVAL;
    SNHIP_CHECK(hipMemcpyAsync(m->tok, tokens, B * sizeof(int32_t), hipMemcpyHostToDevice, m->stream));
    const snhip_status rc = run_steps(m, B, m->logits, false, 1);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipMemcpyAsync(logits, m->logits, (size_t)B * m->vocab * sizeof(float),
                               hipMemcpyDeviceToHost, m->stream));
    SNHIP_CHECK(hipStreamSynchronize(m->stream));
    return SNHIP_OK;
}

snhip_status prefill_host(SnHipRwkv7* m, const int32_t* tokens, int n, float* logits) {
    if (!m || !tokens || n <= 0 || !logits) return SNHIP_E_INVAL;
    if (!tokens_ok(m, tokens, n)) return SNHIP_E_INVAL;
    // rwkv7.c:362-364: the step, once per token, in order.
    for (int i = 0; i < n; ++i) {
        SNHIP_CHECK(hipMemcpyAsync(m->tok, tokens + i, sizeof(int32_t), hipMemcpyHostToDevice, m->stream));
        const snhip_status rc = run_steps(m, 1, m->logits, false, 1);
        if (rc != SNHIP_OK) return rc;
    }
    SNHIP_CHECK(hipMemcpyAsync(logits, m->logits, (size_t)m->vocab * sizeof(float),
                               hipMemcpyDeviceToHost, m->stream));
    SNHIP_CHECK(hipStreamSynchronize(m->stream));
    return SNHIP_OK;
}

}  // namespace
}  // namespace snhip

using namespace snhip;

extern "C" {

SnHipRwkv7* snhip_rk_load(const char* path) {
    return load_rk(path, 1, SNHIP_WEIGHTS_STORED, kRkBlobBlock);
}

SnHipRwkv7* snhip_rk_load_ex(const char* path, int32_t max_batch, int32_t weight_format,
                             int32_t block) {
    return load_rk(path, max_batch, weight_format, block);
}

void snhip_rk_free(SnHipRwkv7* m) {
    if (!m) return;
    // Only this handle's work is waited for (see snhip_free).
    if (m->work) (void)hipStreamSynchronize(m->work);
    (void)hipStreamSynchronize(m->stream);
    free_rk(m);
}

void snhip_rk_reset(SnHipRwkv7* m) {
    if (!m) return;
    const size_t B = m->max_batch;
    (void)hipMemsetAsync(m->S, 0, B * m->L * m->NH * m->HS * m->HS * sizeof(float), m->stream);
    (void)hipMemsetAsync(m->shift, 0, B * m->L * 2 * m->D * sizeof(float), m->stream);
    (void)hipStreamSynchronize(m->stream);
    m->poisoned = 0;
}

void snhip_rk_step(SnHipRwkv7* m, int token, float* logits) {
    const int32_t t = token;
    (void)step_host(m, &t, 1, logits);
}

void snhip_rk_prefill(SnHipRwkv7* m, const int* tokens, int n, float* logits) {
    (void)prefill_host(m, tokens, n, logits);
}

snhip_status snhip_rk_dbg(SnHipRwkv7* m, int token, int layer, float* out) {
    if (!m || !out || layer < 0 || layer >= m->L || token < 0 || token >= m->vocab) return SNHIP_E_INVAL;
    if (check_usable(m) != SNHIP_OK) return SNHIP_E_DEVICE;
    const size_t n = (size_t)9 * m->D;
    float* d = ralloc<float>(m, n);
    if (!d) return SNHIP_E_NOMEM;
    const int32_t t = token;
    snhip_status rc = SNHIP_OK;
    if (hipMemcpyAsync(m->tok, &t, sizeof(int32_t), hipMemcpyHostToDevice, m->stream) != hipSuccess ||
        hipEventRecord(m->ev_in, m->stream) != hipSuccess || hipStreamWaitEvent(m->work, m->ev_in, 0) != hipSuccess)
        rc = SNHIP_E_DEVICE;
    if (rc == SNHIP_OK) rc = enqueue_step(m, 1, m->logits, false, m->work, layer, d);
    if (rc == SNHIP_OK && (hipMemcpyAsync(out, d, n * sizeof(float), hipMemcpyDeviceToHost, m->work) != hipSuccess ||
                           hipStreamSynchronize(m->work) != hipSuccess))
        rc = SNHIP_E_DEVICE;
    (void)hipStreamSynchronize(m->work);
    for (auto it = m->allocs.begin(); it != m->allocs.end(); ++it)
        if (*it == d) { (void)hipFree(d); m->allocs.erase(it); break; }
    return rc;
}

int snhip_rk_vocab(const SnHipRwkv7* m) { return m ? m->vocab : 0; }
int snhip_rk_ready(const SnHipRwkv7* m) { return m && m->ready; }

snhip_status snhip_rk_set_stream(SnHipRwkv7* m, void* stream) {
    if (!m) return SNHIP_E_INVAL;
    m->stream = as_stream(stream);
    return SNHIP_OK;
}

int32_t snhip_rk_max_batch(const SnHipRwkv7* m) { return m ? m->max_batch : 0; }

int32_t snhip_rk_persist_grid(const SnHipRwkv7* m) { return m ? m->p_grid : 0; }

int32_t snhip_rk_persist_exact(const SnHipRwkv7* m) { return m && m->p_grid > 0 && m->p_exact ? 1 : 0; }

int32_t snhip_rk_persist_grid_batch(const SnHipRwkv7* m, int32_t B) {
    if (!m || B < 1 || B > m->max_batch) return 0;
    if (B == 1) return m->p_grid;
    return uses_mi(m, B) ? B * m->p_mi_grid[B] : 0;
}

snhip_status snhip_rk_step_batch_dev(SnHipRwkv7* m, const int32_t* tokens_dev, int32_t B,
                                     float* logits_dev) {
    if (!m || !tokens_dev || !logits_dev || B <= 0 || B > m->max_batch) return SNHIP_E_INVAL;
    SNHIP_CHECK(hipMemcpyAsync(m->tok, tokens_dev, B * sizeof(int32_t), hipMemcpyDeviceToDevice, m->stream));
    return run_steps(m, B, logits_dev, false, 1);
}

snhip_status snhip_rk_decode_greedy_dev(SnHipRwkv7* m, const int32_t* tokens_dev, int32_t B,
                                        int32_t n_steps, int32_t* out_tokens_dev,
                                        float* logits_dev) {
    if (!m || !tokens_dev || !out_tokens_dev || B <= 0 || B > m->max_batch || n_steps <= 0)
        return SNHIP_E_INVAL;
    if ((long)n_steps * B > (long)m->hist_cap || !m->tok_hist) {
        // Grow the token history; graphs bake its address, so drop them.
        SNHIP_CHECK(hipStreamSynchronize(m->stream));
        SNHIP_CHECK(hipStreamSynchronize(m->work));
        for (auto& kv : m->graphs) (void)hipGraphExecDestroy(kv.second);
        m->graphs.clear();
        long cap = 256L * m->max_batch;
        while (cap < (long)n_steps * B) cap *= 2;
        if (cap > (1L << 30)) return SNHIP_E_INVAL;
        int32_t* hbuf = nullptr;
        SNHIP_CHECK(hipMalloc(&hbuf, (size_t)cap * sizeof(int32_t)));
        if (m->tok_hist) {
            (void)hipFree(m->tok_hist);
            for (auto it = m->allocs.begin(); it != m->allocs.end(); ++it)
                if (*it == m->tok_hist) { m->allocs.erase(it); break; }
        }
        m->tok_hist = hbuf;
        m->allocs.push_back(hbuf);
        m->hist_cap = (int)cap;
    }
    SNHIP_CHECK(hipMemcpyAsync(m->tok, tokens_dev, B * sizeof(int32_t), hipMemcpyDeviceToDevice, m->stream));
    SNHIP_CHECK(hipMemsetAsync(m->counter, 0, sizeof(int32_t), m->stream));
    const snhip_status rc = run_steps(m, B, logits_dev ? logits_dev : m->logits, true, n_steps);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipMemcpyAsync(out_tokens_dev, m->tok_hist, (size_t)n_steps * B * sizeof(int32_t),
                               hipMemcpyDeviceToDevice, m->stream));
    return SNHIP_OK;
}

snhip_status snhip_rk_get_state_dev(SnHipRwkv7* m, float* S_dev, float* shift_dev, int32_t B) {
    if (!m || !S_dev || !shift_dev || B <= 0 || B > m->max_batch) return SNHIP_E_INVAL;
    SNHIP_CHECK(hipMemcpyAsync(S_dev, m->S, (size_t)B * m->L * m->NH * m->HS * m->HS * sizeof(float),
                               hipMemcpyDeviceToDevice, m->stream));
    SNHIP_CHECK(hipMemcpyAsync(shift_dev, m->shift, (size_t)B * m->L * 2 * m->D * sizeof(float),
                               hipMemcpyDeviceToDevice, m->stream));
    return SNHIP_OK;
}

snhip_status snhip_rk_set_state_dev(SnHipRwkv7* m, const float* S_dev, const float* shift_dev,
                                    int32_t B) {
    if (!m || !S_dev || !shift_dev || B <= 0 || B > m->max_batch) return SNHIP_E_INVAL;
    SNHIP_CHECK(hipMemcpyAsync(m->S, S_dev, (size_t)B * m->L * m->NH * m->HS * m->HS * sizeof(float),
                               hipMemcpyDeviceToDevice, m->stream));
    SNHIP_CHECK(hipMemcpyAsync(m->shift, shift_dev, (size_t)B * m->L * 2 * m->D * sizeof(float),
                               hipMemcpyDeviceToDevice, m->stream));
    m->poisoned = 0;
    return SNHIP_OK;
}

// sn_abi.c:94-134 mirror
SnHipRwkv7* snhip_abi_rwkv7_load(const char* blob_path) {
    if (!blob_path) return nullptr;
    return snhip_rk_load(blob_path);
}

snhip_status snhip_abi_rwkv7_step(SnHipRwkv7* m, int32_t token, float* logits) {
    if (!m || !logits || token < 0) return SNHIP_E_INVAL;
    return step_host(m, &token, 1, logits);
}

snhip_status snhip_abi_rwkv7_prefill(SnHipRwkv7* m, const int32_t* tokens, int32_t n,
                                     float* logits) {
    if (!m || !tokens || !logits || n <= 0) return SNHIP_E_INVAL;
    return prefill_host(m, tokens, n, logits);
}

snhip_status snhip_abi_rwkv7_reset(SnHipRwkv7* m) {
    if (!m) return SNHIP_E_INVAL;
    snhip_rk_reset(m);
    return SNHIP_OK;
}

void snhip_abi_rwkv7_free(SnHipRwkv7* m) { snhip_rk_free(m); }

int32_t snhip_abi_rwkv7_vocab(const SnHipRwkv7* m) { return m ? m->vocab : 0; }

}  // extern "C"
