// RWKV-7 decode at one sequence as one cooperative launch per step
// (rkpersist.hip): the shared types between the handle (rwkv.hip) and the
// kernel.
#pragma once

#include "common.h"

namespace snhip {

// A weight matrix, row-major (M, K): fp32 w (block 0) or INT4 q + sc with
// group `block` (32 or 64).
struct RkPMat {
    const float* w;
    const uint8_t* q;
    const float* sc;
    int M, K, block;
};

struct RkPLayer {
    RkPMat r, k, v, w1, a1, g1, v1, w2, a2, g2, v2, o, cmk, cmv;
    const float *ln1w, *ln1b, *ln2w, *ln2b, *lerp, *w0, *a0, *v0, *kk, *ka, *rk, *lnxw, *lnxb, *cmk_lerp;
};

struct RkPArgs {
    const RkPLayer* layers;   // device array of L entries
    int L, D, F, NH, vocab;
    float eps;
    const float *embed, *en_w, *en_b, *on_w, *on_b;
    RkPMat head;
    float* S;                 // (L, NH, 64, 64)
    float* shift;             // (L, 2, D)
    float* vfirst;            // (D)
    unsigned long long* xch;  // per-layer exchange slabs, rkp_slab(D, F) words each
    float* logits;            // (vocab)
    unsigned long long* keys; // (2 grid) exchange words of the argmax keys
    int32_t* tok;             // the step's input token (and, greedy, the next one)
    int32_t* tok_hist;        // greedy: (steps, ni) tokens, from row hist0 on
    int32_t* counter;         // set to hist0 + nsteps after a greedy launch
    int hist_cap, greedy;
    int hist0;                // greedy steps of the call before this launch
    // Independent sequences, one per equal slice of the grid (0 or 1: one).
    // Sequence q runs on workgroups [q G, (q+1) G), G = grid / ni, with its
    // own state (S + q L NH 64 64, shift + q L 2 D, vfirst + q D), exchange
    // and key words (xch and keys + q words), token tok[q], token column q of
    // tok_hist and logits + q vocab.
    int ni;
    size_t words;
    unsigned epoch;           // the epoch of the launch's first step (> 0; step st uses epoch + st, and
                              // no epoch is used twice between two clearings of the words)
    int nsteps;               // steps of the launch (greedy; 1 otherwise)
    unsigned* err;
    unsigned spin_limit;
    unsigned stall;           // added to every wait target: tests force time-outs with it
};

constexpr int kRkPMaxD = 1024, kRkPMaxF = 4096, kRkPRank = 256, kRkPMaxGrid = 1024;
constexpr int kRkPMiMax = 32;   // sequences one launch steps at most (a.ni)

// Exchange words of one layer's slab (one 64-bit word per value: the epoch
// of the launch that wrote it above the value's bits): r, k, v, y, x after
// the time mix, x after the channel mix (D each), the four LoRA middles (256
// each), ck (F).
__host__ __device__ inline size_t rkp_slab(int D, int F) { return (size_t)6 * D + 4 * kRkPRank + F; }

bool rkp_shape_ok(int D, int F, int HS, int NH, const int (*ranks)[4], int L);
// The exact-order kernel (rkexact.hip): its shapes, grid and launch. Its
// layer table's matrices are fp32 (output, input) rows (block 0); the head
// may be INT4 (group 32 or 64) or fp32.
bool rke_shape_ok(int D, int F, int HS, int NH, const int (*ranks)[4], int L);
bool rke_grid_ok(int G, int D, int F, int p1rows);
int rke_grid(int NH);
snhip_status launch_rk_exact(const RkPArgs& a, int G, hipStream_t st);
// Workgroups of the launch (a multiple of 8, one per CU), or 0 when the
// device cannot run it.
int rkp_grid(int NH);
snhip_status launch_rk_persist(const RkPArgs& a, int G, hipStream_t st);

}  // namespace snhip
