// Persistent single-sequence decode (persist.hip), shared with model.hip.
#pragma once

#include "common.h"

namespace snhip {

// Row order of the low-rank output q = U v (2 dim values) on this backend:
// the 8 value rows and the 8 gate rows of each channel group are adjacent, so
// one group's 16 rows of U are contiguous (U's rows are permuted at load).
__host__ __device__ inline int qrow_u(int i) { return 16 * (i >> 3) + (i & 7); }
__host__ __device__ inline int qrow_g(int i) { return 16 * (i >> 3) + 8 + (i & 7); }

// Largest dim, and inner / rank, the persistent kernel handles (LDS staging
// and per-thread register arrays are sized for them); larger models use the
// per-kernel path.
constexpr int kPersistMaxD = 1024;
constexpr int kPersistMaxK = 1536;
constexpr int kPersistMaxL = 32;             // layers (the layer table is staged in LDS)

// A weight matrix, row-major (M, Kd): fp32 rows in w, or INT4 codes in q
// ((M, Kd/2) bytes, quant.c packing) with per-group scales sc ((M, Kd/block)).
struct PMat {
    const float* w;
    const uint8_t* q;
    const float* sc;
    int M;
};

struct PLayer {
    const float *ni_g, *ni_c, *nm_g, *nm_c, *dw, *delta;
    float a_tanh, b_gain;
    PMat VW;                // V (rank rows) followed by W_eff (dim rows), both (., dim)
    PMat U, Wz, Wc;         // U rows in the qrow_u / qrow_g order
};

struct PersistArgs {
    const PLayer* layers;   // device array of L layers
    int L, D, I, R, K, kh, vocab, clamp;
    float eps, p_floor;
    const float *embed, *no_g, *no_c;
    PMat head;
    float* s;               // (L, D) state: read at the first step, written back after the last
    float* hist;            // (L, kh, D) conv history, newest first: same
    float* ring;            // (grid, L, kh, D) each workgroup's recent LN_in outputs
    unsigned long long* ex; // (2, kPersistExWords) exchange words, zeroed before the launch
    unsigned long long* sx; // (L, 2, D) new-state words, zeroed before the launch
    unsigned* err;          // set on a poll time-out
    const int32_t* tok_in;  // first input token (device)
    int32_t* out_tok;       // greedy: token chosen after each step (n_steps)
    float* logits;          // if not NULL: logits of the last step (vocab)
    int n_steps, greedy;
    unsigned spin_limit;    // polls before a wait gives up
    unsigned stall;         // added to every awaited epoch: > 0 only to test the time-out path
};

// Exchange words per epoch slot (>= inner, rank, dim and two per workgroup).
constexpr int kPersistExWords = 2048;

// Conv taps the kernel is built for, and its largest grid.
constexpr int kPersistTaps = 4;
constexpr int kPersistMaxGrid = 1024;

// Workgroups per CU the kernel can keep resident (0 if it cannot run).
int persist_occupancy(int blk);
// Grid sizes the kernel accepts for a shape: G divides dim, each workgroup's
// dim / G channels are whole channel groups of 8 or an equal part of one, and
// every workgroup gets rows of V, W_z and the head.
bool persist_grid_ok(int G, int D, int I, int R, int vocab);
snhip_status launch_decode_persist(const PersistArgs& a, int nwg, int blk, hipStream_t st);

}  // namespace snhip
