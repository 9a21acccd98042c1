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
    const uint16_t* h;      // fp16 copy of w (the fp16 format), else null
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
    // k_decode_persist: independent sequences, one per equal slice of the
    // grid (0 or 1: one). Sequence q runs on workgroups [q G, (q+1) G),
    // G = grid / ni, with its own exchange words (ex + 2 q kPersistExWords,
    // sx + q L 2 D), state and history rows (s + q L D, hist + q L kh D),
    // first token tok_in[q], tokens out_tok[step ni + q] and logits
    // logits + q vocab; ring is (grid, L, kh, D) over the whole grid.
    int ni;
};

// Exchange words per epoch slot (>= inner, rank, dim and two per workgroup).
constexpr int kPersistExWords = 2048;

// Conv taps the kernel is built for, and its largest grid.
constexpr int kPersistTaps = 4;
constexpr int kPersistMaxGrid = 1024;
// Sequences one launch of the single-sequence kernel steps at most (a.ni).
constexpr int kPersistMiMax = 64;

// Workgroups per CU the kernel can keep resident (0 if it cannot run).
int persist_occupancy(int blk);
// Grid sizes the kernel accepts for a shape: G divides dim, each workgroup's
// dim / G channels are whole channel groups of 8 or an equal part of one, and
// every workgroup gets rows of V, W_z and the head.
bool persist_grid_ok(int G, int D, int I, int R, int vocab);
snhip_status launch_decode_persist(const PersistArgs& a, int nwg, int blk, hipStream_t st);

// Persistent step of a batch of sequences (batch.hip): every layer of one
// decode step in one cooperative launch, phases separated by grid barriers.
// Each phase writes its outputs to buffers no other phase of the launch
// writes (per-layer slabs), with agent-coherent stores, so a barrier needs no
// cache fences: a line a workgroup reads after a barrier was not cached by
// its XCD earlier in the launch.
constexpr int kBatchMaxK = 1536;       // deepest product: 8 waves x 3 chunks of 64
constexpr int kBatchMaxRow = 2048;     // longest LayerNorm row: 512 threads x 4

struct BatchArgs {
    const PLayer* layers;   // device array of L layers
    int L, B, D, I, R, K, kh, clamp;
    float eps, p_floor;
    const float *no_g, *no_c;
    const int32_t* tok;     // (B) the step's token ids: layer 0's input is their embedding rows
    const float* embed;     // (vocab, D); an id outside [0, vocab) gives a NaN row
    int vocab;
    float* xs;              // (L, B, D) residual after each layer
    float* at;              // (L, B, D) LN_in + conv
    float* v;               // (L, B, R) V at
    float* sfb;             // (L, B, D) W_eff s (old state)
    float* u;               // (L, B, D) gated values
    float* z;               // (L, B, I) W_z u with the wedge
    float* sn;              // (L, B, D) new state
    float* s;               // (B, L, D) state: old in, new out
    float* hist;            // (B, L, kh, D) conv history, newest first
    float* nrm;             // (B, D) LN_out of the last residual (the head's input)
    unsigned* flags;        // batch_flag_words(L, B, ...) dataflow flags, zeroed once
    unsigned epoch;         // this launch's epoch (> 0, one more per launch)
    unsigned* err;          // set on a wait's time-out
    unsigned spin_limit;    // polls before a wait gives up
    unsigned stall;         // added to every awaited epoch: > 0 only to test the time-out path
};

// Flag words of the batched kernel for L layers at B rows: per layer one per
// row (P0) and one per 16 x 16 tile of P1-P4.
__host__ __device__ inline size_t batch_flag_words(int L, int B, int D, int I, int R) {
    const size_t mb = (size_t)(B + 15) / 16;
    return (size_t)L * ((size_t)B + mb * ((size_t)(R + D) / 16 + (size_t)(2 * D) / 16 + (size_t)I / 16 +
                                          (size_t)D / 16));
}

// Shapes the batched kernel handles: products no deeper than kBatchMaxK in
// whole chunks of 64, LayerNorm rows up to kBatchMaxRow, four conv taps.
bool batch_shape_ok(int D, int I, int R, int K, int L);
// Grid for the batched kernel on this device (a multiple of 8, one
// workgroup per CU), 0 if it cannot run.
int batch_grid(int blk, int D, int I, int R);
snhip_status launch_decode_batch(const BatchArgs& a, int G, int blk, hipStream_t st);

}  // namespace snhip
