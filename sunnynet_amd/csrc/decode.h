// Persistent single-sequence decode (persist.hip), shared with model.hip.
#pragma once

#include "common.h"

namespace snhip {

// Largest dim / inner / rank the persistent kernel handles (LDS staging and
// register batches are sized for it); larger models use the per-kernel path.
constexpr int kPersistMaxDim = 2048;
constexpr int kPersistMaxTaps = 8;

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
    PMat V, U, Wz, Wc, Ws;
};

struct PersistArgs {
    const PLayer* layers;   // device array of L layers
    int L, D, I, R, K, kh, vocab, clamp;
    float eps, p_floor;
    const float *embed, *no_g, *no_c;
    PMat head;
    float* s;               // (L, D) state of the sequence
    float* hist;            // (L, kh, D) conv history, newest first
    float *x, *v, *sfb, *u, *z;   // exchange buffers: D, R, D, D, I floats
    unsigned long long* part;     // per-workgroup argmax keys (grid size)
    unsigned* bar;                // barrier words (kPersistBarWords), zeroed before launch
    const int32_t* tok_in;        // first input token (device)
    int32_t* out_tok;             // greedy: token chosen after each step (n_steps)
    float* logits;                // if not NULL: logits of the last step (vocab)
    int n_steps, greedy;
    unsigned spin_limit;    // polls before a barrier wait gives up
    unsigned stall;         // added to every barrier target: > 0 only to test the time-out path
};

// Barrier words: 8 group counters 128 bytes apart, the top counter, the
// time-out flag.
constexpr int kPersistBarWords = 320;
constexpr int kPersistBarErr = 288;

// Workgroups per CU the kernel can keep resident (0 if it cannot run).
int persist_occupancy(int blk);
snhip_status launch_decode_persist(const PersistArgs& a, int nwg, int blk, hipStream_t st);

}  // namespace snhip
