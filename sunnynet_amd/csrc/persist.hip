// Persistent decode of one sequence: every layer of every greedy step in one
// cooperative launch (the B = 1 path of snhip_step / snhip_decode_greedy_dev).
//
// The math is the decode step of sunnynet/runtime/sunnynet.c:212-334 (LayerNorm,
// depthwise conv, low-rank U V product, competitive and decay gates, state
// update, W_z read-out with the wedge, LN over inner, W_c + b s' + W_eff s + x,
// final LN and head). A step is a chain of small matrix-vector products, each
// too short to fill the chip as its own launch; here the whole grid walks
// through the step in phases:
//
//   A(l)  x -> LN_in -> conv -> at;  v = V at (rows spread over the grid),
//         sfb = W_eff s_old for the workgroup's own channels
//   B(l)  q = U v for the workgroup's channel group(s) (16 contiguous rows of U
//         per group: 8 values, 8 gates), competitive + decay gate,
//         s' = p s + (1 - p) u for its own channels
//   C(l)  z = wedge(W_z u)
//   D(l)  y = LN_I(z);  x' = W_c y + b s' + sfb + x for its own channels
//   H     logits = E LN_out(x), per-workgroup argmax key
//   T     every workgroup reduces the keys to the same greedy token
//
// Exchange. Each vector a phase produces (v, u, z, x, the keys) is published as
// 64-bit words (epoch << 32 | float bits) with agent-scope stores; the next
// phase's readers poll those words until every epoch matches. Data and flag
// travel in one single-copy-atomic word, so a reader needs no barrier and no
// second round trip: a phase costs one store-to-load latency across XCDs.
// Words are double-buffered by epoch parity. A writer of epoch e + 2 has read
// epoch e + 1 from every workgroup, and each of those read all of epoch e
// before writing e + 1, so no reader is still on the slot being overwritten
// (every workgroup produces and reads every exchange). Buffers are zeroed
// before each launch and epochs start at 1.
//
// Ownership. Workgroup w owns channels [w cpw, (w + 1) cpw): their state s,
// the W_eff and W_c rows, and the residual x. Everything a channel needs in
// phase D (s', sfb, x) is therefore produced inside the workgroup and never
// exchanged; s' is also published (one word per channel, by step parity) for
// every workgroup's W_eff product in the next step. Every workgroup forms the
// full LN_in(x) of each layer, so each keeps its own copy of the last three
// (a ring in global memory, read and written by the same thread) and computes
// the conv in the reference's order, bit-identical. The handle's s / hist are
// read at the first step and written back by the owners after the last.
//
// Weights stream through two register pools per wave: while one batch of rows
// is multiplied, the next batch (or the next phase's first batch) is in
// flight, so a phase starts with its first weights already loaded. Every poll
// loop is bounded: on time-out the error word is set and every workgroup
// leaves at its next poll.
#include "decode.h"

#define SNHIP_PERSIST_NT 1024
#define SNHIP_PERSIST_NS nt1024
#include "persist_kernel.h"
#undef SNHIP_PERSIST_NT
#undef SNHIP_PERSIST_NS
#undef PROF
#undef JPROF
#define SNHIP_PERSIST_NT 512
#define SNHIP_PERSIST_NS nt512
#include "persist_kernel.h"
#undef SNHIP_PERSIST_NT
#undef SNHIP_PERSIST_NS

namespace snhip {

#ifdef SNHIP_PERSIST_PROF
// Timestamps of the INT4 (1024-thread) kernel.
extern "C" int snhip_persist_prof(unsigned long long* out, int n) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(nt1024::g_prof), sizeof(unsigned long long) * n) == hipSuccess;
}
extern "C" int snhip_persist_jprof(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(nt1024::g_jprof), sizeof(unsigned long long) * 64) == hipSuccess;
}
extern "C" int snhip_persist_clk(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(nt1024::g_clk), sizeof(unsigned long long) * 4) == hipSuccess;
}
#endif

namespace {
// fp32 and fp16 rows stream more bytes per phase: 8 waves per workgroup
// measured faster for fp32 and fp16 (fp16 at SunnyNet-100M B=1: 209 us/step
// on 8 waves, 222 on 16), 16 for INT4 g32. INT4 g64 needs more than the
// 128 VGPRs a 16-wave workgroup leaves each wave (it spilled 102 to scratch:
// 307 us/step at SunnyNet-100M B=1) and runs on 8 waves (197 us/step).
bool wide(int blk) { return blk == 0 || blk == 16 || blk == 64; }
int threads_for(int blk) { return wide(blk) ? 512 : 1024; }
const void* kernel_for(int blk) { return wide(blk) ? nt512::kernel_for(blk) : nt1024::kernel_for(blk); }
}  // namespace

int persist_occupancy(int blk) {
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel_for(blk), threads_for(blk), 0);
    return e == hipSuccess ? nb : 0;
}

bool persist_grid_ok(int G, int D, int I, int R, int vocab) {
    if (G < 1 || G > kPersistMaxGrid || D % G) return false;
    const int cpw = D / G;
    if (cpw % 8 != 0 && 8 % cpw != 0) return false;
    return G <= R && G <= I && G <= vocab;
}

snhip_status launch_decode_persist(const PersistArgs& a, int nwg, int blk, hipStream_t st) {
    const int ni = a.ni > 1 ? a.ni : 1;
    if (a.D > kPersistMaxD || a.I > kPersistMaxK || a.R > kPersistMaxK || a.K != kPersistTaps || a.D % 8 || a.L > kPersistMaxL ||
        ni > kPersistMiMax || nwg % ni || !persist_grid_ok(nwg / ni, a.D, a.I, a.R, a.vocab) || a.n_steps < 1 ||
        (a.greedy && !a.out_tok) || (!a.greedy && a.n_steps != 1)) {
        set_last_error("persistent decode: unsupported shape or arguments");
        return SNHIP_E_INVAL;
    }
    PersistArgs args = a;
    void* kargs[] = {&args};
    SNHIP_CHECK(launch_persistent(kernel_for(blk), dim3(nwg), dim3(threads_for(blk)), kargs, st));
    return SNHIP_OK;
}

}  // namespace snhip
