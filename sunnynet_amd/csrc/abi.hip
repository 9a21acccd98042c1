// Stable C ABI of the HIP backend (include/snhip_abi.h), mirroring
// sunnynet/runtime/sn_abi.c:17-86: same argument validation, status codes
// and version rules; the recurrence and INT4 primitives run on the GPU.
#include <cstdio>
#include <cstring>
#include <set>
#include <thread>
#include <utility>

#include "common.h"

namespace snhip {
namespace {
thread_local std::string g_last_error;
int g_threads = 0;
}  // namespace
void set_last_error(const std::string& msg) { g_last_error = msg; }
const std::string& last_error() { return g_last_error; }
int host_threads() {
    if (g_threads > 0) return g_threads;
    const unsigned n = std::thread::hardware_concurrency();
    return n > 0 ? (int)n : 1;
}
}  // namespace snhip

using namespace snhip;

namespace {
constexpr const char* kVersion = "1.1.0";

int32_t copy_str(const char* src, char* buf, int32_t buflen) {
    const int32_t need = (int32_t)std::strlen(src) + 1;
    if (buf == nullptr || buflen < need) return need;
    std::memcpy(buf, src, (size_t)need);
    return need;
}

// sn_abi.c:52-54
bool dims_bad(const void* p, int32_t a, int32_t b) { return p == nullptr || a <= 0 || b <= 0; }

// Scoped device buffer for the host-pointer entry points.
struct DevBuf {
    void* p = nullptr;
    ~DevBuf() { if (p) (void)hipFree(p); }
};
}  // namespace

extern "C" {

int32_t snhip_abi_version(void) { return SNHIP_ABI_VERSION; }

uint32_t snhip_abi_caps(void) {
    return SNHIP_CAP_RECUR_SCAN | SNHIP_CAP_RECUR_STEP | SNHIP_CAP_RWKV7 | SNHIP_CAP_THREADS |
           SNHIP_CAP_DEVICE_PTR | SNHIP_CAP_SUNNY_MODEL | SNHIP_CAP_INT4 | SNHIP_CAP_BATCH |
           SNHIP_CAP_PREFILL;
}

snhip_status snhip_abi_check(int32_t caller_major) {
    return caller_major == SNHIP_ABI_VERSION_MAJOR ? SNHIP_OK : SNHIP_E_UNSUPPORTED;
}

int32_t snhip_abi_version_string(char* buf, int32_t buflen) { return copy_str(kVersion, buf, buflen); }
int32_t snhip_abi_backend_string(char* buf, int32_t buflen) { return copy_str("hip", buf, buflen); }
int32_t snhip_abi_last_error(char* buf, int32_t buflen) {
    return copy_str(last_error().c_str(), buf, buflen);
}

snhip_status snhip_abi_set_threads(int32_t n) {
    if (n <= 0) return SNHIP_E_INVAL;
    g_threads = (int)n;
    return SNHIP_OK;
}
int32_t snhip_abi_get_threads(void) { return (int32_t)host_threads(); }

// sunnynet.h:42-47. The reference sizes its OpenMP GEMVs with these; here the
// products run on the GPU and the count sizes the host-side load preparation
// (the same setting as snhip_abi_set_threads).
void snhip_set_threads(int n) {
    if (n > 0) g_threads = n;
}
int snhip_get_threads(void) { return host_threads(); }

// Physical cores: distinct (physical id, core id) pairs of /proc/cpuinfo; the
// logical count when the file lists none; 0 when it cannot be read.
int snhip_recommended_threads(void) {
    FILE* f = std::fopen("/proc/cpuinfo", "r");
    if (!f) return 0;
    std::set<std::pair<int, int>> cores;
    char line[512];
    int phys = -1, core = -1;
    auto flush = [&]() {
        if (core >= 0) cores.emplace(phys, core);
        phys = core = -1;
    };
    while (std::fgets(line, sizeof line, f)) {
        int v;
        if (std::sscanf(line, "physical id : %d", &v) == 1) phys = v;
        else if (std::sscanf(line, "core id : %d", &v) == 1) core = v;
        else if (line[0] == '\n') flush();
    }
    flush();
    std::fclose(f);
    if (!cores.empty()) return (int)cores.size();
    const unsigned n = std::thread::hardware_concurrency();
    return (int)n;
}

snhip_status snhip_abi_recur_step_dev(const float* a, const float* b, float* s, int32_t B,
                                      int32_t N, int32_t gated, void* stream) {
    if (dims_bad(a, B, N) || b == nullptr || s == nullptr) return SNHIP_E_INVAL;
    return launch_recur_step(a, b, s, B, N, gated ? 1 : 0, as_stream(stream));
}

snhip_status snhip_abi_recur_scan_dev(const float* a, const float* b, const float* s0,
                                      float* out, float* send, int32_t B, int32_t T,
                                      int32_t N, int32_t gated, void* stream) {
    if (dims_bad(a, B, N) || b == nullptr || s0 == nullptr || out == nullptr ||
        send == nullptr || T <= 0)
        return SNHIP_E_INVAL;
    return launch_recur_scan(a, b, s0, out, send, B, T, N, gated ? 1 : 0, as_stream(stream));
}

snhip_status snhip_abi_scan_bwd_dev(const float* p, const float* nu, const float* s0,
                                    const float* out, const float* dout, float* dp, float* dnu,
                                    float* ds0, int32_t B, int32_t T, int32_t N, void* stream) {
    if (dims_bad(p, B, N) || !nu || !s0 || !out || !dout || !dp || !dnu || !ds0 || T <= 0)
        return SNHIP_E_INVAL;
    return launch_scan_bwd(p, nu, s0, out, dout, dp, dnu, ds0, B, T, N, as_stream(stream));
}

snhip_status snhip_abi_core_fwd_dev(const float* q, const float* delta, const float* s0,
                                    float* states, float* u, float* p, int32_t B, int32_t T,
                                    int32_t D, void* stream) {
    if (!q || !delta || !s0 || !states || !u || !p || B <= 0 || T <= 0 || D <= 0 || D % 8 != 0)
        return SNHIP_E_INVAL;
    return launch_core_fwd(q, delta, s0, states, u, p, B, T, D, as_stream(stream));
}

snhip_status snhip_abi_core_bwd_dev(const float* q, const float* delta, const float* s0,
                                    const float* states, const float* u, const float* p,
                                    const float* dstate, const float* du_in, float* dq,
                                    float* ddelta, float* ds0, int32_t B, int32_t T, int32_t D,
                                    void* stream) {
    if (!q || !delta || !s0 || !states || !u || !p || !dstate || !du_in || !dq || !ddelta || !ds0 ||
        B <= 0 || T <= 0 || D <= 0 || D % 8 != 0)
        return SNHIP_E_INVAL;
    return launch_core_bwd(q, delta, s0, states, u, p, dstate, du_in, dq, ddelta, ds0, B, T, D,
                           as_stream(stream));
}

snhip_status snhip_abi_core_bwd_dev_noalloc(const float* q, const float* delta, const float* s0,
                                            const float* states, const float* u, const float* p,
                                            const float* dstate, const float* du_in, float* dq,
                                            float* ddelta, float* ds0, int32_t B, int32_t T,
                                            int32_t D, void* stream) {
    if (!q || !delta || !s0 || !states || !u || !p || !dstate || !du_in || !dq || !ddelta || !ds0 ||
        B <= 0 || T <= 0 || D <= 0 || D % 8 != 0)
        return SNHIP_E_INVAL;
    return launch_core_bwd_noalloc(q, delta, s0, states, u, p, dstate, du_in, dq, ddelta, ds0, B, T, D,
                                   as_stream(stream));
}

snhip_status snhip_abi_recur_step(const float* a, const float* b, float* s, int32_t B,
                                  int32_t N, int32_t gated) {
    if (dims_bad(a, B, N) || b == nullptr || s == nullptr) return SNHIP_E_INVAL;
    const size_t n = (size_t)B * N * sizeof(float);
    DevBuf da, db, ds;
    SNHIP_CHECK(hipMalloc(&da.p, n));
    SNHIP_CHECK(hipMalloc(&db.p, n));
    SNHIP_CHECK(hipMalloc(&ds.p, n));
    SNHIP_CHECK(hipMemcpy(da.p, a, n, hipMemcpyHostToDevice));
    SNHIP_CHECK(hipMemcpy(db.p, b, n, hipMemcpyHostToDevice));
    SNHIP_CHECK(hipMemcpy(ds.p, s, n, hipMemcpyHostToDevice));
    const snhip_status rc = launch_recur_step((const float*)da.p, (const float*)db.p,
                                              (float*)ds.p, B, N, gated ? 1 : 0, nullptr);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipMemcpy(s, ds.p, n, hipMemcpyDeviceToHost));
    return SNHIP_OK;
}

snhip_status snhip_abi_recur_scan(const float* a, const float* b, const float* s0, float* out,
                                  float* send, int32_t B, int32_t T, int32_t N, int32_t gated) {
    if (dims_bad(a, B, N) || b == nullptr || s0 == nullptr || out == nullptr ||
        send == nullptr || T <= 0)
        return SNHIP_E_INVAL;
    const size_t nbt = (size_t)B * T * N * sizeof(float), nb = (size_t)B * N * sizeof(float);
    DevBuf da, db, d0, dout, dsend;
    SNHIP_CHECK(hipMalloc(&da.p, nbt));
    SNHIP_CHECK(hipMalloc(&db.p, nbt));
    SNHIP_CHECK(hipMalloc(&dout.p, nbt));
    SNHIP_CHECK(hipMalloc(&d0.p, nb));
    SNHIP_CHECK(hipMalloc(&dsend.p, nb));
    SNHIP_CHECK(hipMemcpy(da.p, a, nbt, hipMemcpyHostToDevice));
    SNHIP_CHECK(hipMemcpy(db.p, b, nbt, hipMemcpyHostToDevice));
    SNHIP_CHECK(hipMemcpy(d0.p, s0, nb, hipMemcpyHostToDevice));
    const snhip_status rc = launch_recur_scan((const float*)da.p, (const float*)db.p,
                                              (const float*)d0.p, (float*)dout.p,
                                              (float*)dsend.p, B, T, N, gated ? 1 : 0, nullptr);
    if (rc != SNHIP_OK) return rc;
    SNHIP_CHECK(hipMemcpy(out, dout.p, nbt, hipMemcpyDeviceToHost));
    SNHIP_CHECK(hipMemcpy(send, dsend.p, nb, hipMemcpyDeviceToHost));
    return SNHIP_OK;
}

snhip_status snhip_abi_quant_i4_dev(const float* x, uint8_t* q, float* scale, int32_t rows,
                                    int32_t N, int32_t block, void* stream) {
    if (dims_bad(x, rows, N) || q == nullptr || scale == nullptr || block <= 0 || (block & 1) ||
        N % block)
        return SNHIP_E_INVAL;
    return launch_quant_i4(x, q, scale, rows, N, block, as_stream(stream));
}

snhip_status snhip_abi_dequant_i4_dev(const uint8_t* q, const float* scale, float* x,
                                      int32_t rows, int32_t N, int32_t block, void* stream) {
    if (dims_bad(x, rows, N) || q == nullptr || scale == nullptr || block <= 0 || (block & 1) ||
        N % block)
        return SNHIP_E_INVAL;
    return launch_dequant_i4(q, scale, x, rows, N, block, as_stream(stream));
}

}  // extern "C"
