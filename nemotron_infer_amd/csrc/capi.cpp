// capi.cpp -- extern "C" boundary of libnmi.so (declared in include/nmi_fp8_linear.h).
//
// Validates every argument on the host before anything is launched (the reference checks
// nothing: ops/gemv.cuh:92-104 and ops/gemm.cuh:325-403 launch unconditionally and ignore
// return codes), records a per-thread error message, and dispatches on M as the reference's
// fp8 blocks do (model/mlp_block.cuh:142: M == 1 -> GEMV, otherwise GEMM).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "nmi_fp8_linear.h"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return NMI_OK;
    return fail((int)e, "%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const float* s,
                 const void* y, int64_t ldy, int M, int N, int K, const char* fn) {
    if (!x || !w || !s || !y) return fail(NMI_ERR_INVALID_ARG, "%s: NULL pointer argument", fn);
    if (M < 1 || N < 1) return fail(NMI_ERR_INVALID_ARG, "%s: M=%d N=%d must be >= 1", fn, M, N);
    if (K < 16 || K % 16 != 0)
        return fail(NMI_ERR_INVALID_ARG, "%s: K=%d must be a positive multiple of 16", fn, K);
    if (ldx < K || ldw < K || ldy < N)
        return fail(NMI_ERR_INVALID_ARG, "%s: strides ldx=%lld ldw=%lld ldy=%lld too small for K=%d N=%d",
                    fn, (long long)ldx, (long long)ldw, (long long)ldy, K, N);
    if (!aligned(w, 16) || ldw % 16 != 0)
        return fail(NMI_ERR_ALIGNMENT, "%s: W and ldw must be 16-byte aligned", fn);
    if (!aligned(x, 16) || ldx % 8 != 0)
        return fail(NMI_ERR_ALIGNMENT, "%s: x and ldx*2 must be 16-byte aligned", fn);
    if (!aligned(s, 4)) return fail(NMI_ERR_ALIGNMENT, "%s: w_scale must be 4-byte aligned", fn);
    if (!aligned(y, 2)) return fail(NMI_ERR_ALIGNMENT, "%s: y must be 2-byte aligned", fn);
    return NMI_OK;
}

std::mutex g_dev_mu;
std::vector<DeviceInfo> g_devs;

}  // namespace

void set_last_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

const DeviceInfo& device_info() {
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(g_dev_mu);
    if ((int)g_devs.size() <= dev) g_devs.resize(dev + 1);
    DeviceInfo& d = g_devs[dev];
    if (d.device < 0) {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cu > 0)
            d.num_cu = cu;
        d.device = dev;
    }
    return d;
}

Tuning& tuning() {
    static Tuning t;
    return t;
}

namespace {
constexpr int kAsyncMaxDevices = 64;
std::atomic<uint32_t*> g_async_words{nullptr};
std::once_flag g_async_once;
}  // namespace

uint32_t* async_error_word() {
    std::call_once(g_async_once, [] {
        // pinned, coherent host memory: the kernel's system-scope store is visible to the host
        // without a GPU synchronisation; one word per device
        void* p = nullptr;
        if (hipHostMalloc(&p, kAsyncMaxDevices * sizeof(uint32_t), hipHostMallocCoherent | hipHostMallocPortable) ==
                hipSuccess &&
            p) {
            std::memset(p, 0, kAsyncMaxDevices * sizeof(uint32_t));
            g_async_words.store(static_cast<uint32_t*>(p), std::memory_order_release);
        } else {
            (void)hipGetLastError();
        }
    });
    uint32_t* w = g_async_words.load(std::memory_order_acquire);
    const int dev = device_info().device;
    return (w && dev >= 0 && dev < kAsyncMaxDevices) ? w + dev : nullptr;
}

bool take_async_error(const char* fn) {
    uint32_t* w = g_async_words.load(std::memory_order_acquire);
    if (!w) return false;                           // no stream-K launch yet in this process
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kAsyncMaxDevices) return false;
    if (__atomic_load_n(w + dev, __ATOMIC_ACQUIRE) == 0u) return false;
    __atomic_store_n(w + dev, 0u, __ATOMIC_RELAXED);
    set_last_error("%s: a stream-K GEMM launched earlier on device %d gave up waiting for a partial tile, so that "
                   "launch's output is wrong (the error word of its workspace, byte %d, is set; its flags were left "
                   "re-armed); nothing was launched by this call",
                   fn, dev, NMI_WS_ERROR_OFFSET);
    return true;
}

}  // namespace nmi

namespace nmi {

size_t linear_workspace_bytes(int M, int64_t total_n, int K) {
    if (M < 1 || K < 16 || K % 16 != 0 || total_n < 1) return 0;
    const int t = tuning().gemm_tile;
    if (M > 16 && M < 512)                            // the short-prompt kernel's K-split partials
        return (t == 0 || t == 2) ? gemm_short_workspace_bytes(M, (int)std::min<int64_t>(total_n, 1 << 30), K) : 0;
    if (M > 16) return gemm_workspace_bytes(M);       // stream-K flags and partials of the GEMM
    return 0;                                         // the GEMV and skinny kernels use none
}

bool gemm_workspace_has_flags(int M) { return M >= 512 && choose_path(M) == Path::Gemm && gemm_workspace_bytes(M) > 0; }

// M == 1 -> GEMV kernel, M == 2 -> GEMV kernel when it fuses the RMSNorm, else the 16x16x32
// skinny kernel where it takes the shape (dispatch_linear), M <= 16 -> the skinny kernels
// (16x16x32, or 4x4x4 where that one declines), M > 16 -> MFMA GEMM.
Path choose_path(int M) {
    const Tuning& t = tuning();
    if (M == 1) {
        if (t.m1_path == 3) return Path::Skinny4;
        return Path::Gemv;
    }
    if (M <= 16) {
        if ((t.skinny_path == 3 && M <= 4) || (t.skinny_path == 0 && M == 2)) return Path::Gemv;
        return Path::Skinny4;
    }
    return Path::Gemm;
}

bool gemv_fuses_norm(int M, int K) {
    if (choose_path(M) != Path::Gemv || !gemv_norm_supported(M, K)) return false;
    return !(M == 2 && tuning().skinny_path == 0 && K % 64 == 0 && skinny16_wanted(M, K));
}

hipError_t dispatch_linear(const uint16_t* x, int64_t ldx, int M, int K, GemvGroup* g, int ng, void* ws,
                           size_t ws_bytes, hipStream_t st, const Norm& norm) {
    const Path path = choose_path(M);
    if (norm.w && path != Path::Gemv) return hipErrorInvalidValue;
    switch (path) {
        case Path::Gemv: {
            // M = 2 without a fused RMSNorm: the 16x16x32 skinny kernel where it takes the shape
            hipError_t e = hipSuccess;
            if (M == 2 && !norm.w && tuning().skinny_path == 0 && launch_skinny16_grouped(x, ldx, M, K, g, ng, st, &e))
                return e;
            return launch_gemv_grouped(x, ldx, M, K, g, ng, st, norm);
        }
        case Path::Skinny4: {
            hipError_t e = hipSuccess;
            if (launch_skinny16_grouped(x, ldx, M, K, g, ng, st, &e)) return e;
            return launch_skinny4_grouped(x, ldx, M, K, g, ng, st);
        }
        case Path::Gemm: break;
    }
    return launch_gemm_grouped(x, ldx, M, K, g, ng, st, ws, ws_bytes);
}

}  // namespace nmi

using namespace nmi;

namespace {

int dispatch(const uint16_t* x, int64_t ldx, int M, int K, GemvGroup* g, int ng, void* ws,
             size_t ws_bytes, hipStream_t st, const char* fn) {
    return hip_status(dispatch_linear(x, ldx, M, K, g, ng, ws, ws_bytes, st), fn);
}

int64_t total_rows(const nmi_linear_group* groups, int ngroups) {
    int64_t r = 0;
    for (int i = 0; i < ngroups; ++i) r += groups[i].N;
    return r;
}

}  // namespace

extern "C" {

int nmi_abi_version(void) { return 10000; }

const char* nmi_last_error(void) { return g_last_error.c_str(); }

int nmi_gemv_fp8(const void* x_bf16, const void* w_e4m3, const float* w_scale, void* y_bf16,
                 int N, int K, void* stream) {
    int rc = check_linear(x_bf16, K, w_e4m3, K, w_scale, y_bf16, N, 1, N, K, "nmi_gemv_fp8");
    if (rc) return rc;
    if (take_async_error("nmi_gemv_fp8")) return NMI_ERR_ASYNC;
    return hip_status(launch_gemv_m1(static_cast<const uint16_t*>(x_bf16),
                                     static_cast<const uint8_t*>(w_e4m3), K, w_scale,
                                     static_cast<uint16_t*>(y_bf16), N, K,
                                     static_cast<hipStream_t>(stream)),
                      "nmi_gemv_fp8 launch");
}


int nmi_linear_fp8_w8a16(const void* x_bf16, int64_t ldx, const void* w_e4m3, int64_t ldw,
                         const float* w_scale, void* y_bf16, int64_t ldy, int M, int N, int K,
                         void* stream) {
    return nmi_linear_fp8_w8a16_ws(x_bf16, ldx, w_e4m3, ldw, w_scale, y_bf16, ldy, M, N, K, nullptr, 0,
                                   stream);
}

int nmi_linear_fp8_w8a16_ws(const void* x_bf16, int64_t ldx, const void* w_e4m3, int64_t ldw,
                            const float* w_scale, void* y_bf16, int64_t ldy, int M, int N, int K,
                            void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = workspace ? "nmi_linear_fp8_w8a16_ws" : "nmi_linear_fp8_w8a16";
    int rc = check_linear(x_bf16, ldx, w_e4m3, ldw, w_scale, y_bf16, ldy, M, N, K, fn);
    if (rc) return rc;
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    if (workspace && !aligned(workspace, 256))
        return fail(NMI_ERR_ALIGNMENT, "%s: workspace must be 256-byte aligned", fn);
    GemvGroup g{static_cast<const uint8_t*>(w_e4m3), ldw, w_scale, static_cast<uint16_t*>(y_bf16), ldy, N, 0, 0, Epi{}};
    return dispatch(static_cast<const uint16_t*>(x_bf16), ldx, M, K, &g, 1, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream), fn);
}

int nmi_linear_fp8_w8a16_grouped(const void* x_bf16, int64_t ldx, int M, int K,
                                 const nmi_linear_group* groups, int ngroups, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_linear_fp8_w8a16_grouped";
    if (!groups || ngroups < 1 || ngroups > NMI_MAX_GROUPS)
        return fail(NMI_ERR_INVALID_ARG, "%s: ngroups=%d must be in [1, %d]", fn, ngroups, NMI_MAX_GROUPS);
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    if (workspace && !aligned(workspace, 256))
        return fail(NMI_ERR_ALIGNMENT, "%s: workspace must be 256-byte aligned", fn);
    if (total_rows(groups, ngroups) > (int64_t)1 << 30)
        return fail(NMI_ERR_INVALID_ARG, "%s: too many rows in total", fn);
    GemvGroup g[kMaxGroups];
    for (int i = 0; i < ngroups; ++i) {
        const nmi_linear_group& G = groups[i];
        int rc = check_linear(x_bf16, ldx, G.w_e4m3, G.ldw, G.w_scale, G.y_bf16, G.ldy, M, G.N, K, fn);
        if (rc) return rc;
        g[i] = GemvGroup{static_cast<const uint8_t*>(G.w_e4m3), G.ldw, G.w_scale,
                         static_cast<uint16_t*>(G.y_bf16), G.ldy, G.N, 0, 0, Epi{}};
    }
    return dispatch(static_cast<const uint16_t*>(x_bf16), ldx, M, K, g, ngroups, workspace, workspace_bytes,
                    static_cast<hipStream_t>(stream), fn);
}

int nmi_linear_fp8_w8a16_batch(const nmi_linear_job* jobs, int njobs, int M, void* stream) {
    const char* fn = "nmi_linear_fp8_w8a16_batch";
    static_assert(NMI_MAX_BATCH <= kS16MaxBatch, "batch size");
    if (!jobs || njobs < 1 || njobs > NMI_MAX_BATCH)
        return fail(NMI_ERR_INVALID_ARG, "%s: njobs=%d must be in [1, %d]", fn, njobs, NMI_MAX_BATCH);
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    GemvGroup g[NMI_MAX_BATCH];
    const uint16_t* xs[NMI_MAX_BATCH];
    int64_t ldxs[NMI_MAX_BATCH];
    int Ks[NMI_MAX_BATCH];
    int64_t rows = 0;
    for (int i = 0; i < njobs; ++i) {
        const nmi_linear_job& J = jobs[i];
        const nmi_linear_group& G = J.w;
        int rc = check_linear(J.x_bf16, J.ldx, G.w_e4m3, G.ldw, G.w_scale, G.y_bf16, G.ldy, M, G.N, J.K, fn);
        if (rc) return rc;
        rows += G.N;
        g[i] = GemvGroup{static_cast<const uint8_t*>(G.w_e4m3), G.ldw, G.w_scale,
                         static_cast<uint16_t*>(G.y_bf16), G.ldy, G.N, 0, 0, Epi{}};
        xs[i] = static_cast<const uint16_t*>(J.x_bf16);
        ldxs[i] = J.ldx;
        Ks[i] = J.K;
    }
    if (rows > (int64_t)1 << 30) return fail(NMI_ERR_INVALID_ARG, "%s: too many rows in total", fn);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (M >= 2 && M <= 16 && launch_skinny16_batch(xs, ldxs, Ks, g, njobs, M, st, &e))
        return hip_status(e, fn);
    for (int i = 0; i < njobs; ++i) {
        const int rc = dispatch(xs[i], ldxs[i], M, Ks[i], &g[i], 1, nullptr, 0, st, fn);
        if (rc) return rc;
    }
    return NMI_OK;
}

// GEMV chain: the planned phase table and per-wave step counts live in device memory for the
// handle's lifetime; one launch per segment (a run of phases up to the next one that waits).  A
// segment of one phase (every phase of a fully dependent chain) is launched as the single GEMV
// launch of that phase instead: x staged once per workgroup in LDS rather than read per step,
// the same arithmetic and so the same bytes (measured on MI355X: config 1 as a dependent chain
// 33.0 -> 30.4 us, the rate of four separate launches).
struct ChainSegment {
    int p0, nphases;                        // phases of the segment
    int total_rg;                           // its row groups
    int grid;
    size_t steps_off;                       // its waves' step counts in wave_steps
};
struct nmi_gemv_chain {
    StreamPhase* dev = nullptr;             // the phase table
    int* wave_steps = nullptr;              // steps of each wave, segment by segment
    std::vector<ChainSegment> seg;
    std::vector<StreamPhase> host;          // the phase table on the host (single-phase segments)
    int nphases = 0;
    int device = -1;
};

int nmi_gemv_chain_create(const nmi_gemv_phase* phases, int nphases, nmi_gemv_chain** out) {
    const char* fn = "nmi_gemv_chain_create";
    if (!out) return fail(NMI_ERR_INVALID_ARG, "%s: out is NULL", fn);
    *out = nullptr;
    if (!phases || nphases < 1 || nphases > NMI_MAX_CHAIN_PHASES)
        return fail(NMI_ERR_INVALID_ARG, "%s: nphases=%d must be in [1, %d]", fn, nphases, NMI_MAX_CHAIN_PHASES);
    std::vector<StreamPhase> host((size_t)nphases);
    std::vector<ChainSegment> seg;
    int64_t rgs = 0;
    for (int p = 0; p < nphases; ++p) {
        const nmi_gemv_phase& P = phases[p];
        if (P.ngroups < 1 || P.ngroups > NMI_MAX_GROUPS)
            return fail(NMI_ERR_INVALID_ARG, "%s: phase %d: ngroups=%d must be in [1, %d]", fn, p, P.ngroups,
                        NMI_MAX_GROUPS);
        StreamPhase& ph = host[(size_t)p];
        ph = StreamPhase{};
        ph.x = static_cast<const uint16_t*>(P.x_bf16);
        ph.K = P.K;
        ph.ngroups = P.ngroups;
        for (int i = 0; i < P.ngroups; ++i) {
            const nmi_linear_group& G = P.groups[i];
            int rc = check_linear(P.x_bf16, P.K, G.w_e4m3, G.ldw, G.w_scale, G.y_bf16, G.ldy, 1, G.N, P.K, fn);
            if (rc) return rc;
            ph.g[i] = StreamGroup{static_cast<const uint8_t*>(G.w_e4m3), G.ldw, G.w_scale,
                                  static_cast<uint16_t*>(G.y_bf16), nullptr, G.N, 0, kEpiNone, 0, 0, 0};
            rgs += (G.N + kStreamChainT - 1) / kStreamChainT;
        }
        if (p == 0 || P.wait_prev) seg.push_back(ChainSegment{p, 0, 0, 0, 0});
        ++seg.back().nphases;
    }
    if (rgs >= ((int64_t)1 << 30)) return fail(NMI_ERR_INVALID_ARG, "%s: too many rows in total", fn);
    // Within a segment the phases are independent, so a long segment is laid out in order of
    // decreasing K slices (a stable order): waves take row groups round-robin in that order, so
    // the row groups of the longest rows are spread over the waves first and the launch ends on
    // the short ones instead of on a few waves still walking long rows.  A row's result does not
    // depend on which wave computes it.  Measured on MI355X: config 4's 84-phase chain 432.2 ->
    // 425.0 us; config 1's four phases 23.7 -> 25.5 us (a short launch is set by its start, not its
    // tail), so segments of at most 8 phases keep the caller's order.
    for (const ChainSegment& sg : seg)
        if (sg.nphases > 8)
            std::stable_sort(host.begin() + sg.p0, host.begin() + sg.p0 + sg.nphases,
                             [](const StreamPhase& a, const StreamPhase& b) {
                                 return ((a.K >> 4) + 255) / 256 > ((b.K >> 4) + 255) / 256;
                             });
    hipError_t e = hipSuccess;
    std::vector<int> steps;
    for (ChainSegment& sg : seg) {
        sg.total_rg = stream_chain_plan(host.data() + sg.p0, sg.nphases);
        if (e == hipSuccess) e = stream_chain_grid(sg.total_rg, &sg.grid);
        if (e != hipSuccess) break;
        sg.steps_off = steps.size();
        steps.resize(steps.size() + (size_t)sg.grid * 4);
        stream_chain_wave_steps(host.data() + sg.p0, sg.nphases, sg.grid * 4, steps.data() + sg.steps_off);
    }
    auto* c = new nmi_gemv_chain;
    c->nphases = nphases;
    c->seg = seg;
    c->host = host;
    if (e == hipSuccess) e = hipGetDevice(&c->device);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&c->dev), host.size() * sizeof(StreamPhase));
    if (e == hipSuccess)
        e = hipMemcpy(c->dev, host.data(), host.size() * sizeof(StreamPhase), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&c->wave_steps), steps.size() * sizeof(int));
    if (e == hipSuccess)
        e = hipMemcpy(c->wave_steps, steps.data(), steps.size() * sizeof(int), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (c->dev) (void)hipFree(c->dev);
        if (c->wave_steps) (void)hipFree(c->wave_steps);
        delete c;
        return hip_status(e, fn);
    }
    *out = c;
    return NMI_OK;
}

size_t nmi_gemv_chain_workspace_bytes(int nphases) {
    (void)nphases;
    return 0;                                                 // no launch of a chain writes one
}

int nmi_gemv_chain_launch(const nmi_gemv_chain* chain, void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_gemv_chain_launch";
    (void)workspace;
    (void)workspace_bytes;
    if (!chain || !chain->dev) return fail(NMI_ERR_INVALID_ARG, "%s: invalid chain", fn);
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    int dev = -1;
    if (hipGetDevice(&dev) == hipSuccess && dev != chain->device)
        return fail(NMI_ERR_INVALID_ARG, "%s: chain was created on device %d, current is %d", fn, chain->device, dev);
    for (const ChainSegment& sg : chain->seg) {
        hipError_t e;
        if (sg.nphases == 1) {
            const StreamPhase& ph = chain->host[(size_t)sg.p0];
            GemvGroup g[kMaxGroups];
            for (int i = 0; i < ph.ngroups; ++i) {
                const StreamGroup& G = ph.g[i];
                g[i] = GemvGroup{G.W, G.ldw, G.s, G.y, G.N, G.N, 0, 0, Epi{}};
            }
            e = launch_gemv_grouped(ph.x, ph.K, 1, ph.K, g, ph.ngroups, static_cast<hipStream_t>(stream), Norm{});
        } else {
            e = launch_gemv_stream_chain(chain->dev + sg.p0, chain->wave_steps + sg.steps_off, sg.nphases,
                                         sg.total_rg, sg.grid, static_cast<hipStream_t>(stream));
        }
        if (e != hipSuccess) return hip_status(e, fn);
    }
    return NMI_OK;
}

int nmi_gemv_chain_destroy(nmi_gemv_chain* chain) {
    if (!chain) return NMI_OK;
    hipError_t e = chain->dev ? hipFree(chain->dev) : hipSuccess;
    const hipError_t e2 = chain->wave_steps ? hipFree(chain->wave_steps) : hipSuccess;
    if (e == hipSuccess) e = e2;
    delete chain;
    return hip_status(e, "nmi_gemv_chain_destroy");
}

size_t nmi_linear_workspace_bytes(int M, int64_t total_n, int K) { return linear_workspace_bytes(M, total_n, K); }

int nmi_gemm_fp8_w8a16(const void* x_bf16, int64_t ldx, const void* w_e4m3, int64_t ldw,
                       const float* w_scale, void* y_bf16, int64_t ldy, int M, int N, int K,
                       void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_linear(x_bf16, ldx, w_e4m3, ldw, w_scale, y_bf16, ldy, M, N, K,
                          "nmi_gemm_fp8_w8a16");
    if (rc) return rc;
    if (workspace && !aligned(workspace, 256))
        return fail(NMI_ERR_ALIGNMENT, "nmi_gemm_fp8_w8a16: workspace must be 256-byte aligned");
    if (take_async_error("nmi_gemm_fp8_w8a16")) return NMI_ERR_ASYNC;
    return hip_status(launch_gemm(static_cast<const uint16_t*>(x_bf16), ldx,
                                  static_cast<const uint8_t*>(w_e4m3), ldw, w_scale,
                                  static_cast<uint16_t*>(y_bf16), ldy, M, N, K,
                                  static_cast<hipStream_t>(stream), Epi{}, workspace, workspace_bytes),
                      "nmi_gemm_fp8_w8a16 launch");
}

int nmi_fp8_e4m3_decode(const void* codes, float* out_f32, float* out_scaled, void* out_bf16,
                        float scale, int n, void* stream) {
    if (!codes || !out_f32 || !out_scaled || !out_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_fp8_e4m3_decode: NULL pointer argument");
    if (n < 4 || n % 4 != 0)
        return fail(NMI_ERR_INVALID_ARG, "nmi_fp8_e4m3_decode: n=%d must be a positive multiple of 4", n);
    if (!aligned(codes, 4) || !aligned(out_f32, 16) || !aligned(out_scaled, 16) || !aligned(out_bf16, 8))
        return fail(NMI_ERR_ALIGNMENT, "nmi_fp8_e4m3_decode: misaligned buffer");
    return hip_status(launch_decode(static_cast<const uint8_t*>(codes), out_f32, out_scaled,
                                    static_cast<uint16_t*>(out_bf16), scale, n,
                                    static_cast<hipStream_t>(stream)),
                      "nmi_fp8_e4m3_decode launch");
}

int nmi_tuning_set(const char* knob, int value) {
    if (!knob) return fail(NMI_ERR_INVALID_ARG, "nmi_tuning_set: NULL knob");
    Tuning& t = tuning();
    if (!std::strcmp(knob, "gemv.ks")) t.gemv_ks = value;
    else if (!std::strcmp(knob, "gemv.t")) t.gemv_t = value;
    else if (!std::strcmp(knob, "gemv.p")) t.gemv_p = value;
    else if (!std::strcmp(knob, "gemv.xg")) t.gemv_xg = value;
    else if (!std::strcmp(knob, "gemm.tile")) t.gemm_tile = value;
    else if (!std::strcmp(knob, "m1.path")) t.m1_path = value;
    else if (!std::strcmp(knob, "skinny.path")) t.skinny_path = value;
    else if (!std::strcmp(knob, "s4.ks")) t.s4_ks = value;
    else if (!std::strcmp(knob, "s4.t")) t.s4_t = value;
    else if (!std::strcmp(knob, "s4.u")) t.s4_u = value;
    else if (!std::strcmp(knob, "gemm.sk")) t.gemm_sk = value;
    else if (!std::strcmp(knob, "gemm.sk_spin")) t.gemm_sk_spin = value;
    else if (!std::strcmp(knob, "gemm.sk_lostflag")) t.gemm_sk_lostflag = value;
    else if (!std::strcmp(knob, "gemm.gh")) t.gemm_gh = value;
    else if (!std::strcmp(knob, "chain.wgs")) t.chain_wgs = value;
    else if (!std::strcmp(knob, "gemv.wgs")) t.gemv_wgs = value;
    else if (!std::strcmp(knob, "gemv.multirow")) t.gemv_multirow = value;
    else if (!std::strcmp(knob, "sdpa.chunk")) t.sdpa_chunk = value;
    else if (!std::strcmp(knob, "gemv.grid")) t.gemv_grid = value;
    else if (!std::strcmp(knob, "gemv.balance")) t.gemv_balance = value;
    else if (!std::strcmp(knob, "gemm.splits")) t.gemm_splits = value;
    else if (!std::strcmp(knob, "gemm.short")) t.gemm_short = value;
    else if (!std::strcmp(knob, "gemm.sk_cap")) t.gemm_sk_cap = value;
    else if (!std::strcmp(knob, "gemm.bm")) t.gemm_bm = value;
    else if (!std::strcmp(knob, "s16")) t.s16 = value;
    else if (!std::strcmp(knob, "s16.r")) t.s16_r = value;
    else if (!std::strcmp(knob, "s16.w")) t.s16_w = value;
    else if (!std::strcmp(knob, "s16.t")) t.s16_t = value;
    else if (!std::strcmp(knob, "mamba.scan")) t.mamba_scan = value;
    else return fail(NMI_ERR_INVALID_ARG, "nmi_tuning_set: unknown knob '%s'", knob);
    return NMI_OK;
}

int nmi_sync(void) {
    const int rc = hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (rc) return rc;
    return take_async_error("nmi_sync") ? NMI_ERR_ASYNC : NMI_OK;
}

int nmi_async_status(void) { return take_async_error("nmi_async_status") ? NMI_ERR_ASYNC : NMI_OK; }

}  // extern "C"
