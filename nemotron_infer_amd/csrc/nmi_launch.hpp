// nmi_launch.hpp -- host-side launchers of the gfx950 kernels (internal to libnmi.so).
//
// The C ABI (capi.cpp) validates arguments, then calls these.  Each launcher assumes its
// arguments were validated (shapes, strides, alignment) and returns the hipError_t of the
// launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nmi {

struct DeviceInfo {
    int device = -1;
    int num_cu = 256;
    int num_xcd = 8;
};

// Records the calling thread's last error message (returned by nmi_last_error()).
void set_last_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Per-device properties, queried once per device (thread-safe).
const DeviceInfo& device_info();

// Tuning knobs (0 = automatic).  Set through nmi_tuning_set() for sweeps; never needed for
// correctness.
struct Tuning {
    int gemv_ks = 0;       // M = 1 GEMV: waves of a workgroup that split K (1, 2, 4)
    int gemv_t = 0;        // M = 1 GEMV: weight rows per wave (1, 2, 4)
    int gemv_p = 0;        // M = 1 GEMV: 16-byte chunks per lane per row per batch (2, 3, 4)
    int gemv_xg = 0;       // M = 1 GEMV: 1 reads x from global memory instead of LDS
    int gemm_tile = 0;     // GEMM tile variant id (see gemm_fp8.hip)
    int skinny_ks = 0;     // skinny kernel: waves of a workgroup that split K (1, 2, 4)
    int skinny_kg = 0;     // skinny kernel: workgroups that split K (needs a workspace)
    int skinny_u = 0;      // skinny kernel: 16-byte weight loads per lane per batch (8, 16)
    int m1_path = 0;       // M = 1: 0 automatic, 1 GEMV kernel, 2 split-K skinny kernel, 3 4x4x4 kernel
    int skinny_path = 0;   // 2 <= M <= 16: 0 automatic, 1 split-K 16x16x32 kernel, 2 4x4x4 kernel,
                           // 3 GEMV kernel (M <= 4)
    int s4_ks = 0;         // 4x4x4 skinny kernel: waves splitting K (1, 2, 4)
    int s4_t = 0;          // 4x4x4 skinny kernel: row groups of 4 per wave (1, 2)
    int s4_u = 0;          // 4x4x4 skinny kernel: chunks per lane per batch (2, 4, 8)
    int s4_dma = 0;        // 4x4x4 skinny kernel: 0 pipelined form where it applies, 2 windowed form
    int s4_kg = 0;         // 4x4x4 skinny kernel: workgroups splitting K (> 1, with a workspace; 0, 1: none)
    int gemm_sk = 0;       // GEMM stream-K: 1 whenever a workspace allows; otherwise one tile per workgroup
    int chain_wgs = 0;     // GEMV chain: workgroups per CU (0: 4, or fewer if fewer are resident)
    int chain_wait_us = 0; // GEMV chain: bound of a wait in microseconds (0: 200000)
};
Tuning& tuning();

// Fused output epilogue of a linear (computed by epilogue() in nmi_device.hpp): none, relu^2,
// or the residual add out = res + y with res [M, N] at row stride ldres elements.
enum : int { kEpiNone = 0, kEpiRelu2 = 1, kEpiResidual = 2 };
struct Epi {
    int kind = 0;
    const uint16_t* res = nullptr;
    int64_t ldres = 0;
};

// One matrix of a grouped launch: W [N, K] (row stride ldw bytes), s [N], y [M, N] (row
// stride ldy elements).  wg_begin and ws_col are filled in by the launchers.
constexpr int kMaxGroups = 4;
struct GemvGroup {
    const uint8_t* W;
    int64_t ldw;
    const float* s;
    uint16_t* y;
    int64_t ldy;
    int N;
    int wg_begin;
    int ws_col;
    Epi epi;
};

// RMSNorm of the activations (model/mlp_block.cuh:140, ops/reduce.cuh:135-244):
// y[m, k] = bf16_rne(x[m, k] * (r_m * w[k])), r_m = 1 / sqrt(sum_k x[m, k]^2 / K + eps), the sum
// in float32 in a fixed order that the GEMV kernel's fused form repeats exactly.
struct Norm {
    const float* w = nullptr;   // [K] float32; nullptr: no normalisation
    float eps = 0.f;
};

// M = 1 GEMV over up to kMaxGroups matrices that share x [K] (one launch).
hipError_t launch_gemv_m1_grouped(const uint16_t* x, int K, const GemvGroup* groups, int ngroups,
                                  hipStream_t stream);

// 1 <= M <= 16 on bf16 MFMA over up to kMaxGroups matrices sharing x [M, K].  With a
// workspace of at least skinny_workspace_bytes() bytes (zero-filled before its first use; every
// launch leaves it re-armed) K is also split between workgroups.
size_t skinny_workspace_bytes(int M, int K, int64_t total_rows, int num_cu);
hipError_t launch_skinny_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                                 int ngroups, void* workspace, size_t workspace_bytes, hipStream_t stream);

// 2 <= M <= 16 on 4x4x4 MFMA with coalesced weight reads.  With a workspace of at least
// skinny4_workspace_bytes() bytes (zero-filled before its first use; every launch leaves it
// re-armed; 0 = the schedule has no K split) K is also split between workgroups.
size_t skinny4_workspace_bytes(int M, int K, int64_t total_rows, int num_cu);
hipError_t launch_skinny4_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                                  int ngroups, void* workspace, size_t workspace_bytes, hipStream_t stream);

// The GEMV kernel for 1 <= M <= 4 activation rows (x row stride ldx elements).  With norm.w
// set (only where gemv_norm_supported(M, K)), x is the raw input and every workgroup applies
// the RMSNorm while staging it, with results identical to launch_rmsnorm's.
bool gemv_norm_supported(int M, int K);
hipError_t launch_gemv_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                               int ngroups, hipStream_t stream, const Norm& norm = Norm{});

// RMSNorm of M rows of K bf16 activations (K % 8 == 0): y [M, K] (row stride ldy) from x [M, K]
// (row stride ldx), one 256-thread workgroup per row.
hipError_t launch_rmsnorm(const uint16_t* x, int64_t ldx, const Norm& norm, uint16_t* y, int64_t ldy,
                          int M, int K, hipStream_t stream);

hipError_t launch_gemv_m1(const uint16_t* x, const uint8_t* W, int64_t ldw, const float* s,
                          uint16_t* y, int N, int K, hipStream_t stream);

// One phase of a GEMV chain (M = 1): the grouped GEMV of x [K] against up to kMaxGroups
// matrices.  gemv_chain_plan fills ks, window, item_begin, nitems, signal and each group's
// wg_begin (first work item of the group, relative to the phase); wait = 1 makes the phase wait
// until the previous one has completed before reading x (x may be that phase's output).
struct ChainPhase {
    const uint16_t* x;
    int K;
    int ks;             // waves splitting K (1, 2 or 4)
    int window;         // x chunks staged per window
    int item_begin;     // first work item of the phase
    int nitems;
    int ngroups;
    int wait;
    int signal;         // the next phase waits: completions of this one are counted
    GemvGroup g[kMaxGroups];
};
// Fills the derived fields of phases[0..n) and returns the number of work items; *lds_bytes
// receives the dynamic LDS the launch needs.
int gemv_chain_plan(ChainPhase* phases, int nphases, size_t* lds_bytes);
// One work item of a planned chain, everything its workgroup needs in one 80-byte record (read
// with scalar loads and no dependent lookups: walking a phase table per item cost about 10% of
// the chain's streaming rate): the item's rows of one group.
struct ChainItem {
    const uint8_t* w;       // first weight row of the item
    const uint16_t* x;      // the phase's activations [K]
    uint16_t* y;            // output of the item's first row
    const float* s;         // scale of the item's first row
    int64_t ldw;
    int rows;               // rows of the item that exist (the last item of a group may be short)
    int K;
    int ks;                 // waves splitting K (1, 2, 4)
    int window;             // x chunks per LDS window
    int phase;
    int flags;              // kChainWait | kChainSignal
    int wait_need;          // done count of the previous phase that completes it
    int stripe;             // completion stripe of the item
    int stripe_items;       // items of the phase in that stripe
};
static_assert(sizeof(ChainItem) == 80, "one 80-byte record per item");
enum : int { kChainWait = 1, kChainSignal = 2 };
// The items of planned phases[0..n) in order (out: the count gemv_chain_plan returned).
void gemv_chain_items(const ChainPhase* planned, int nphases, ChainItem* out);
// Counter workspace of a chain: per phase kChainStripes stripe counters and one done counter,
// then kChainStripes exit counters and one exit-done counter, each on its own 128-byte line;
// the last line (an even number of lines: a multiple of 256 bytes) holds the error word; zero
// at rest.
constexpr int kChainStripes = 8;
constexpr int kChainLineWords = 32;
constexpr int gemv_chain_counter_lines(int nphases) {
    return ((nphases + 1) * (kChainStripes + 1) + 2) & ~1;
}
inline size_t gemv_chain_counter_bytes(int nphases) {
    return (size_t)gemv_chain_counter_lines(nphases) * kChainLineWords * sizeof(uint32_t);
}
// Workgroups of the launch: the items, at most as many as are resident at once on the current
// device (the workgroups wait on each other's items) and at most 4 per CU (tuning knob
// chain.wgs sets that cap).
hipError_t gemv_chain_grid(size_t lds_bytes, int total_items, int* grid);
// items: the item table in device memory; ctr: gemv_chain_counter_bytes(nphases) bytes.
hipError_t launch_gemv_chain(const ChainItem* items, int nphases, int total_items, int grid, size_t lds_bytes,
                             uint32_t* ctr, hipStream_t stream);

// Prefill GEMM.  Given a workspace of at least gemm_workspace_bytes(M) bytes whose first 64 KiB
// (the flag region) are zero -- every launch leaves them zero again -- the DMA-fed kernel splits
// the k tiles of all tiles evenly between the CUs (stream-K) when the tiles cover at most half
// of them (tuning knob gemm.sk = 1: always, also for the 8-wave kernels; 2: never); otherwise
// one tile per workgroup.  launch_sk_flags_clear zeroes the flag region (one small kernel, safe
// under graph capture).
size_t gemm_workspace_bytes(int M);
hipError_t launch_sk_flags_clear(void* ws, hipStream_t stream);
hipError_t launch_gemm(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw,
                       const float* s, uint16_t* y, int64_t ldy, int M, int N, int K,
                       hipStream_t stream, const Epi& epi = Epi{}, void* ws = nullptr, size_t ws_bytes = 0);

hipError_t launch_decode(const uint8_t* codes, float* out_f32, float* out_scaled,
                         uint16_t* out_bf16, float scale, int n, hipStream_t stream);

// Kernel chosen for a linear with M activation rows (tuning knobs may override).
enum class Path { Gemv, Skinny, Skinny4, Gemm };
Path choose_path(int M);

// One or more linears sharing x [M, K] on the kernel choose_path(M) names (GEMM: one launch per
// matrix).  norm (GEMV path only, where gemv_norm_supported) applies the RMSNorm to x first.
hipError_t dispatch_linear(const uint16_t* x, int64_t ldx, int M, int K, GemvGroup* g, int ng, void* ws,
                           size_t ws_bytes, hipStream_t stream, const Norm& norm = Norm{});

}  // namespace nmi
