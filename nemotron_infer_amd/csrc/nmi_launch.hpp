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

// Asynchronous errors of the stream-K GEMM: a finisher that gave up waiting for a partial tile
// (that launch's output is wrong) sets the current device's word in pinned host memory as well as
// the workspace's.  async_error_word() returns the device's word (allocated on first use, one
// array for the process; nullptr if that fails, and then the GEMM does not use stream-K).
// take_async_error(fn) reads and clears it without synchronising the GPU; when it was set it
// records a message naming fn and returns true (the caller returns NMI_ERR_ASYNC).
uint32_t* async_error_word();
bool take_async_error(const char* fn);

// Tuning knobs (0 = automatic).  Set through nmi_tuning_set() for sweeps; never needed for
// correctness.
struct Tuning {
    int gemv_ks = 0;       // M = 1 GEMV: waves of a workgroup that split K (1, 2, 4)
    int gemv_t = 0;        // M = 1 GEMV: weight rows per wave (1, 2, 4; the stream kernel: 2, or 4)
    int gemv_p = 0;        // M = 1 GEMV: 16-byte chunks per lane per row per batch (2, 3, 4)
    int gemv_xg = 0;       // M = 1 GEMV: 1 reads x from global memory instead of LDS
    int gemm_tile = 0;     // GEMM tile variant id (see gemm_fp8.hip)
    int m1_path = 0;       // M = 1: 0 automatic, 1 GEMV kernel, 3 4x4x4 kernel
    int skinny_path = 0;   // 2 <= M <= 16: 0 automatic, 2 the skinny kernels also at M = 2, 3 GEMV
                           // kernel (M <= 4)
    int s4_ks = 0;         // 4x4x4 skinny kernel: waves splitting K (1, 2, 4)
    int s4_t = 0;          // 4x4x4 skinny kernel: row groups of 4 per wave (1, 2)
    int s4_u = 0;          // 4x4x4 skinny kernel: chunks per lane per batch (2, 4, 8)
    int gemm_sk = 0;       // GEMM stream-K: 1 whenever a workspace allows; otherwise one tile per workgroup
    int gemm_sk_spin = 0;  // GEMM stream-K: polls of a flag before the wait gives up (0: 2^26)
    int gemm_sk_lostflag = 0;  // GEMM stream-K (tests): 1 = contributors raise their flags only after the finisher gave up
    int chain_wgs = 0;     // GEMV chain: workgroups per CU (0: 2, or fewer if fewer are resident)
    int gemv_wgs = 0;      // M = 1 stream GEMV: workgroups per CU at most (1, 2; 0: 1)
    int gemv_multirow = 0; // M = 1: 1 runs the multi-row GEMV kernel (gemv_fp8.hip) instead of the stream kernel
    int sdpa_chunk = 0;    // attention decode: positions per split (0: kSdpaMinChunk, capped by the grid size)
    int gemv_grid = 0;     // M = 1 stream GEMV (single launches): explicit workgroup count
    int gemv_balance = 0;  // M = 1 stream GEMV (single launches): 2 turns off the grid sizing that makes row groups divide evenly
    int gemm_splits = 0;   // short-prompt GEMM (17 <= M < 512): workgroups splitting K (0: automatic)
    int gemm_short = 0;    // short-prompt GEMM: f + 1 forces kernel form f (0..7, gemm_short.hip)
    int gemm_bm = 0;       // DMA-fed GEMM tile rows: 0 automatic (128 where 256-row tiles cover at most half the CUs), 128, 256
    int gemm_sk_cap = 0;   // GEMM stream-K: at most this many workgroups per tile (0: 2; -1: one per CU)
    int gemm_gh = 0;       // DMA-fed GEMM: row bands per group of the tile order (0: all of them, stream-K: 1)
    int s16 = 0;           // 16x16x32 skinny kernel: 0 automatic (M >= 3), 1 for 2 <= M <= 16, 2 never
    int s16_r = 0;         // 16x16x32 skinny kernel: row tiles of 16 per workgroup (1, 2; 0: by rows)
    int s16_t = 0;         // 16x16x32 skinny kernel: 1 row runs (0: DMA where it fits)
    int s16_w = 0;         // 16x16x32 skinny kernel: waves per workgroup (2, 4; 0: by row tiles)
    int mamba_scan = 0;    // Mamba-2 prefill scan: 0 chunked (MFMA), 1 the token recurrence
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

// 2 <= M <= 16 on 4x4x4 MFMA with coalesced weight reads and x staged by LDS DMA; the GEMM takes
// the call where x rows are not 16-byte aligned or x spans 4 GiB or more.
hipError_t launch_skinny4_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                                  int ngroups, hipStream_t stream);

// M <= 16 on 16x16x32 MFMA, one row tile per workgroup with K split between its waves
// (skinny16_fp8.hip): taken for the M and K skinny16_wanted() accepts when the operands suit it
// (K % 64 == 0, 16-byte aligned x rows and weight rows).  launch_skinny16_grouped returns false,
// launching nothing, when the kernel cannot take the call; otherwise *err is the launch's status.
bool skinny16_wanted(int M, int K);
bool launch_skinny16_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups, int ngroups,
                             hipStream_t stream, hipError_t* err);
// Independent linears in one launch of the same kernel: matrix i (groups[i]) times its own
// activations xs[i] [M, Ks[i]] (row stride ldxs[i]); at most kS16MaxBatch of them.  Returns
// false, launching nothing, where the kernel cannot take every one of them.
constexpr int kS16MaxBatch = 8;
bool launch_skinny16_batch(const uint16_t* const* xs, const int64_t* ldxs, const int* Ks, const GemvGroup* groups,
                           int n, int M, hipStream_t stream, hipError_t* err);

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

// The M = 1 stream GEMV (gemv_stream.hip).  A phase is a grouped GEMV of one x [K] against up to
// kMaxGroups matrices; rows go 2 or 4 at a time ("row groups", numbered across all phases; 4 in
// chains, kStreamChainT), K in slices of at most 256 16-byte chunks.  Single launches carry one
// phase in the kernel arguments and stage x in LDS (K <= 16 * kStreamMaxLdsChunks); chains keep
// a table of phases in device memory and read x per step from global memory.
constexpr int kStreamChainT = 4;
constexpr int kStreamMaxLdsChunks = 2048;
struct StreamGroup {
    const uint8_t* W;
    int64_t ldw;
    const float* s;
    uint16_t* y;
    const uint16_t* res;    // residual [N] (epi == kEpiResidual)
    int N;
    int rg_begin;           // first row group of the group within its phase
    int epi;                // kEpiNone / kEpiRelu2 / kEpiResidual
    int ldy;                // elements between output rows (two activation rows)
    int ldres;              // elements between residual rows (two activation rows)
    int pad;
};
static_assert(sizeof(StreamGroup) == 64, "64-byte group record");
struct StreamPhase {
    const uint16_t* x;
    int K;
    int C;                  // chunks (K / 16)
    int S;                  // slices
    int sw;                 // chunks per slice (the last slice may be shorter)
    int ngroups;
    int g_begin, g_end;     // row groups of the phase, numbered across its launch
    StreamGroup g[kMaxGroups];
};
struct StreamArgs {
    StreamPhase one;            // single launches
    const StreamPhase* tab;     // chains: the launch's phases
    const int* wave_steps;      // chains: steps of each wave of the grid
    const float* norm_w;        // single launches: fused RMSNorm weight (nullptr: none)
    float eps;
    int nphases;
    int total_rg;
    int xs_half;                // LDS chunks per x half (single launches)
    int64_t ldx;                // elements between activation rows (single launches, M > 1)
    int M;                      // activation rows (single launches)
};
// Single launch (one phase) on the stream kernel for M = 1 or 2 activation rows (x row stride
// ldx); norm.w applies the RMSNorm to x while staging.
bool gemv_stream_supported(int M, int K, bool norm);
hipError_t launch_gemv_stream(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups, int ngroups,
                              hipStream_t stream, const Norm& norm = Norm{});
// Chains: one launch per run of phases up to the next phase that waits for its predecessor.
// stream_chain_plan fills the slices and row groups of a run's phases and returns its row
// groups; stream_chain_grid sizes its grid (at most 2 workgroups per CU, or tuning knob
// chain.wgs); stream_chain_wave_steps gives each of its nw waves' step counts.
int stream_chain_plan(StreamPhase* phases, int nphases);
void stream_chain_wave_steps(const StreamPhase* phases, int nphases, int nw, int* out);
hipError_t stream_chain_grid(int total_rg, int* grid);
hipError_t launch_gemv_stream_chain(const StreamPhase* tab, const int* wave_steps, int nphases, int total_rg, int grid,
                                    hipStream_t stream);

// Prefill GEMM.  Given a workspace of at least gemm_workspace_bytes(M) bytes whose first 64 KiB
// (the flag region) are zero -- every launch leaves them zero again -- the DMA-fed kernel splits
// the k tiles of all tiles evenly between the CUs (stream-K) when the tiles cover at most half
// of them (tuning knob gemm.sk = 1: always, also for the 8-wave kernels; 2: never); otherwise
// one tile per workgroup.  launch_sk_flags_clear zeroes the flag region (one small kernel, safe
// under graph capture).
size_t gemm_workspace_bytes(int M);
// Short prompts (17 <= M < 512; gemm_short.hip): the pipelined 128-row-tile kernel, with K split
// between workgroups when a workspace of gemm_short_workspace_bytes(M, N, K) bytes is given
// (float32 partials, no initialisation needed; 0: the schedule does not split).
bool gemm_short_supported(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, int M, int N, int K);
int gemm_short_splits(int M, int N, int K);
size_t gemm_short_workspace_bytes(int M, int N, int K);
// Workspace bytes a linear of M rows over matrices of total_n rows and K columns can use
// (nmi_linear_workspace_bytes); whether that region holds stream-K flags that must start at zero
// (launch_sk_flags_clear) -- the short-prompt kernel's partials need no initialisation.
size_t linear_workspace_bytes(int M, int64_t total_n, int K);
bool gemm_workspace_has_flags(int M);
// The fp8 MLP block (block.cpp) behind nmi_mlp_forward_fp8 (split = true) and its allocation-free
// form (split = false: the short-prompt GEMMs run unsplit, so the workspace has no partial
// region); fn names the entry point in error messages.
size_t mlp_workspace_bytes(int M, int hidden, int inter, bool split);
int mlp_forward_fp8(const void* input_bf16, const float* norm_w, const void* up_w_e4m3, const float* up_scale,
                    const void* down_w_e4m3, const float* down_scale, void* out_bf16, int M, int hidden, int inter,
                    float eps, void* workspace, size_t workspace_bytes, void* stream, bool split, const char* fn);
hipError_t launch_gemm_short(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, const float* s,
                             uint16_t* y, int64_t ldy, int M, int N, int K, hipStream_t stream, const Epi& epi,
                             void* ws, size_t ws_bytes);
// Attention decode (sdpa_decode.hip): q [H, 128] against the caches [H_KV, cap, 128] over
// positions [0, S), then K_new / V_new appended at position S; H / H_KV in 1..kSdpaMaxGroup.
// The workspace (sdpa_decode_workspace_bytes) holds the fp32 partials of split launches.
constexpr int kSdpaHead = 128;
constexpr int kSdpaMaxGroup = 6;
constexpr int kSdpaMinChunk = 64;
constexpr int kSdpaMaxSplits = 256;
void sdpa_decode_plan(int S, int n_kv, int* nsplit, int* chunk);
size_t sdpa_decode_workspace_bytes(int n_heads, int S, int n_kv);
hipError_t launch_sdpa_decode(const uint16_t* q, uint16_t* k_cache, uint16_t* v_cache, const uint16_t* k_new,
                              const uint16_t* v_new, uint16_t* o, int S, int cap, int n_heads, int n_kv,
                              void* workspace, hipStream_t stream);

// Mamba-2 mixer at decode (mamba_decode.hip): conv1d step + SiLU, SSM state update and
// output, gated RMSNorm, for `batch` sequences of one token.  Shapes: H heads of P, G groups,
// state size kMambaDState, conv width kMambaConvK (mamba_decode_supported).
constexpr int kMambaDState = 128;
constexpr int kMambaConvK = 4;
struct MambaDecodeArgs {
    const uint16_t* proj;   // [batch, proj_ld] bf16: z [inter] | xBC [conv_dim] | dt [H]
    int64_t proj_ld;
    const float* conv_w;    // [conv_dim, 4]
    const float* conv_b;    // [conv_dim]
    const float* A_log;     // [H]
    const float* D;         // [H]
    const float* dt_bias;   // [H]
    const float* gnorm_w;   // [inter]
    float* conv_state;      // [batch, conv_dim, 3]
    float* ssm_state;       // [batch, H, P, 128]
    uint16_t* y;            // [batch, inter] bf16: SSM output
    uint16_t* g;            // [batch, inter] bf16: gated-norm output (out_proj's input)
    int H, P, G, inter, conv_dim;
    float eps;
    int bc_state;           // 1: the gated-norm kernel also shifts the B and C conv states (decode)
};
bool mamba_decode_supported(int H, int P, int G, int d_state, int conv_k);
hipError_t launch_mamba_decode_mixer(const MambaDecodeArgs& a, int batch, hipStream_t stream);
// The gated RMSNorm alone over `rows` rows of y and z (a.proj, row stride a.proj_ld).
hipError_t launch_mamba_gated_norm(const MambaDecodeArgs& a, int rows, hipStream_t stream);

// Mamba-2 mixer over prompts (mamba_prefill.hip): the causal conv1d + SiLU over each sequence
// of S tokens, then the SSM scan from a zero state; the final states when the pointers are set.
struct MambaPrefillArgs {
    const uint16_t* proj;   // [batch * S, proj_ld] bf16: z | xBC | dt
    int64_t proj_ld;
    uint16_t* xc;           // [batch * S, xc_ld] bf16: conv outputs x | B | C
    int64_t xc_ld;
    const float* conv_w;    // [conv_dim, 4]
    const float* conv_b;
    const float* A_log;
    const float* D;
    const float* dt_bias;
    float* conv_state;      // [batch, conv_dim, 3] or nullptr
    float* ssm_state;       // [batch, H, P, 128] or nullptr
    uint16_t* y;            // [batch * S, y_ld] bf16
    int64_t y_ld;
    int S, H, P, G, inter, conv_dim;
    int x_vec, y_vec;       // 16-byte x reads / y stores possible (row strides and P multiples of 8)
};
hipError_t launch_mamba_prefill_mixer(const MambaPrefillArgs& a, int batch, hipStream_t stream);

// Causal attention over a prompt (sdpa_prefill.hip), token-major q [S, ldq], k [S, ldk], v
// [S, ldv], o [S, ldo] (head h at column 128 h); one launch, no workspace.  launch_kv_cache fills the
// KV caches [H_KV, cap, 128] positions [0, S) from k and v.
hipError_t launch_kv_cache(const uint16_t* k, int64_t ldk, const uint16_t* v, int64_t ldv, int S, int H_KV,
                           uint16_t* k_cache, uint16_t* v_cache, int cap, hipStream_t stream);
hipError_t launch_sdpa_prefill(const uint16_t* q, int64_t ldq, const uint16_t* k, int64_t ldk, const uint16_t* v,
                               int64_t ldv, uint16_t* o, int64_t ldo, int S, int H, int H_KV, hipStream_t stream);

hipError_t launch_sk_flags_clear(void* ws, hipStream_t stream);
// Several matrices sharing x: one launch of the DMA-fed kernel where it takes them all (M >= 512),
// else launch_gemm per matrix.
hipError_t launch_gemm_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* g, int ng,
                               hipStream_t stream, void* ws, size_t ws_bytes);
hipError_t launch_gemm(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw,
                       const float* s, uint16_t* y, int64_t ldy, int M, int N, int K,
                       hipStream_t stream, const Epi& epi = Epi{}, void* ws = nullptr, size_t ws_bytes = 0);

hipError_t launch_decode(const uint8_t* codes, float* out_f32, float* out_scaled,
                         uint16_t* out_bf16, float scale, int n, hipStream_t stream);

// Kernel chosen for a linear with M activation rows (tuning knobs may override).
enum class Path { Gemv, Skinny4, Gemm };
Path choose_path(int M);
// Whether a block runs the RMSNorm inside its first projection (the GEMV kernel staging x, M <= 2)
// rather than as its own launch: where the GEMV kernel takes that projection and supports the
// fused form; at M = 2 only where the 16x16x32 skinny kernel would not take the projection, so
// that a block's projections always run on the kernels the separate linear calls use.
bool gemv_fuses_norm(int M, int K);

// One or more linears sharing x [M, K] on the kernel choose_path(M) names (GEMM: one launch per
// matrix).  norm (GEMV path only, where gemv_norm_supported) applies the RMSNorm to x first.
hipError_t dispatch_linear(const uint16_t* x, int64_t ldx, int M, int K, GemvGroup* g, int ng, void* ws,
                           size_t ws_bytes, hipStream_t stream, const Norm& norm = Norm{});

}  // namespace nmi
