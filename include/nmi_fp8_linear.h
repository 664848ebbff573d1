/*
 * nmi_fp8_linear.h -- C ABI of the MI355X (gfx950) fp8 W8A16 linear library (libnmi.so).
 *
 * The library computes, for bf16 activations x [M,K], OCP e4m3 weights W [N,K] and per-row
 * float32 scales s [N]:
 *
 *     y[m,n] = bf16_rne( (sum_k float(W[n,k]) * float(x[m,k])) * s[n] )     y: [M,N] bf16
 *
 * with float32 accumulation and a single bf16 rounding.  All pointers are device pointers
 * (hipMalloc / torch CUDA tensors) unless stated otherwise.  `stream` is a hipStream_t passed
 * as void* (NULL = the null stream).  No entry point allocates device memory (except nmi_alloc,
 * and the block and SDPA entries called without a workspace), synchronizes the device (except
 * nmi_sync), or retains pointers after it returns; launches are asynchronous on `stream`.
 *
 * Return value: NMI_OK (0) on success; a negative NMI_ERR_* for argument errors detected on
 * the host before anything is launched; a positive hipError_t value when a HIP call fails.
 * nmi_last_error() describes the last failure of the calling thread.
 * NMI_ERR_ASYNC reports a failure of an earlier launch on the device that the host learnt of
 * since (a stream-K GEMM that gave up waiting for a partial tile, see nmi_linear_fp8_w8a16_ws):
 * every entry point that launches a linear, a GEMM or a block returns it, launching nothing, at
 * its first call after that launch has finished; nmi_sync after synchronising, nmi_async_status
 * without synchronising.  Each such failure is reported once.
 *
 * Layouts: x row m starts at x + m*ldx elements; W row n at W + n*ldw bytes; y row m at
 * y + m*ldy elements.  Row-sliced calls pass offset pointers (W + r0*ldw, s + r0, y + r0)
 * with ldy of the full output, as nemotron_infer's mamba block does for in_proj
 * (csrc/include/model/mamba_block.cuh:386-391, 476-481).
 *
 * Requirements checked on every call (NMI_ERR_INVALID_ARG / NMI_ERR_ALIGNMENT otherwise):
 *   M >= 1, N >= 1, K >= 16, K % 16 == 0, ldx >= K, ldw >= K, ldy >= N,
 *   W and ldw 16-byte aligned, x and ldx*2 16-byte aligned, s 4-byte aligned,
 *   y 2-byte aligned, no NULL pointers.
 * The reference silently assumes K % 16 == 0 (ops/gemv.cuh:61-63 casts every row to uint4);
 * this ABI rejects other K instead.
 */
#ifndef NMI_FP8_LINEAR_H
#define NMI_FP8_LINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NMI_OK = 0,
    NMI_ERR_INVALID_ARG = -1,
    NMI_ERR_ALIGNMENT = -2,
    NMI_ERR_UNSUPPORTED = -3,
    NMI_ERR_WORKSPACE = -4,
    NMI_ERR_ALLOC = -5,
    NMI_ERR_ASYNC = -6,
};

/* Version of this ABI (major*10000 + minor*100 + patch). */
int nmi_abi_version(void);

/* Human-readable description of the calling thread's last error ("" if none). */
const char* nmi_last_error(void);

/*
 * M = 1 decode GEMV: y[n] = bf16_rne((sum_k e4m3(W[n,k]) * x[k]) * s[n]).
 * Replaces nemotron::ops::gemv_fp8(x, W, w_scale, y, N, K, stream)
 * (nemotron_infer/csrc/include/ops/gemv.cuh:92-104); same argument meaning, plus a status.
 * x: [K] bf16, W: [N,K] e4m3 with row stride K, s: [N] f32, y: [N] bf16.
 */
int nmi_gemv_fp8(const void* x_bf16, const void* w_e4m3, const float* w_scale, void* y_bf16,
                 int N, int K, void* stream);

/*
 * General W8A16 linear with explicit strides and an M dispatch that refines the
 * reference's M == 1 switch: M == 1 -> the GEMV kernel, 2 <= M <= 16 -> the skinny kernels
 * (weight-streaming on bf16 MFMA: 16x16x32 with both operands brought into LDS by DMA; where K
 * is not a multiple of 64 or x / W are not 16-byte aligned, the GEMV kernel at M = 2 (one pass
 * over W for both activation rows) and the 4x4x4 kernel above), M > 16 -> the MFMA GEMM.  Replaces the fp8 branch of mlp_block_forward_fp8
 * (nemotron_infer/csrc/include/model/mlp_block.cuh:142-171) and the per-projection calls
 * in attention_block.cuh:330-350,400-409 and mamba_block.cuh:383-391,419-423,476-481,508-509.
 * Unlike the reference's M > 1 branch, activations are NOT quantized to e4m3
 * (ops/gemm.cuh:257-307 is not reproduced): the product is computed on bf16 activations.
 */
int nmi_linear_fp8_w8a16(const void* x_bf16, int64_t ldx, const void* w_e4m3, int64_t ldw,
                         const float* w_scale, void* y_bf16, int64_t ldy, int M, int N, int K,
                         void* stream);

/*
 * As nmi_linear_fp8_w8a16, with a caller-owned device workspace that lets the short-prompt
 * GEMM (17 <= M < 512) split K between workgroups.  For M >= 512 the prefill GEMM needs none:
 * where its 256 x 256 tiles would cover at most half of the CUs (e.g. N = 3136 at M = 2048) it
 * takes 128 x 256 tiles instead.  Its stream-K form (the k tiles of a few large tiles split
 * between all CUs: fp32 partial tiles and per-workgroup flags in the workspace) runs only under
 * the tuning knob gemm.sk = 1 (or gemm.bm = 256), and nmi_linear_workspace_bytes sizes the
 * workspace for it only then.
 * workspace: 256-byte aligned, at least nmi_linear_workspace_bytes(M, N, K) bytes, zero-filled
 * before its first use; every launch leaves it ready for the next one.  NULL / too small ->
 * the kernels run without the split (same results up to float32 summation order).  Two
 * launches that may run concurrently must not share a workspace.  The reference's blocks
 * likewise hand a workspace to their prefill GEMMs (model/mlp_block.cuh:133,156,160-161).
 * Stream-K ordering: a contributor stores its partial tile, then releases its flag at device
 * scope; the finisher polls the flag and acquires at device scope before reading the partial.
 * The wait is bounded: if a flag does not come in time (a workgroup that is stalled or never
 * ran), the finisher gives up, leaves that partial out, marks the slot abandoned and sets the
 * 32-bit error word at byte NMI_WS_ERROR_OFFSET of the workspace to 1 and the device's
 * asynchronous error (NMI_ERR_ASYNC, returned by the next call).  The results of that launch are
 * wrong; the flags still end it at zero (a contributor that finds its slot abandoned lowers its
 * flag again), so the workspace needs no reset and the next launch on it is correct.  The error
 * word stays set until the workspace is zero-filled.
 */
#define NMI_WS_ERROR_OFFSET 65532
int nmi_linear_fp8_w8a16_ws(const void* x_bf16, int64_t ldx, const void* w_e4m3, int64_t ldw,
                            const float* w_scale, void* y_bf16, int64_t ldy, int M, int N, int K,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Several weight matrices that share the activation x [M, K] in one dispatch (one kernel
 * launch for M <= 16): q/k/v of an attention block, which the reference runs as three GEMVs
 * on the same normed input (model/attention_block.cuh:400-402, 332-337), or the row slices of
 * a Mamba in_proj (model/mamba_block.cuh:476-481, 386-391).  Group i computes
 * y_i[M, N_i] = bf16((x . e4m3(W_i)^T) * s_i); each group is validated like
 * nmi_linear_fp8_w8a16.  Workspace as for nmi_linear_fp8_w8a16_ws, sized for the sum of N_i.
 */
#define NMI_MAX_GROUPS 4
typedef struct nmi_linear_group {
    const void* w_e4m3;   /* [N, K] e4m3, row stride ldw bytes */
    int64_t ldw;
    const float* w_scale; /* [N] */
    void* y_bf16;         /* [M, N] bf16, row stride ldy elements */
    int64_t ldy;
    int N;
} nmi_linear_group;
int nmi_linear_fp8_w8a16_grouped(const void* x_bf16, int64_t ldx, int M, int K,
                                 const nmi_linear_group* groups, int ngroups, void* workspace,
                                 size_t workspace_bytes, void* stream);

/*
 * Independent linears in one dispatch: job i computes y_i[M, N_i] = bf16((x_i . e4m3(W_i)^T) * s_i)
 * with its own activations x_i [M, K_i] -- a set of projections whose inputs are all ready (the
 * decode shapes with an independent activation row per sequence).  No counterpart in the reference, which launches one
 * GEMV or GEMM per projection (ops/gemv.cuh:92-104, ops/gemm.cuh:325-337); it is the skinny-M
 * sibling of the GEMV chain below.  For 2 <= M <= 16, when the 16x16x32 skinny kernel takes
 * every job (K_i % 64 == 0, 16-byte aligned x_i rows and W_i rows), the jobs run as one kernel
 * launch (one row tile per workgroup over all of the jobs' rows, the jobs of largest K_i first:
 * their tiles take longest, so they start in the first round); otherwise each job runs as
 * nmi_linear_fp8_w8a16 (no workspace) would run it, one after another.  Every output is the one
 * a separate call with the same kernel schedule gives.  Each job is validated like
 * nmi_linear_fp8_w8a16; 1 <= njobs <= NMI_MAX_BATCH.
 */
#define NMI_MAX_BATCH 8
typedef struct nmi_linear_job {
    const void* x_bf16;   /* [M, K] bf16, row stride ldx elements */
    int64_t ldx;
    int K;
    nmi_linear_group w;   /* the matrix, its scales and the output */
} nmi_linear_job;
int nmi_linear_fp8_w8a16_batch(const nmi_linear_job* jobs, int njobs, int M, void* stream);

/*
 * GEMV chain (M = 1): a sequence of GEMVs with as few launches as the dependencies allow.  A
 * chain is a list of phases, each a grouped GEMV of one activation vector x [K] (bf16) against
 * up to NMI_MAX_GROUPS e4m3 matrices, computed exactly as nmi_linear_fp8_w8a16(_grouped) computes
 * it at M = 1 (the same per-row results, bit for bit).  Phases with wait_prev = 0 (x ready before
 * the launch) stream back to back in one kernel launch; a phase with wait_prev = 1 reads its x
 * only after the previous phase has completed, so x may be that phase's output: it starts a new
 * launch on the same stream (stream order is the synchronisation).  Replaces a sequence of
 * per-projection gemv_fp8 launches (ops/gemv.cuh:92-104 at model/attention_block.cuh:400-402,409,
 * model/mlp_block.cuh:142-148, model/mamba_block.cuh:476-481,508-509); the reference has no
 * chained form.
 *   nmi_gemv_chain_create   validates the phases as nmi_linear_fp8_w8a16_grouped would (M = 1),
 *                           plans the work split and the grids for the current device and copies
 *                           the plan to device memory (hipMalloc + hipMemcpy: call it outside
 *                           graph capture, once per set of pointers).
 *   nmi_gemv_chain_launch   one kernel launch per run of phases up to the next waiting phase,
 *                           asynchronous on `stream`; capturable in a HIP graph.  workspace /
 *                           workspace_bytes are accepted for compatibility and never accessed
 *                           (NULL / 0 is fine).
 *   nmi_gemv_chain_destroy  frees the plan.
 * Buffers: a phase's output may overlap another phase's x or output only when a waiting phase
 * lies between the two (phases of one launch may run at the same time).
 */
#define NMI_MAX_CHAIN_PHASES 4096
typedef struct nmi_gemv_phase {
    const void* x_bf16;   /* [K] bf16 */
    int K;
    int ngroups;
    int wait_prev;        /* 1: read x only after the previous phase has completed */
    nmi_linear_group groups[NMI_MAX_GROUPS];
} nmi_gemv_phase;
typedef struct nmi_gemv_chain nmi_gemv_chain;
int nmi_gemv_chain_create(const nmi_gemv_phase* phases, int nphases, nmi_gemv_chain** out);
size_t nmi_gemv_chain_workspace_bytes(int nphases);     /* 0: no launch writes a workspace */
int nmi_gemv_chain_launch(const nmi_gemv_chain* chain, void* workspace, size_t workspace_bytes, void* stream);
int nmi_gemv_chain_destroy(nmi_gemv_chain* chain);

/* Workspace bytes the kernels can use for M rows, total_n output rows (the sum over groups)
 * and K on the current device; 0 when the selected kernel needs none (the GEMV, the skinny
 * kernels by default, which split K inside the workgroup only).  With the 4x4x4 kernel's K
 * split (s4.kg > 1): 64 KiB of arrival counters and the fp32 partials, s4.kg x M x total_n x 4
 * bytes (fewer K groups when K has fewer windows).  For 17 <= M < 512 (the short-prompt GEMM) a
 * 64 KiB region it leaves alone, then the fp32 partials of its K split (0 when the schedule does
 * not split K).  For M >= 512 about 64 MiB: a 64 KiB flag region and one 256 x 256 fp32 partial
 * tile per CU.  Every kernel leaves the first 64 KiB as it found it (zero at rest), so one
 * zero-filled workspace serves every M in turn. */
size_t nmi_linear_workspace_bytes(int M, int64_t total_n, int K);

/*
 * Prefill GEMM y[M,N] = bf16_rne((x[M,K] . e4m3(W[N,K])^T) * s[n]) on bf16 MFMA, any M >= 1.
 * Replaces nemotron::ops::gemm_fp8(x_fp8, W_fp8, y_bf16, x_scale, w_scale, M, N, K, ws,
 * ws_size, stream) (nemotron_infer/csrc/include/ops/gemm.cuh:325-403) including its
 * per-row scale epilogue (gemm.cuh:227-238, 398-402), which here is fused and rounds once.
 * x is bf16 (no activation scale); `workspace`/`workspace_bytes` as for
 * nmi_linear_fp8_w8a16_ws (NULL/0: every tile in one workgroup, no stream-K).
 */
int nmi_gemm_fp8_w8a16(const void* x_bf16, int64_t ldx, const void* w_e4m3, int64_t ldw,
                       const float* w_scale, void* y_bf16, int64_t ldy, int M, int N, int K,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * Device-side e4m3 decode of `n` codes through the kernels' own conversion helper (e4m3 ->
 * bf16, exact; every GEMV and MFMA kernel decodes weights this way): out_bf16[i] =
 * bf16(e4m3(codes[i])), out_f32[i] = that value widened to float (exact), out_scaled[i] =
 * out_f32[i] * scale (f32 RNE product, as in the reference's GEMV epilogue).  Test entry point for the 256-code bit-exact check; mirrors
 * static_cast<float>(__nv_fp8_e4m3) (ops/gemv.cuh:40-42) and the per-row scale product of
 * the epilogue (ops/gemv.cuh:87-88).  n must be a positive multiple of 4; codes 4-byte,
 * out_f32/out_scaled 16-byte and out_bf16 8-byte aligned.
 */
int nmi_fp8_e4m3_decode(const void* codes, float* out_f32, float* out_scaled, void* out_bf16,
                        float scale, int n, void* stream);

/*
 * RMSNorm of M rows of bf16 activations; replaces rmsnorm_bf16(in0, out0, weight, rows, cols,
 * eps, stream) (nemotron_infer/csrc/include/ops/reduce.cuh:229-244) and the binding's
 * rmsnorm(in, out, w, M) (csrc/include/binding.cu:71-73: cols = HIDDEN, eps = 1e-5):
 *     y[m,k] = bf16_rne(x[m,k] * (r_m * w[k])),   r_m = 1 / sqrt(sum_k x[m,k]^2 / K + eps)
 * with a float32 sum of squares in a fixed order (the reference reduces in its own order and
 * uses rsqrtf; results agree up to rare last-bit differences).  x, y: [M, K] contiguous bf16;
 * w: [K] float32.  Requires M >= 1, K >= 8, K % 8 == 0, x, y and w 16-byte aligned.
 */
int nmi_rmsnorm_bf16(const void* x_bf16, const float* w, void* y_bf16, int M, int K, float eps, void* stream);

/*
 * The fp8 MLP block; replaces mlp_block_forward_fp8<HIDDEN, INTER>(input, w, out, M, stream)
 * (nemotron_infer/csrc/include/model/mlp_block.cuh:121-176) and the binding's
 * mlp_forward_fp8(input, block_norm_w, up_w, up_s, down_w, down_s, out, M)
 * (csrc/include/binding.cu:201-208: hidden = 3136, inter = 12544, eps = 1e-5):
 *     h   = rmsnorm(input)                                      [M, hidden]  bf16
 *     act = bf16_rne(relu(bf16_rne((h . W_up^T) * up_s))^2)      [M, inter]   bf16
 *     out = bf16_rne(input + bf16_rne((act . W_down^T) * down_s)) [M, hidden]  bf16
 * input, out: [M, hidden] contiguous bf16 (out may be input); norm_w [hidden] float32;
 * up_w [inter, hidden] e4m3 and up_s [inter]; down_w [hidden, inter] e4m3 and down_s [hidden].
 * The projections are W8A16 for every M: the reference quantizes prefill activations to e4m3
 * (mlp_block.cuh:151-171), this library keeps them bf16.  M <= 2 takes two launches (the
 * RMSNorm applied while the up projection stages its activations, relu^2 and the residual add
 * in the projections' stores), larger M three (a separate RMSNorm).
 * workspace: nmi_mlp_workspace_bytes(M, hidden, inter) bytes, 16-byte aligned, no
 * initialisation needed (for 17 <= M < 512 it includes the short-prompt GEMMs' K-split partials;
 * from M = 512 the GEMMs' stream-K region, whose flags each call zeroes with one small kernel);
 * calls that may overlap in time need distinct workspaces.  NULL
 * takes it from the bump allocator (nmi_alloc, so a slab may be hipMalloc'd), valid until
 * nmi_alloc_rewind(), as the reference's blocks do (binding.cu:7-9).
 * Requires M >= 1, hidden and inter positive multiples of 16, input, norm_w and both weights
 * 16-byte aligned, scales 4-byte aligned, out 2-byte aligned.
 */
size_t nmi_mlp_workspace_bytes(int M, int hidden, int inter);
int nmi_mlp_forward_fp8(const void* input_bf16, const float* norm_w, const void* up_w_e4m3, const float* up_scale,
                        const void* down_w_e4m3, const float* down_scale, void* out_bf16, int M, int hidden,
                        int inter, float eps, void* workspace, size_t workspace_bytes, void* stream);

/*
 * nmi_mlp_forward_fp8 without any allocation: the same block, with the transient buffers in a
 * file-scope device array of nmi_mlp_noalloc_scratch_bytes() bytes (4 MiB) that each GPU the
 * library runs on holds until the process ends.  No counterpart in the reference: for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Calls no hipMalloc / hipFree.  The result equals nmi_mlp_forward_fp8's bit for
 * bit for M <= 16; for 17 <= M the short-prompt GEMMs run without their K split (whose partials
 * would not fit), so the two agree up to float32 summation order (bit for bit with tuning knob
 * gemm.splits = 1).  Needs the block's buffers without the split partials (M * inter * 2 bytes,
 * plus M * hidden * 2 for the normed input unless the RMSNorm is fused into the up projection's
 * GEMV -- M = 1, or M = 2 where hidden is not a multiple of 64 -- each rounded up to 256; this is
 * nmi_mlp_workspace_bytes under tuning knob gemm.splits = 1) within the array (hidden 3136, inter
 * 12544: M <= 133), else NMI_ERR_WORKSPACE.  Every call on a GPU shares that GPU's array: calls that
 * may overlap in time on one GPU (other streams, other threads) race.  Same argument
 * requirements as nmi_mlp_forward_fp8.
 */
size_t nmi_mlp_noalloc_scratch_bytes(void);
int nmi_mlp_forward_fp8_noalloc(const void* input_bf16, const float* norm_w, const void* up_w_e4m3,
                                const float* up_scale, const void* down_w_e4m3, const float* down_scale,
                                void* out_bf16, int M, int hidden, int inter, float eps, void* stream);

/*
 * Attention decode, one query token per head against the KV cache
 * (replaces sdpa_decode_bf16<128>, nemotron_infer/csrc/include/ops/attention/
 * sdpa_decode.cuh:267-285, kernels :57-180):
 *   o[h] = bf16( softmax(q[h] . K[kv(h), 0:S_cache]^T / sqrt(128)) . V[kv(h), 0:S_cache] ),
 *   kv(h) = h / (n_heads / n_kv_heads), float32 arithmetic; then K[kv, S_cache] = k_new[kv] and
 *   V[kv, S_cache] = v_new[kv].  As in the reference the query attends the S_cache cached
 *   positions only (the new token's K/V are stored after), and S_cache == 0 gives o = 0.
 * q, o [n_heads, 128]; k_new, v_new [n_kv_heads, 128]; caches [n_kv_heads, cache_cap, 128],
 * all bf16.  Head dim 128; 1 <= n_heads / n_kv_heads <= 6; 0 <= S_cache < cache_cap.
 * workspace: nmi_sdpa_decode_workspace_bytes(n_heads, n_kv_heads, S_cache) bytes (0 when the
 * positions are not split; the fp32 partials otherwise), 16-byte aligned, no initialisation;
 * NULL takes it from the bump allocator.  q, the caches, k_new and v_new 16-byte aligned, o
 * 4-byte aligned.
 */
size_t nmi_sdpa_decode_workspace_bytes(int n_heads, int n_kv_heads, int S_cache);
int nmi_sdpa_decode_bf16(const void* q_bf16, void* k_cache_bf16, void* v_cache_bf16, void* o_bf16,
                         const void* k_new_bf16, const void* v_new_bf16, int S_cache, int cache_cap, int n_heads,
                         int n_kv_heads, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The fp8 attention block at decode (replaces attention_block_decode_fp8<HIDDEN, H_Q, H_KV, 128>,
 * nemotron_infer/csrc/include/model/attention_block.cuh:371-414; binding attn_decode_fp8,
 * csrc/include/binding.cu:189-199):
 *   h = rmsnorm(input) (bf16); q, k_new, v_new = bf16 linears of h (e4m3 weights, per-row
 *   scales); o = nmi_sdpa_decode_bf16(q, caches, k_new, v_new, S_cache); out = bf16(input +
 *   bf16(o . o_w^T * o_s)).  NoPE (no rotary), as the reference.  The caches receive this token's
 *   K/V at position S_cache.
 * input, out [1, hidden] bf16 (out may be input); q_w [n_heads*128, hidden], k_w and v_w
 * [n_kv_heads*128, hidden], o_w [hidden, n_heads*128] e4m3 with float32 scales of their row
 * counts.  Launches: the q|k|v GEMV (RMSNorm applied while staging), the SDPA kernel(s), the o
 * GEMV with the residual add in its stores.
 * workspace: nmi_attn_decode_workspace_bytes(hidden, n_heads, n_kv_heads, S_cache) bytes,
 * 16-byte aligned, no initialisation; NULL takes it from the bump allocator.
 */
size_t nmi_attn_decode_workspace_bytes(int hidden, int n_heads, int n_kv_heads, int S_cache);
int nmi_attn_decode_fp8(const void* input_bf16, const float* norm_w, const void* q_w_e4m3, const float* q_scale,
                        const void* k_w_e4m3, const float* k_scale, const void* v_w_e4m3, const float* v_scale,
                        const void* o_w_e4m3, const float* o_scale, void* k_cache_bf16, void* v_cache_bf16,
                        int S_cache, int cache_cap, void* out_bf16, int hidden, int n_heads, int n_kv_heads,
                        float eps, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Causal attention over a prompt (replaces sdpa_prefill_bf16<32, 128>,
 * nemotron_infer/csrc/include/ops/attention/sdpa_prefill.cuh:364-395, kernel :224-320):
 *   o[s, h] = bf16( softmax_{t <= s}(q[s, h] . k[t, kv(h)] / sqrt(128)) . v[t, kv(h)] ),
 *   kv(h) = h / (n_heads / n_kv_heads), float32 softmax and sums.
 * Token-major layouts (as the projections write them; the reference's kernel takes head-major
 * [H, S, 128] and its block transposes around it): q, o [S, >= n_heads*128] with head h at
 * column 128 h, k, v [S, >= n_kv_heads*128]; row strides ldq, ldk, ldv (multiples of 8) and ldo
 * (multiple of 4) in elements.  q, k, v 16-byte aligned, o 8-byte aligned.
 * No workspace: nmi_sdpa_prefill_workspace_bytes returns 0 and the workspace arguments are
 * ignored (kept so that callers written against a sized workspace need no change).  One launch.
 */
size_t nmi_sdpa_prefill_workspace_bytes(int n_kv_heads, int S);
int nmi_sdpa_prefill_bf16(const void* q_bf16, int64_t ldq, const void* k_bf16, int64_t ldk, const void* v_bf16,
                          int64_t ldv, void* o_bf16, int64_t ldo, int S, int n_heads, int n_kv_heads, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * The fp8 attention block over a prompt (replaces attention_block_forward_fp8<HIDDEN, H_Q, H_KV, 128>,
 * nemotron_infer/csrc/include/model/attention_block.cuh:289-366; binding attn_forward_fp8,
 * csrc/include/binding.cu:177-187):
 *   h = rmsnorm(input) [S, hidden] (bf16); q, k, v = bf16 linears of h; o = causal attention
 *   (nmi_sdpa_prefill_bf16); out = bf16(input + bf16(o . o_w^T * o_s)); when k_cache and v_cache
 *   are both non-NULL, positions [0, S) of the caches [n_kv_heads, cache_cap, 128]
 *   (cache_cap <= 0: S) receive k and v.  NoPE, as the reference.  The activations stay bf16
 *   into every linear (the reference quantizes them to e4m3 first, attention_block.cuh:330-350).
 * input, out [S, hidden] bf16 (out may be input); weights as nmi_attn_decode_fp8.
 * workspace: nmi_attn_forward_workspace_bytes(S, hidden, n_heads, n_kv_heads) bytes, 256-byte
 * aligned, no initialisation; NULL takes it from the bump allocator.
 */
size_t nmi_attn_forward_workspace_bytes(int S, int hidden, int n_heads, int n_kv_heads);
int nmi_attn_forward_fp8(const void* input_bf16, const float* norm_w, const void* q_w_e4m3, const float* q_scale,
                         const void* k_w_e4m3, const float* k_scale, const void* v_w_e4m3, const float* v_scale,
                         const void* o_w_e4m3, const float* o_scale, void* out_bf16, int S, void* k_cache_bf16,
                         void* v_cache_bf16, int cache_cap, int hidden, int n_heads, int n_kv_heads, float eps,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * The fp8 Mamba-2 block at decode, one token per sequence (replaces
 * mamba_block_decode_fp8<HIDDEN, H, P, N, G, 4>, nemotron_infer/csrc/include/model/
 * mamba_block.cuh:436-515; binding mamba_decode_fp8, csrc/include/binding.cu:162-175):
 *   h = rmsnorm(input) (bf16); proj = [z | xBC | dt] = in_proj(h) (bf16, one GEMV over all
 *   n_heads*head_dim + conv_dim + n_heads rows); the causal conv1d step with SiLU on xBC
 *   (conv_state [batch, conv_dim, 3] updated); the SSM step on x, B, C (ssm_state
 *   [batch, n_heads, head_dim, d_state] updated) giving y (bf16); the gated RMSNorm of y with
 *   gate z over n_groups groups (bf16); out = bf16(input + bf16(out_proj(...))).
 *   conv_dim = n_heads*head_dim + 2*n_groups*d_state; states float32, as the reference.
 * input, out [batch, hidden] bf16 (out may be input); in_proj_w [n_heads*head_dim + conv_dim +
 * n_heads, hidden] and out_proj_w [hidden, n_heads*head_dim] e4m3 with float32 per-row scales;
 * conv_w [conv_dim, 4], conv_b [conv_dim], A_log, D, dt_bias [n_heads], gnorm_w
 * [n_heads*head_dim] float32.  Supported: d_state 128, conv_k 4, n_groups dividing n_heads
 * with groups of at most 2048 values, head_dim <= 128.  The reference's GEMV path computes batch
 * row 0 only; this entry computes every row (the linears dispatch on M = batch).
 * workspace: nmi_mamba_decode_workspace_bytes(batch, hidden, n_heads, head_dim, n_groups,
 * d_state) bytes, 16-byte aligned, no initialisation; NULL takes it from the bump allocator.
 */
/*
 * The mixer of the Mamba-2 block at decode, between its projections (replaces the op calls
 * causal_conv1d_decode_bf16, ssm_decode_bf16 and rmsnorm_gated_bf16 of
 * mamba_block.cuh:476-509, kernels ops/mamba2/causal_conv1d.cuh:391-459,
 * ops/mamba2/ssm.cuh:46-130, ops/reduce.cuh:383-500): from proj = [z | xBC | dt]
 * ([batch, proj_ld] bf16, the in_proj output), the conv step (conv_state updated), the SSM step
 * (ssm_state updated) giving y [batch, n_heads*head_dim] bf16, and the gated RMSNorm of y with
 * gate z giving g [batch, n_heads*head_dim] bf16 (out_proj's input).  Same shapes and
 * requirements as nmi_mamba_decode_fp8; proj, y, g, conv_w, gnorm_w and ssm_state 16-byte
 * aligned, proj_ld a multiple of 8.  Two launches.
 */
int nmi_mamba_mixer_decode(const void* proj_bf16, int64_t proj_ld, const float* conv_w, const float* conv_b,
                           const float* A_log, const float* D, const float* dt_bias, const float* gnorm_w,
                           float* conv_state, float* ssm_state, void* y_bf16, void* g_bf16, int batch, int n_heads,
                           int head_dim, int n_groups, int d_state, int conv_k, float eps, void* stream);
size_t nmi_mamba_decode_workspace_bytes(int batch, int hidden, int n_heads, int head_dim, int n_groups,
                                        int d_state);
int nmi_mamba_decode_fp8(const void* input_bf16, const float* norm_w, const void* in_proj_w_e4m3,
                         const float* in_proj_scale, const float* conv_w, const float* conv_b, const float* A_log,
                         const float* D, const float* dt_bias, const float* gnorm_w, const void* out_proj_w_e4m3,
                         const float* out_proj_scale, float* conv_state, float* ssm_state, void* out_bf16, int batch,
                         int hidden, int n_heads, int head_dim, int n_groups, int d_state, int conv_k, float eps,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * The fp8 Mamba-2 block over prompts (replaces mamba_block_forward_fp8<HIDDEN, H, P, N, G, 4>,
 * nemotron_infer/csrc/include/model/mamba_block.cuh:346-425; binding mamba_forward_fp8,
 * csrc/include/binding.cu:147-160): input, out [batch * S, hidden] bf16 (batch sequences of S
 * tokens; out may be input).  h = rmsnorm(input); proj = in_proj(h); per sequence the causal
 * conv1d + SiLU from a zero state and the SSM scan from a zero state (the recurrence in float32,
 * where the reference runs the chunked form with TF32 products); the gated RMSNorm; out =
 * bf16(input + bf16(out_proj(...))).  When given, conv_state_out [batch, conv_dim, 3] and
 * ssm_state_out [batch, n_heads, head_dim, d_state] (float32) receive each sequence's final
 * states, for nmi_mamba_decode_fp8 to continue from.  Weights and supported shapes as
 * nmi_mamba_decode_fp8.
 * workspace: nmi_mamba_forward_workspace_bytes(batch, S, hidden, n_heads, head_dim, n_groups,
 * d_state) bytes, 256-byte aligned, no initialisation; NULL takes it from the bump allocator.
 */
size_t nmi_mamba_forward_workspace_bytes(int batch, int S, int hidden, int n_heads, int head_dim, int n_groups,
                                         int d_state);
int nmi_mamba_forward_fp8(const void* input_bf16, const float* norm_w, const void* in_proj_w_e4m3,
                          const float* in_proj_scale, const float* conv_w, const float* conv_b, const float* A_log,
                          const float* D, const float* dt_bias, const float* gnorm_w, const void* out_proj_w_e4m3,
                          const float* out_proj_scale, void* out_bf16, int batch, int S, float* conv_state_out,
                          float* ssm_state_out, int hidden, int n_heads, int head_dim, int n_groups, int d_state,
                          int conv_k, float eps, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Tuning knobs for sweeps ("gemv.ks", "gemv.t", "gemv.p", "gemv.xg": schedule of the multi-row
 * GEMV kernel (M = 2, or M = 1 with "gemv.multirow" = 1), "gemv.t" = 4 also 4 rows per step for
 * the M = 1 stream kernel, "gemv.wgs": its workgroups per CU (1, 2), "gemv.grid": its exact
 * workgroup count, "gemv.balance": 2 keeps the plain grid instead of one whose waves get equal
 * row counts, "sdpa.chunk": cache positions per workgroup of the attention decode, "gemm.tile"
 * (1, 2: short-prompt kernel, 20, 21, 24), "gemm.sk", "gemm.splits": workgroups splitting K in
 * the short-prompt GEMM (1: none), "gemm.short": f + 1 forces its tile form f (0..7),
 * "gemm.sk_cap": workgroups per tile of the stream-K form at most (0: 2, -1: one workgroup per
 * CU), "skinny.path" (2: the skinny kernels take M = 2 too, 3: the GEMV kernel takes M <= 4),
 * "m1.path" (3: M = 1 on the 4x4x4 skinny kernel), "s4.ks", "s4.t", "s4.u",
 * "s4.dma": 2 selects the windowed form of the 4x4x4 skinny kernel instead of the pipelined one,
 * "s4.kg": K groups split between workgroups by the pipelined form (> 1; needs the workspace
 * nmi_linear_workspace_bytes then reports), "s16": the 16x16x32 skinny kernel (0: automatic, from
 * M = 3, 1: for 2 <= M <= 16, 2: never), "s16.r": its row tiles of 16 (1) or 32 (2), "s16.w": its
 * waves per workgroup (2, 4), "s16.t": 1 its row-run form instead of the DMA form, "chain.wgs":
 * workgroups per CU of a GEMV chain created afterwards); 0 restores the automatic choice.
 * Process-wide, not thread-safe against concurrent launches; results do not depend on them
 * beyond float32 summation order.  No counterpart in the
 * reference (its launch shapes are compile-time constants, ops/gemv.cuh:100-103).
 */
int nmi_tuning_set(const char* knob, int value);

/*
 * Bump allocator for transient per-block device workspace, on hipMalloc slabs.
 * Replaces nemotron::BumpAllocator / default_allocator()
 * (nemotron_infer/csrc/include/tensor/allocator.cuh:58-183) and the binding's
 * reset_allocator()/free_allocator() (csrc/include/binding.cu:59-61).
 *   nmi_alloc(bytes, &ptr)  128-byte aligned block from the current slab; a new slab
 *                           (>= 64 MiB) is hipMalloc'd only when none fits.
 *   nmi_alloc_rewind()      offset back to slab 0, slabs kept (no hipMalloc/hipFree).
 *   nmi_alloc_reset()       hipFree every slab.
 *   nmi_alloc_stats(&total_allocated, &num_slabs)   either pointer may be NULL.
 * Thread-safe (one mutex); one process-global allocator per process, as in the reference.
 */
int nmi_alloc(size_t bytes, void** out_ptr);
int nmi_alloc_rewind(void);
int nmi_alloc_reset(void);
int nmi_alloc_stats(size_t* total_allocated, size_t* num_slabs);

/* hipDeviceSynchronize(); replaces the binding's sync() (csrc/include/binding.cu:62).  Returns
 * NMI_ERR_ASYNC if a launch that finished had an asynchronous error not yet reported. */
int nmi_sync(void);

/*
 * The current device's asynchronous error, read and cleared without synchronising the GPU:
 * NMI_ERR_ASYNC (with nmi_last_error()) if a launch that has finished had one not yet reported,
 * else NMI_OK.  No counterpart in the reference, which checks no kernel for errors.
 */
int nmi_async_status(void);

#ifdef __cplusplus
}
#endif

#endif /* NMI_FP8_LINEAR_H */
