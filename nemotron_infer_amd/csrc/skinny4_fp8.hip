// skinny4_fp8.hip -- fp8 (OCP e4m3) W8A16 linear for 2 <= M <= 16 on 4x4x4 bf16 MFMA (gfx950).
//
//   y[m,n] = bf16_rne( (sum_k float(W[n,k]) * float(x[m,k])) * s[n] )
//
// The crossover between the reference's M == 1 GEMV (ops/gemv.cuh:48-104) and its prefill
// GEMM (ops/gemm.cuh:325-403, reached for every M > 1 at model/mlp_block.cuh:149-171).  For
// M <= 16 the work is bound by streaming W from HBM (<= 31.5 flop/B), so the kernel keeps the
// coalesced weight-read pattern of the GEMV and moves the products onto the matrix cores:
//
// * v_mfma_f32_4x4x4_16b_bf16 computes 16 independent 4x4x4 blocks; block b is lanes
//   4b..4b+3, A row i comes from lane 4b+i, B column j from lane 4b+j, element e of each is
//   k = e, and D[i][j] lands in register i of lane 4b+j (measured on gfx950).
// * A wave owns 4 weight rows per row group.  Lane 4b+i loads 16 bytes (16 codes) of row i
//   at chunk c0 + b + 16u, so one load instruction fetches 4 rows x 256 contiguous bytes.
//   The codes become bf16 in registers (v_cvt_scalef32_pk_bf16_fp8, exact) and feed four
//   MFMAs (k groups of 4) per group of 4 activation rows: lane 4b+j supplies x[4g+j] for the
//   same 16 k, read from LDS, so every MFMA output is useful (4 weight rows x 4 activation
//   rows).  T row groups per wave reuse the same activation registers.
// * The 16 blocks hold partial sums over different chunks; they are added across lanes at
//   the end (xor 4, 8, 16, 32, a fixed order), KS waves of a workgroup split K and their
//   partials are summed in order through LDS, then the per-row scale and one bf16 rounding.
// * Two forms stage x [M, window] per workgroup in LDS:
//   - pipelined (skinny4_dma_kernel, the default): windows of exactly one batch per wave,
//     staged by LDS DMA into two buffers, so the next window's weights and x are in flight
//     while this one is multiplied; optionally (s4.kg > 1, with a workspace) K is also split
//     between workgroups, whose float32 partials the last one of a row block adds in order;
//   - windowed (skinny4_fp8_kernel, s4.dma = 2): x staged through registers as
//     [m][k group (4)][chunk] 8-byte words, each window's weights loaded after it is staged.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kWaves = 4;
constexpr int kStageBytes = 32 * 1024;      // LDS for one x window

struct Skinny4Args {
    const uint16_t* x;
    int64_t ldx;
    int M, K;
    int window;          // chunks per LDS window
    int xs_stride;       // 8-byte words between (m, k group) rows of the LDS window
    int ngroups;
    GemvGroup g[kMaxGroups];  // wg_begin counts row blocks; ws_col is the group's first partial column
    // K split between workgroups (pipelined form): workgroup b computes row block b / kgroups over
    // chunks [cpg (b % kgroups), cpg (b % kgroups + 1)) and writes float32 partials to
    // ws[kg][m][ws_ld]; the last of a row block's workgroups (arrival counter) adds them in
    // K-group order and stores.  kgroups = 1: no split, no workspace.
    int kgroups;
    int cpg;
    float* ws;
    uint32_t* counters;      // one per row block; zero between launches
    int ws_ld;               // sum of N over the groups
};

// Workspace of the K split: a fixed block of arrival counters, then the partials (the layout of
// the split-K 16x16x32 kernel, so that either kernel may use a workspace the other has used).
constexpr int kSplitCounterSlots = 16384;
constexpr size_t kSplitCounterBytes = kSplitCounterSlots * sizeof(uint32_t);

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x4 as_bf16x4(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(bf16x4, uint2{lo, hi});
}

// The end of both forms: the 16 MFMA blocks of a lane group summed across lanes, the KS waves'
// partials summed in order through LDS, then the scale, one bf16 rounding and the epilogue.
template <int KS, int T, int G>
__device__ __forceinline__ void skinny4_finish(f32x4 (&acc)[T][G], f32x4 (&partial)[KS > 1 ? KS : 1][kWaves / KS][T][G][4],
                                               const GemvGroup& grp, int M, int row_base, int q, int gw, int lane,
                                               int li) {
    // Sum the 16 blocks (lanes with equal lane % 4) in a fixed order: xor 4, 8, 16, 32.
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = acc[t][g][r];
                v += __shfl_xor(v, 4);
                v += __shfl_xor(v, 8);
                v += __shfl_xor(v, 16);
                v += __shfl_xor(v, 32);
                acc[t][g][r] = v;
            }
    // Lane li (block 0) holds D[r][li] = rows 4 t + r, activation row 4 g + li.
    if constexpr (KS > 1) {
        if (lane < 4) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int g = 0; g < G; ++g) partial[q][gw][t][g][li] = acc[t][g];
        }
        __syncthreads();
        if (q != 0) return;
        if (lane < 4) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    f32x4 v = partial[0][gw][t][g][li];
#pragma unroll
                    for (int qq = 1; qq < KS; ++qq) {
                        const f32x4 p = partial[qq][gw][t][g][li];
                        v = f32x4{v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w};
                    }
                    acc[t][g] = v;
                }
        }
    }
    if (lane < 4) {
        // residuals first (clamped in bounds), then the stores
        uint16_t rres[T][G][4];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    rres[t][g][r] = grp.epi.kind == kEpiResidual
                                        ? grp.epi.res[(int64_t)min(4 * g + li, M - 1) * grp.epi.ldres +
                                                      min(row_base + 4 * t + r, grp.N - 1)]
                                        : 0;
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int m = 4 * g + li;
                if (m >= M) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = row_base + 4 * t + r;
                    if (n < grp.N)
                        grp.y[(int64_t)m * grp.ldy + n] = epilogue(acc[t][g][r], grp.s[n], grp.epi.kind, rres[t][g][r]);
                }
            }
    }
}

// The end of a K-split workgroup: the same cross-lane and cross-wave sums, then the partial
// tile (agent-scope stores, visible to every XCD), the row block's arrival count, and in the
// last workgroup to arrive the sum of the K groups' partials in order 0..kgroups-1, the scale, one
// bf16 rounding and the epilogue.  Every word that crosses workgroups is written and read with
// agent-scope atomics; the arrival is an agent-scope acquire-release read-modify-write (after the
// workgroup barrier that orders the partial stores of all its threads before it), so the last
// arrival's reads of the others' partials happen after their stores.  The counter is re-armed
// by the last arrival.
template <int KS, int T, int G>
__device__ __forceinline__ void skinny4_finish_split(f32x4 (&acc)[T][G],
                                                     f32x4 (&partial)[KS > 1 ? KS : 1][kWaves / KS][T][G][4],
                                                     const Skinny4Args& a, const GemvGroup& grp, int rb_all, int kg,
                                                     int rb_row0, int row_base, int q, int gw, int lane, int li,
                                                     int tid) {
    __shared__ uint32_t last_flag;
    const int M = a.M;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = acc[t][g][r];
                v += __shfl_xor(v, 4);
                v += __shfl_xor(v, 8);
                v += __shfl_xor(v, 16);
                v += __shfl_xor(v, 32);
                acc[t][g][r] = v;
            }
    if constexpr (KS > 1) {
        if (lane < 4) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int g = 0; g < G; ++g) partial[q][gw][t][g][li] = acc[t][g];
        }
        __syncthreads();
        if (q == 0 && lane < 4) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    f32x4 v = partial[0][gw][t][g][li];
#pragma unroll
                    for (int qq = 1; qq < KS; ++qq) {
                        const f32x4 p = partial[qq][gw][t][g][li];
                        v = f32x4{v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w};
                    }
                    acc[t][g] = v;
                }
        }
    }
    if (q == 0 && lane < 4) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int m = 4 * g + li;
            if (m >= M) continue;
            float* dst = a.ws + ((int64_t)kg * M + m) * a.ws_ld + grp.ws_col;
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int n = row_base + 4 * t + r;
                    if (n < grp.N) __hip_atomic_store(dst + n, acc[t][g][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);              // this wave's partial stores have completed
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev =
            __hip_atomic_fetch_add(a.counters + rb_all, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = (prev == (uint32_t)(a.kgroups - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (!last_flag) return;
    // the row block's outputs: kWaves / KS * 4 T rows x M activation rows, spread over the threads;
    // each issues its loads of up to 8 K groups at once, then adds them in order
    constexpr int kRows = kWaves / KS * 4 * T;
    for (int o = tid; o < kRows * M; o += 256) {
        const int m = o / kRows;
        const int n = rb_row0 + (o - m * kRows);
        if (n >= grp.N) continue;
        const float* src = a.ws + (int64_t)m * a.ws_ld + grp.ws_col + n;
        const int64_t step = (int64_t)M * a.ws_ld;
        float tsum = 0.f;
        for (int k0 = 0; k0 < a.kgroups; k0 += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                v[j] = __hip_atomic_load(src + (int64_t)min(k0 + j, a.kgroups - 1) * step, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (k0 + j < a.kgroups) tsum += v[j];
        }
        const uint16_t res = grp.epi.kind == kEpiResidual ? grp.epi.res[(int64_t)m * grp.epi.ldres + n] : 0;
        grp.y[(int64_t)m * grp.ldy + n] = epilogue(tsum, grp.s[n], grp.epi.kind, res);
    }
    if (tid == 0) __hip_atomic_store(a.counters + rb_all, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// KS: waves splitting K; T: row groups (4 rows each) per wave; U: chunks per lane per batch;
// G: groups of 4 activation rows (M <= 4 G).
template <int KS, int T, int U, int G>
__global__ __launch_bounds__(256) void skinny4_fp8_kernel(const Skinny4Args a) {
    extern __shared__ uint2 xs[];                     // [m][kg][xs_stride] + 1 zero word
    constexpr int kRowGroups = kWaves / KS;
    constexpr int kRowsPerWave = 4 * T;
    constexpr int kRowsPerWG = kRowGroups * kRowsPerWave;
    __shared__ f32x4 partial[KS > 1 ? KS : 1][kRowGroups][T][G][4];

    int gi = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && (int)blockIdx.x >= a.g[i].wg_begin) gi = i;
    const GemvGroup grp = a.g[gi];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int gw = wave / KS;                    // row group of this wave within the workgroup
    const int q = wave % KS;                     // K slice of this wave
    const int blk = lane >> 2;                   // MFMA block = chunk offset of this lane
    const int li = lane & 3;                     // A row / B column within the block
    const int row_base = ((int)blockIdx.x - grp.wg_begin) * kRowsPerWG + gw * kRowsPerWave;
    const int M = a.M;
    const int C = a.K >> 4;
    const int window = a.window;
    const int xst = a.xs_stride;
    const int zero_word = M * 4 * xst;

    const uint8_t* __restrict__ wrow[T];
#pragma unroll
    for (int t = 0; t < T; ++t) wrow[t] = grp.W + (int64_t)min(row_base + 4 * t + li, grp.N - 1) * grp.ldw;

    f32x4 acc[T][G];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int g = 0; g < G; ++g) acc[t][g] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (tid == 0) xs[zero_word] = uint2{0, 0};
    constexpr int kXPieces = kStageBytes / 16 / 256;  // 16-byte x pieces per thread per window
    for (int w0 = 0; w0 < C; w0 += window) {
        const int wc = min(window, C - w0);
        const int npieces = 2 * M * wc;               // 16-byte pieces (8 bf16) in the window
        // 1. this window's activations (issued first)
        uint4 xr[kXPieces];
#pragma unroll
        for (int p = 0; p < kXPieces; ++p) {
            const int e = min(tid + 256 * p, npieces - 1);
            const int mm = e / (2 * wc);
            const int rem = e - mm * 2 * wc;
            xr[p] = load16(a.x + (int64_t)mm * a.ldx + (int64_t)(w0 + (rem >> 1)) * 16 + (rem & 1) * 8);
        }
        // 2. this wave's K slice of the window and its first batch of weights
        const int cb = w0 + (q * wc) / KS;
        const int ce = w0 + ((q + 1) * wc) / KS;
        const int clast = max(ce - 1, cb);
        int c0 = cb + blk;
        uint4 wv[T][U];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int u = 0; u < U; ++u)
                wv[t][u] = load_stream16(wrow[t] + (int64_t)min(c0 + 16 * u, clast) * 16);
        // 3. stage x: piece (m, chunk, half) -> words (m, kg = 2 half + {0, 1}, chunk)
        if (w0 != 0) __syncthreads();
#pragma unroll
        for (int p = 0; p < kXPieces; ++p) {
            const int e = tid + 256 * p;
            if (e < npieces) {
                const int mm = e / (2 * wc);
                const int rem = e - mm * 2 * wc;
                const int c = rem >> 1, h = rem & 1;
                xs[(mm * 4 + 2 * h) * xst + c] = uint2{xr[p].x, xr[p].y};
                xs[(mm * 4 + 2 * h + 1) * xst + c] = uint2{xr[p].z, xr[p].w};
            }
        }
        __syncthreads();
        // 4. consume
        for (;;) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 16 * u;
                const bool cvalid = c < ce;
                // B operands: x[4 g + li][chunk c][4 kg .. 4 kg + 3] (zero past M or the slice)
                uint2 xb[G][4];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const int m = 4 * g + li;
                    const bool ok = cvalid && m < M;
#pragma unroll
                    for (int kg = 0; kg < 4; ++kg)
                        xb[g][kg] = xs[ok ? (m * 4 + kg) * xst + (c - w0) : zero_word];
                }
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const uint4 w = wv[t][u];
                    const uint2 p0 = e4m3x4_to_bf16(w.x), p1 = e4m3x4_to_bf16(w.y);
                    const uint2 p2 = e4m3x4_to_bf16(w.z), p3 = e4m3x4_to_bf16(w.w);
                    const bf16x4 A0 = as_bf16x4(p0.x, p0.y), A1 = as_bf16x4(p1.x, p1.y);
                    const bf16x4 A2 = as_bf16x4(p2.x, p2.y), A3 = as_bf16x4(p3.x, p3.y);
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A0, as_bf16x4(xb[g][0].x, xb[g][0].y), acc[t][g], 0, 0, 0);
                        acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A1, as_bf16x4(xb[g][1].x, xb[g][1].y), acc[t][g], 0, 0, 0);
                        acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A2, as_bf16x4(xb[g][2].x, xb[g][2].y), acc[t][g], 0, 0, 0);
                        acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A3, as_bf16x4(xb[g][3].x, xb[g][3].y), acc[t][g], 0, 0, 0);
                    }
                }
            }
            c0 += 16 * U;
            if (c0 - blk >= ce) break;                 // uniform across the wave
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int u = 0; u < U; ++u)
                    wv[t][u] = load_stream16(wrow[t] + (int64_t)min(c0 + 16 * u, clast) * 16);
        }
    }

    skinny4_finish<KS, T, G>(acc, partial, grp, M, row_base, q, gw, lane, li);
}

// Waits until at most N vector memory loads of this wave are outstanding and every LDS access
// has completed, then s_barrier.  Loads complete in issue order, so N = the loads issued after
// the ones that must have landed.
template <int N>
__device__ __forceinline__ void wait_loads_barrier() {
    if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Pipelined form.  The same lane layout, products, reduction and epilogue; K is walked in
// windows of 16 U KS chunks, one batch of U chunks per lane for each of the KS waves splitting a
// window, and the x windows are staged by LDS DMA (no register staging) into two buffers, so
// that the weights and activations of window w + 1 are in flight while window w is multiplied.
// Buffer layout: [4 G rows m][2 halves h][kS words] of 16 bytes; word c of row (m, h) holds
// x[m][16 (w0 + c) + 8 h .. + 8].  kS == 2 (mod 16): the 16 lanes (blk 4p..4p+3, li 0..3) of a
// quarter of one 16-byte read fall in distinct bank groups.  Rows m >= M hold copies of row M - 1
// (their products land only in outputs that are not stored); words past the end of K hold zeros
// (their weight chunks are clamped copies of the row's last chunk).
template <int KS, int T, int U, int G>
__global__ __launch_bounds__(256) void skinny4_dma_kernel(const Skinny4Args a) {
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ uint4 xw[];
    constexpr int kRowGroups = kWaves / KS;
    constexpr int kRowsPerWave = 4 * T;
    constexpr int kRowsPerWG = kRowGroups * kRowsPerWave;
    constexpr int kWin = 16 * U * KS;                  // chunks per window
    constexpr int kS = kWin + 2;                       // words per (m, h) row of a buffer
    constexpr int kBuf = 4 * G * 2 * kS;               // words per buffer
    constexpr int kBlk = kWin < 64 ? kWin : 64;        // chunks per DMA instruction
    constexpr int kBlkPerRow = kWin / kBlk;
    constexpr int kJobs = 4 * G * 2 * kBlkPerRow;      // DMA instructions per window
    __shared__ f32x4 partial[KS > 1 ? KS : 1][kRowGroups][T][G][4];

    const int rb_all = (int)blockIdx.x / a.kgroups;   // row block over all groups
    const int kg = (int)blockIdx.x - rb_all * a.kgroups;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && rb_all >= a.g[i].wg_begin) gi = i;
    const GemvGroup grp = a.g[gi];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int gw = wave / KS;
    const int q = wave % KS;
    const int blk = lane >> 2;
    const int li = lane & 3;
    const int rb_row0 = (rb_all - grp.wg_begin) * kRowsPerWG;
    const int row_base = rb_row0 + gw * kRowsPerWave;
    const int M = a.M;
    const int c_begin = kg * a.cpg;                    // this workgroup's chunks [c_begin, c_end)
    const int c_end = min(a.K >> 4, c_begin + a.cpg);
    const int nw = (c_end - c_begin + kWin - 1) / kWin;
    const uint32_t xw_addr = (uint32_t)(uintptr_t)(lds_void*)xw;

    const uint8_t* __restrict__ wrow[T];
#pragma unroll
    for (int t = 0; t < T; ++t) wrow[t] = grp.W + (int64_t)min(row_base + 4 * t + li, grp.N - 1) * grp.ldw;

    f32x4 acc[T][G];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int g = 0; g < G; ++g) acc[t][g] = f32x4{0.f, 0.f, 0.f, 0.f};

    // x window w into buffer b: job j = (row r = (m, h), block) has lane l copy chunk
    // 64 block + l of the row; lanes past the end of K write zeros instead
    auto stage = [&](int w, int b) {
        const int w0 = c_begin + w * kWin;
        const int wc = min(kWin, c_end - w0);
        for (int j = wave; j < kJobs; j += kWaves) {
            const int r = j / kBlkPerRow;
            const int c = (j - r * kBlkPerRow) * kBlk + lane;
            const int m = min(r >> 1, M - 1);
            const int word = b * kBuf + r * kS + c - lane;
            if (lane < kBlk) {
                if (c < wc)
                    dma16_lds(a.x, (uint32_t)(((int64_t)m * a.ldx + (int64_t)(w0 + c) * 16 + 8 * (r & 1)) * 2),
                              xw_addr + (uint32_t)word * 16);
                else
                    xw[word + lane] = uint4{0, 0, 0, 0};
            }
        }
    };
    // this wave's batch of window w: lane 4 blk + li loads chunk (window slice q) + blk + 16 u of
    // row 4 t + li (chunks past the slice clamped to its last one), as ordinary non-temporal loads
    // that the compiler tracks: it waits for a destination register itself before the register's
    // first use, so nothing depends on how it allocates, copies or spills them.
    auto load_w = [&](u32x4 (&wv)[T][U], int w) {
        const int cb = c_begin + w * kWin + q * 16 * U + blk;
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int u = 0; u < U; ++u)
                wv[t][u] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(wrow[t] + (int64_t)min(cb + 16 * u, c_end - 1) * 16));
    };
    auto consume = [&](const u32x4 (&wv)[T][U], int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int cl = q * 16 * U + blk + 16 * u;
            uint4 xb[G][2];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int h = 0; h < 2; ++h) xb[g][h] = xw[b * kBuf + ((4 * g + li) * 2 + h) * kS + cl];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const u32x4 w = wv[t][u];
                const uint2 p0 = e4m3x4_to_bf16(w[0]), p1 = e4m3x4_to_bf16(w[1]);
                const uint2 p2 = e4m3x4_to_bf16(w[2]), p3 = e4m3x4_to_bf16(w[3]);
                const bf16x4 A0 = as_bf16x4(p0.x, p0.y), A1 = as_bf16x4(p1.x, p1.y);
                const bf16x4 A2 = as_bf16x4(p2.x, p2.y), A3 = as_bf16x4(p3.x, p3.y);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A0, as_bf16x4(xb[g][0].x, xb[g][0].y), acc[t][g], 0, 0, 0);
                    acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A1, as_bf16x4(xb[g][0].z, xb[g][0].w), acc[t][g], 0, 0, 0);
                    acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A2, as_bf16x4(xb[g][1].x, xb[g][1].y), acc[t][g], 0, 0, 0);
                    acc[t][g] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(A3, as_bf16x4(xb[g][1].z, xb[g][1].w), acc[t][g], 0, 0, 0);
                }
            }
        }
    };

    // Two windows in flight: (wa, buffer 0) holds the even windows, (wb, buffer 1) the odd ones.
    // Each window's x DMA is issued before its weights, so waiting until only the next window's
    // weight loads are outstanding covers this window's weights and x and the next window's x.
    // The control flow keeps the compiler's own waits (it tracks the weight loads, not the x DMA)
    // from covering the next window's weights: one window alone is its own path; otherwise every
    // path into the loop over window pairs (windows w + 2 and w + 3 exist: both loads are issued
    // unconditionally) and into the tail (two or three windows left) has the same loads in flight,
    // and the tail's two cases are written out separately.
    u32x4 wa[T][U], wb[T][U];
    stage(0, 0);
    load_w(wa, 0);
    if (nw == 1) {
        wait_loads_barrier<0>();
        consume(wa, 0);
    } else {
        stage(1, 1);
        load_w(wb, 1);
        int w = 0;
        for (; w + 4 <= nw; w += 2) {
            wait_loads_barrier<T * U>();
            consume(wa, 0);
            asm volatile("s_barrier" ::: "memory");    // every wave is done reading buffer 0
            stage(w + 2, 0);
            load_w(wa, w + 2);
            wait_loads_barrier<T * U>();
            consume(wb, 1);
            asm volatile("s_barrier" ::: "memory");    // every wave is done reading buffer 1
            stage(w + 3, 1);
            load_w(wb, w + 3);
        }
        // windows w, w + 1 (in flight) and perhaps w + 2
        wait_loads_barrier<T * U>();
        consume(wa, 0);
        if (w + 3 == nw) {
            asm volatile("s_barrier" ::: "memory");
            stage(w + 2, 0);
            load_w(wa, w + 2);
            wait_loads_barrier<T * U>();
            consume(wb, 1);
            wait_loads_barrier<0>();
            consume(wa, 0);
        } else {
            wait_loads_barrier<0>();
            consume(wb, 1);
        }
    }

    if (a.kgroups > 1)
        skinny4_finish_split<KS, T, G>(acc, partial, a, grp, rb_all, kg, rb_row0, row_base, q, gw, lane, li, tid);
    else
        skinny4_finish<KS, T, G>(acc, partial, grp, M, row_base, q, gw, lane, li);
}

// Dynamic LDS of the pipelined form: two windows of 4 G x 2 rows of 16 U KS + 2 words (the
// static partial sums take at most 2 KiB of the 160 KiB).
constexpr size_t dma_lds_bytes(int KS, int U, int G) { return 2 * (size_t)(8 * G) * (16 * U * KS + 2) * 16; }
constexpr size_t kDmaLdsMax = 156 * 1024;

template <int KS, int T, int U, int G>
hipError_t launch_cfg(Skinny4Args& a, bool dma, hipStream_t stream) {
    constexpr int rows_per_wg = (kWaves / KS) * 4 * T;
    int blocks = 0, col = 0;
    for (int i = 0; i < a.ngroups; ++i) {
        a.g[i].wg_begin = blocks;
        a.g[i].ws_col = col;
        blocks += (a.g[i].N + rows_per_wg - 1) / rows_per_wg;
        col += a.g[i].N;
    }
    a.ws_ld = col;
    if constexpr (dma_lds_bytes(KS, U, G) <= kDmaLdsMax) {
        if (dma) {
            constexpr size_t lds = dma_lds_bytes(KS, U, G);
            constexpr auto kernel = &skinny4_dma_kernel<KS, T, U, G>;
            if constexpr (lds > 64 * 1024) {
                static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                if (attr != hipSuccess) return attr;
            }
            hipLaunchKernelGGL(kernel, dim3(blocks * a.kgroups), dim3(256), lds, stream, a);
            return hipGetLastError();
        }
    }
    if constexpr (T <= 2) {
        if (a.kgroups != 1) return hipErrorInvalidValue;
        const size_t lds = ((size_t)a.M * 4 * a.xs_stride + 1) * sizeof(uint2);
        hipLaunchKernelGGL((skinny4_fp8_kernel<KS, T, U, G>), dim3(blocks), dim3(256), lds, stream, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

template <int KS, int T, int U>
hipError_t launch_g(int M, Skinny4Args& a, bool dma, hipStream_t stream) {
    if (M <= 4) return launch_cfg<KS, T, U, 1>(a, dma, stream);
    if (M <= 8) return launch_cfg<KS, T, U, 2>(a, dma, stream);
    return launch_cfg<KS, T, U, 4>(a, dma, stream);
}

template <int KS, int T>
hipError_t launch_u(int u, int M, Skinny4Args& a, bool dma, hipStream_t stream) {
    switch (u) {
        case 2: return launch_g<KS, T, 2>(M, a, dma, stream);
        case 4: return launch_g<KS, T, 4>(M, a, dma, stream);
        default:
            if constexpr (T == 4) return launch_g<KS, T, 4>(M, a, dma, stream);   // T = 4 x U = 8: too many registers
            else return launch_g<KS, T, 8>(M, a, dma, stream);
    }
}

template <int KS>
hipError_t launch_t(int t, int u, int M, Skinny4Args& a, bool dma, hipStream_t stream) {
    if constexpr (KS == 1)
        if (t == 4 && dma) return launch_u<1, 4>(u, M, a, dma, stream);   // 4 row groups: pipelined form, KS = 1 only
    return t >= 2 ? launch_u<KS, 2>(u, M, a, dma, stream) : launch_u<KS, 1>(u, M, a, dma, stream);
}

// Schedule of the 4x4x4 kernel for M activation rows, K, `rows` weight rows in all groups.
struct S4Plan {
    bool dma;       // pipelined form
    int ks, t, u;
    int kgroups;    // workgroups splitting K (pipelined form with a workspace)
    int cpg;        // chunks per K group
};

S4Plan s4_plan(int M, int K, int64_t rows, int num_cu, bool dma_ok, bool split_ok) {
    const Tuning& tn = tuning();
    const int C = K >> 4;
    S4Plan p{};
    p.dma = dma_ok && tn.s4_dma != 2;
    p.kgroups = 1;
    p.cpg = C;
    if (p.dma) {
        // one batch of U chunks per lane per window; KS = 1 and T = 1 keep the most workgroups
        // and the LDS to two windows of 64 (M > 4) or 128 chunks (measured on config 2: K split
        // between waves widens the window and halves the workgroups per CU)
        p.ks = 1, p.t = 1, p.u = M > 4 ? 4 : 8;
        // M > 8: two row groups per wave once one group would give more than ~3 workgroups per
        // CU (config 2 at M = 16: up_proj 27.1 -> 23.5 us; the smaller shapes lose workgroups)
        if (M > 8 && (rows + 15) / 16 >= 3 * (int64_t)num_cu) p.t = 2;
        // K split between workgroups (s4.kg > 1 K groups; measured slower than no split at every
        // config-2 shape, so not chosen automatically): row tiles of 2 row groups per wave share
        // one 32-chunk x window
        if (split_ok && tn.s4_kg > 1) {
            int ks = 1, t = 2, u = 2;
            if (tn.s4_ks == 1 || tn.s4_ks == 2 || tn.s4_ks == 4) ks = tn.s4_ks;
            if (tn.s4_t == 1 || tn.s4_t == 2 || tn.s4_t == 4) t = tn.s4_t;
            if (tn.s4_u == 2 || tn.s4_u == 4) u = tn.s4_u;
            if (ks != 1 && t == 4) t = 2;
            const int win = 16 * u * ks;
            const int64_t rb = (rows + (kWaves / ks) * 4 * t - 1) / ((kWaves / ks) * 4 * t);
            const int nwin = (C + win - 1) / win;
            const int64_t kg = tn.s4_kg > nwin ? nwin : tn.s4_kg;
            const int cpg = (int)(((C + kg - 1) / kg + win - 1) / win) * win;
            const int kgroups = (C + cpg - 1) / cpg;
            if (kgroups > 1 && rb + kMaxGroups <= kSplitCounterSlots &&
                dma_lds_bytes(ks, u, (M + 3) / 4) <= kDmaLdsMax) {
                p.ks = ks, p.t = t, p.u = u, p.kgroups = kgroups, p.cpg = cpg;
                return p;
            }
        }
        if (tn.s4_ks == 1 || tn.s4_ks == 2 || tn.s4_ks == 4) p.ks = tn.s4_ks;
        if (tn.s4_t == 1 || tn.s4_t == 2 || tn.s4_t == 4) p.t = tn.s4_t;
        if (tn.s4_u == 2 || tn.s4_u == 4 || tn.s4_u == 8) p.u = tn.s4_u;
        if (p.ks != 1 && p.t == 4) p.t = 2;
        if (dma_lds_bytes(p.ks, p.u, (M + 3) / 4) <= kDmaLdsMax) return p;
        p.dma = false;
    }
    // windowed form: K split inside the workgroup so that a lane has 2-8 chunks per window; T = 2
    // when there are enough rows to keep ~3 workgroups per CU
    const int wmax = kStageBytes / (32 * M);
    const int slice = C < wmax ? C : wmax;
    p.ks = slice >= 16 * 8 * 4 ? 4 : (slice >= 16 * 8 * 2 ? 2 : 1);
    if (tn.s4_ks == 1 || tn.s4_ks == 2 || tn.s4_ks == 4) p.ks = tn.s4_ks;
    const int64_t wg_t1 = (rows + (int64_t)(kWaves / p.ks) * 4 - 1) / ((int64_t)(kWaves / p.ks) * 4);
    p.t = (wg_t1 >= 6 * (int64_t)num_cu) ? 2 : 1;
    if (tn.s4_t == 1 || tn.s4_t == 2) p.t = tn.s4_t;
    const int per_lane = (slice / p.ks + 15) / 16;
    p.u = per_lane <= 2 ? 2 : (per_lane <= 4 ? 4 : 8);
    if (tn.s4_u == 2 || tn.s4_u == 4 || tn.s4_u == 8) p.u = tn.s4_u;
    return p;
}

}  // namespace

size_t skinny4_workspace_bytes(int M, int K, int64_t total_rows, int num_cu) {
    const S4Plan p = s4_plan(M, K, total_rows, num_cu, true, true);
    if (!p.dma || p.kgroups <= 1) return 0;
    return kSplitCounterBytes + (size_t)p.kgroups * M * total_rows * sizeof(float);
}

hipError_t launch_skinny4_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                                  int ngroups, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const DeviceInfo& dev = device_info();
    Skinny4Args a{};
    a.x = x;
    a.ldx = ldx;
    a.M = M;
    a.K = K;
    a.ngroups = ngroups;
    int64_t rows = 0;
    for (int i = 0; i < ngroups; ++i) {
        a.g[i] = groups[i];
        rows += groups[i].N;
    }
    const int C = K >> 4;
    // windowed form: x window of 2 M w 16-byte pieces <= 2048 (8 per thread) and M x 32 w bytes
    // <= 32 KiB; (m, kg) rows padded to a stride of 2 mod 8 words (the 4 activation rows one read
    // touches start in different 64-byte bank groups)
    const int wmax = kStageBytes / (32 * M);
    a.window = C < wmax ? C : wmax;
    a.xs_stride = ((a.window + 5) & ~7) + 2;
    // the pipelined form needs 16-byte x rows (LDS DMA) with 32-bit byte offsets
    const bool dma_ok = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (ldx & 7) == 0 &&
                        (int64_t)M * ldx * 2 < ((int64_t)1 << 32);
    const size_t need = skinny4_workspace_bytes(M, K, rows, dev.num_cu);
    const bool split_ok = workspace != nullptr && need > 0 && workspace_bytes >= need &&
                          (reinterpret_cast<uintptr_t>(workspace) & 15) == 0;
    const S4Plan p = s4_plan(M, K, rows, dev.num_cu, dma_ok, split_ok);
    a.kgroups = p.kgroups;
    a.cpg = p.cpg;
    if (p.kgroups > 1) {
        a.counters = static_cast<uint32_t*>(workspace);
        a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kSplitCounterBytes);
    }
    switch (p.ks) {
        case 1: return launch_t<1>(p.t, p.u, M, a, p.dma, stream);
        case 2: return launch_t<2>(p.t, p.u, M, a, p.dma, stream);
        default: return launch_t<4>(p.t, p.u, M, a, p.dma, stream);
    }
}

}  // namespace nmi
