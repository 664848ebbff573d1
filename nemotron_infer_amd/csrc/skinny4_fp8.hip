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
// * x [M, window] is staged per workgroup in LDS by DMA into two buffers, windows of exactly one
//   batch of U chunks per lane, so the next window's weights and x are in flight while this one
//   is multiplied (skinny4_dma_kernel).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kWaves = 4;

struct Skinny4Args {
    const uint16_t* x;
    int64_t ldx;
    int M, K;
    int ngroups;
    GemvGroup g[kMaxGroups];  // wg_begin counts row blocks
};

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x4 as_bf16x4(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(bf16x4, uint2{lo, hi});
}

// The end of the kernel: the 16 MFMA blocks of a lane group summed across lanes, the KS waves'
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

    const int rb_all = (int)blockIdx.x;              // row block over all groups
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
    const int c_begin = 0;                             // the workgroup's chunks [c_begin, c_end)
    const int c_end = a.K >> 4;
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

    skinny4_finish<KS, T, G>(acc, partial, grp, M, row_base, q, gw, lane, li);
}

// Dynamic LDS: two windows of 4 G x 2 rows of 16 U KS + 2 words (the static partial sums take at
// most 2 KiB of the 160 KiB).
constexpr size_t dma_lds_bytes(int KS, int U, int G) { return 2 * (size_t)(8 * G) * (16 * U * KS + 2) * 16; }
constexpr size_t kDmaLdsMax = 156 * 1024;

template <int KS, int T, int U, int G>
hipError_t launch_cfg(Skinny4Args& a, hipStream_t stream) {
    constexpr int rows_per_wg = (kWaves / KS) * 4 * T;
    int blocks = 0;
    for (int i = 0; i < a.ngroups; ++i) {
        a.g[i].wg_begin = blocks;
        blocks += (a.g[i].N + rows_per_wg - 1) / rows_per_wg;
    }
    if constexpr (dma_lds_bytes(KS, U, G) <= kDmaLdsMax) {
        constexpr size_t lds = dma_lds_bytes(KS, U, G);
        constexpr auto kernel = &skinny4_dma_kernel<KS, T, U, G>;
        if constexpr (lds > 64 * 1024) {
            static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (attr != hipSuccess) return attr;
        }
        hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), lds, stream, a);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

template <int KS, int T, int U>
hipError_t launch_g(int M, Skinny4Args& a, hipStream_t stream) {
    if (M <= 4) return launch_cfg<KS, T, U, 1>(a, stream);
    if (M <= 8) return launch_cfg<KS, T, U, 2>(a, stream);
    return launch_cfg<KS, T, U, 4>(a, stream);
}

template <int KS, int T>
hipError_t launch_u(int u, int M, Skinny4Args& a, hipStream_t stream) {
    switch (u) {
        case 2: return launch_g<KS, T, 2>(M, a, stream);
        case 4: return launch_g<KS, T, 4>(M, a, stream);
        default:
            if constexpr (T == 4) return launch_g<KS, T, 4>(M, a, stream);   // T = 4 x U = 8: too many registers
            else return launch_g<KS, T, 8>(M, a, stream);
    }
}

template <int KS>
hipError_t launch_t(int t, int u, int M, Skinny4Args& a, hipStream_t stream) {
    if constexpr (KS == 1)
        if (t == 4) return launch_u<1, 4>(u, M, a, stream);   // 4 row groups: KS = 1 only
    return t >= 2 ? launch_u<KS, 2>(u, M, a, stream) : launch_u<KS, 1>(u, M, a, stream);
}

// Schedule of the 4x4x4 kernel for M activation rows, K, `rows` weight rows in all groups: waves
// splitting K, row groups per wave, chunks per lane per window.
struct S4Plan {
    int ks, t, u;
};

S4Plan s4_plan(int M, int64_t rows, int num_cu) {
    const Tuning& tn = tuning();
    // one batch of U chunks per lane per window; KS = 1 and T = 1 keep the most workgroups and the
    // LDS to two windows of 64 (M > 4) or 128 chunks (measured on config 2: K split between waves
    // widens the window and halves the workgroups per CU)
    S4Plan p{1, 1, M > 4 ? 4 : 8};
    // M > 8: two row groups per wave once one group would give more than ~3 workgroups per CU
    // (config 2 at M = 16: up_proj 27.1 -> 23.5 us; the smaller shapes lose workgroups)
    if (M > 8 && (rows + 15) / 16 >= 3 * (int64_t)num_cu) p.t = 2;
    if (tn.s4_ks == 1 || tn.s4_ks == 2 || tn.s4_ks == 4) p.ks = tn.s4_ks;
    if (tn.s4_t == 1 || tn.s4_t == 2 || tn.s4_t == 4) p.t = tn.s4_t;
    if (tn.s4_u == 2 || tn.s4_u == 4 || tn.s4_u == 8) p.u = tn.s4_u;
    if (p.ks != 1 && p.t == 4) p.t = 2;
    // a knob choice whose windows do not fit the LDS: halve the chunks per lane, then the K split
    while (dma_lds_bytes(p.ks, p.u, (M + 3) / 4) > kDmaLdsMax && p.u > 2) p.u /= 2;
    while (dma_lds_bytes(p.ks, p.u, (M + 3) / 4) > kDmaLdsMax && p.ks > 1) p.ks /= 2;
    return p;
}

}  // namespace

hipError_t launch_skinny4_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                                  int ngroups, hipStream_t stream) {
    // the LDS DMA of x needs 16-byte rows and 32-bit byte offsets; otherwise (not reached from the
    // C ABI, which requires the alignment; an x of 4 GiB or more) the GEMM takes the call
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (ldx & 7) != 0 || (int64_t)M * ldx * 2 >= ((int64_t)1 << 32))
        return launch_gemm_grouped(x, ldx, M, K, groups, ngroups, stream, nullptr, 0);
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
    const S4Plan p = s4_plan(M, rows, device_info().num_cu);
    switch (p.ks) {
        case 1: return launch_t<1>(p.t, p.u, M, a, stream);
        case 2: return launch_t<2>(p.t, p.u, M, a, stream);
        default: return launch_t<4>(p.t, p.u, M, a, stream);
    }
}

}  // namespace nmi
