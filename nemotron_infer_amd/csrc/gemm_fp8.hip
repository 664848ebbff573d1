// gemm_fp8.hip -- prefill fp8-weight GEMM on bf16 MFMA for gfx950.
//
//   y[m,n] = bf16_rne( (sum_k float(x[m,k]) * float(W[n,k])) * s[n] )
//
// Replaces the reference's prefill path (nemotron_infer/csrc/include/ops/gemm.cuh:325-403:
// activation quantization to e4m3, cuBLASLt fp8 matmul, then a separate per-row scale
// kernel that rounds to bf16 a second time, gemm.cuh:227-238).  Here the activations stay
// bf16 and the result is rounded once:
//
// * Block tile BM x BN x 64, 4 waves in a 2 x 2 arrangement, each wave a (BM/2) x (BN/2)
//   tile of v_mfma_f32_16x16x32_bf16 (fp32 accumulation).
// * Per K step the workgroup loads the bf16 x tile (16 B per lane) and the e4m3 W tile
//   (16 codes per lane) into registers, converts the codes to bf16 with
//   v_cvt_scalef32_pk_bf16_fp8 (exact), and writes both tiles to LDS, double-buffered so
//   the global loads of step t+1 overlap the MFMAs of step t.
// * LDS rows are 64 bf16 (eight 16-byte chunks); chunk c of row r is stored at swz(r, c),
//   which spreads the 16 rows an MFMA operand read touches over all banks.
// * Epilogue: acc * s[n] in float32, one bf16 RNE rounding, masked for ragged M and N.
#include <algorithm>
#include <type_traits>

#include "nmi_device.hpp"
#include "nmi_fp8_linear.h"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kBK = 64;

// LDS position of 16-byte chunk c (of 8) in a 128-byte tile row.  An MFMA operand read has 16
// consecutive lanes on 16 consecutive rows at the same chunk; with 64 four-byte banks, rows r
// and r + 2 start on the same bank, so the chunk is permuted by bits 1-3 of the row: the 16 rows
// then cover 16 distinct 16-byte bank groups (an XOR with row & 7 left rows r and r + 8 on the
// same group, a two-way conflict measured with SQ_LDS_BANK_CONFLICT).  Row-order writes (8 or 4
// lanes per row) stay conflict-free.
__device__ __forceinline__ int swz(int row, int c) { return c ^ ((row >> 1) & 7); }

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_fp8_w8a16_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ W, int64_t ldw,
    const float* __restrict__ s, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, const Epi epi) {
    constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
    constexpr int TM = WM / 16, TN = WN / 16;    // MFMA tiles per wave
    constexpr int A_PER = BM * (kBK / 8) / 256;  // 16-byte bf16 chunks per thread
    constexpr int B_PER = BN * (kBK / 16) / 256; // 16-byte e4m3 chunks per thread
    static_assert(A_PER >= 1 && B_PER >= 1, "tile too small for 256 threads");
    __shared__ __attribute__((aligned(16))) uint16_t lds[2][(BM + BN) * kBK];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;

    uint4 ra[A_PER], rb[B_PER];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int id = tid + 256 * i;
            const int row = id >> 3, kc = id & 7;
            const int gm = m0 + row, gk = k0 + kc * 8;
            ra[i] = (gm < M && gk < K) ? load16(x + (int64_t)gm * ldx + gk) : uint4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int id = tid + 256 * i;
            const int row = id >> 2, kc = id & 3;
            const int gn = n0 + row, gk = k0 + kc * 16;
            rb[i] = (gn < N && gk < K) ? load16(W + (int64_t)gn * ldw + gk) : uint4{0, 0, 0, 0};
        }
    };
    auto sstore = [&](int buf) {
        uint16_t* A = lds[buf];
        uint16_t* B = lds[buf] + BM * kBK;
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int id = tid + 256 * i;
            const int row = id >> 3, kc = id & 7;
            *reinterpret_cast<uint4*>(A + row * kBK + (swz(row, kc) << 3)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int id = tid + 256 * i;
            const int row = id >> 2, kc = id & 3;
            const uint2 d0 = e4m3x4_to_bf16(rb[i].x), d1 = e4m3x4_to_bf16(rb[i].y);
            const uint2 d2 = e4m3x4_to_bf16(rb[i].z), d3 = e4m3x4_to_bf16(rb[i].w);
            const int c0 = 2 * kc, c1 = 2 * kc + 1;
            *reinterpret_cast<uint4*>(B + row * kBK + (swz(row, c0) << 3)) = uint4{d0.x, d0.y, d1.x, d1.y};
            *reinterpret_cast<uint4*>(B + row * kBK + (swz(row, c1) << 3)) = uint4{d2.x, d2.y, d3.x, d3.y};
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jn = 0; jn < TN; ++jn) acc[i][jn] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int KT = (K + kBK - 1) / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * kBK);
        const uint16_t* A = lds[buf];
        const uint16_t* B = lds[buf] + BM * kBK;
#pragma unroll
        for (int ks = 0; ks < kBK / 32; ++ks) {
            const int chunk = ks * 4 + (lane >> 4);
            bf16x8 af[TM], bfr[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int row = wm * WM + i * 16 + (lane & 15);
                af[i] = *reinterpret_cast<const bf16x8*>(A + row * kBK + (swz(row, chunk) << 3));
            }
#pragma unroll
            for (int jn = 0; jn < TN; ++jn) {
                const int row = wn * WN + jn * 16 + (lane & 15);
                bfr[jn] = *reinterpret_cast<const bf16x8*>(B + row * kBK + (swz(row, chunk) << 3));
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int jn = 0; jn < TN; ++jn)
                    acc[i][jn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[jn], acc[i][jn], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds D[(lane>>4)*4 + t][lane & 15] of each 16x16 tile.  Residuals are
    // loaded (clamped in bounds) before the first store.
    uint16_t rres[TN][TM][4];
#pragma unroll
    for (int jn = 0; jn < TN; ++jn)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int n = min(n0 + wn * WN + jn * 16 + (lane & 15), N - 1);
                const int m = min(m0 + wm * WM + i * 16 + (lane >> 4) * 4 + t, M - 1);
                rres[jn][i][t] = epi.kind == kEpiResidual ? epi.res[(int64_t)m * epi.ldres + n] : 0;
            }
#pragma unroll
    for (int jn = 0; jn < TN; ++jn) {
        const int n = n0 + wn * WN + jn * 16 + (lane & 15);
        if (n >= N) continue;
        const float sc = s[n];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = m0 + wm * WM + i * 16 + (lane >> 4) * 4 + t;
                if (m < M) y[(int64_t)m * ldy + n] = epilogue(acc[i][jn][t], sc, epi.kind, rres[jn][i][t]);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Large tiles: BM x BN x 64 with 4 waves of (BM/2) x (BN/2) (128 x 128 for 256 x 256), W as
// the MFMA A operand (16 weight rows per block) and x as B, so each lane ends with four
// consecutive output columns n of one row m: one 8-byte store and one scale per n.
// Double-buffered in dynamic LDS (2 x (BM + BN) x 64 bf16 = 128 KiB at 256 x 256), one
// barrier per K step, global loads of step t+1 in flight during the MFMAs of step t.
// Workgroups are dispatched to the 8 XCDs round-robin; tile t is given to the workgroup
// that lands on XCD t / ceil(T / 8), so each XCD works through a contiguous run of tiles
// (n fastest: consecutive tiles share their x rows in that XCD's L2).
// Loads read clamped in-range addresses unconditionally; K-tail pieces are zeroed in
// registers before the LDS store (rows past M or N only feed outputs that are not stored).
struct GemmArgs {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* W;
    int64_t ldw;
    const float* s;
    uint16_t* y;
    int64_t ldy;
    int M, N, K;
    int tiles_m, tiles_n, per_xcd;
    int gh;                 // DMA-fed kernel: tile order, row bands per group (tile_coords)
    int vec_store;          // y 8-byte aligned and ldy % 4 == 0
    int vec_res;            // residual 8-byte aligned and ldres % 4 == 0
    Epi epi;
    // Stream-K (DMA-fed kernel): sk_total = tiles * K steps (0: one tile per workgroup); the
    // workspace's flag slots (zero at rest), its error word (set when a wait for a flag gave up)
    // and fp32 partial tiles, one per workgroup; this device's error word in pinned host memory
    // (set with it); the wait's poll limit; sk_lostflag (tests only): contributors raise their
    // flags only after their finisher has given up waiting (a late flag), so that every wait
    // runs into its limit.
    int64_t sk_total;
    uint32_t* sk_flags;
    float* sk_part;
    uint32_t* sk_error;
    uint32_t* sk_host_error;
    int sk_spin;
    int sk_lostflag;
    // DMA-fed kernel's epilogue: s 16-byte aligned; y and the residual 16-byte aligned with row
    // strides that keep every row so (16-byte row pieces)
    int vec_scale, vec16, vec16_res;
    // DMA-fed kernel: the matrices sharing x (grouped launches; one for a plain GEMM).  Column
    // band tn of the launch (tiles_n bands over all groups) belongs to the last group whose
    // tn_begin <= tn, at columns (tn - tn_begin) * 256 of that group.
    struct Group {
        const uint8_t* W;
        int64_t ldw;
        const float* s;
        uint16_t* y;
        int64_t ldy;
        const uint16_t* res;
        int64_t ldres;
        int N, tn_begin, epi, vec_scale, vec16, vec16_res;
    };
    int ngroups;
    Group grp[kMaxGroups];
};

// ---------------------------------------------------------------------------------------
// 32 x 32 x 16 MFMA variant of the large-tile kernel: the same tiles, LDS layout, XCD order
// and epilogue, but v_mfma_f32_32x32x16_bf16 (half the fragment registers per k step of the
// 16 x 16 x 32 form), with the fragments of k step s+1 read from LDS while the MFMAs of
// step s run (two fragment register sets).  Operand layouts (gfx950): A lane l holds row
// l % 32, k 8 (l / 32) .. +7; B lane l holds column l % 32, the same k; D register r of lane l
// is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
// Schedule: the next k tile's LDS stores go between the MFMA groups of the current one, and each
// group's fragment reads are interleaved one by one with the previous group's MFMAs.  Used where
// the DMA-fed kernel cannot take the operands (K not a multiple of 64, unaligned x or W).
template <int BM, int BN, int NW>
__global__ __launch_bounds__(NW * 64, 1) void gemm_fp8_w8a16_m32_kernel(const GemmArgs a) {
    constexpr int BK = kBK;
    constexpr int NT = NW * 64;                     // threads
    constexpr int WGN = NW == 8 ? 4 : 2;            // waves along n
    constexpr int WTM = BM / 2, WTN = BN / WGN;     // wave tile (m x n)
    constexpr int TM = WTM / 32, TN = WTN / 32;     // 32 x 32 MFMA tiles per wave
    constexpr int XP = BM * (BK / 8) / NT;
    constexpr int WP = BN * (BK / 16) / NT;
    constexpr int STAGE = (BM + BN) * BK;
    static_assert(XP >= 1 && WP >= 1 && TM >= 1 && TN >= 1, "tile too small");
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];

    const int M = a.M, N = a.N, K = a.K;
    const int KT = (K + BK - 1) / BK;
    int m0 = 0, n0 = 0;                             // origin of the tile being computed

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wn = wave % WGN, wm = wave / WGN;

    uint4 rx[XP], rw[WP];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int p = tid + NT * i;
            const int row = p >> 3, kc = p & 7;
            const int gm = min(m0 + row, M - 1), gk = min(k0 + kc * 8, K - 8);
            rx[i] = load16(a.x + (int64_t)gm * a.ldx + gk);
        }
#pragma unroll
        for (int i = 0; i < WP; ++i) {
            const int p = tid + NT * i;
            const int row = p >> 2, kc = p & 3;
            const int gn = min(n0 + row, N - 1), gk = min(k0 + kc * 16, K - 16);
            rw[i] = load16(a.W + (int64_t)gn * a.ldw + gk);
        }
    };
    // LDS tile layout: rows of eight 16-byte chunks, chunk c of row r at swz(r, c).
    auto put16 = [&](uint16_t* T, int rows, int row, int c, uint4 v) {
        (void)rows;
        *reinterpret_cast<uint4*>(T + row * BK + (swz(row, c) << 3)) = v;
    };
    auto get16 = [&](const uint16_t* T, int rows, int row, int c) -> bf16x8 {
        (void)rows;
        return *reinterpret_cast<const bf16x8*>(T + row * BK + (swz(row, c) << 3));
    };
    auto sstore_x = [&](int buf, int k0) {
        uint16_t* Xs = lds + buf * STAGE + BN * BK;
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int p = tid + NT * i;
            const int row = p >> 3, kc = p & 7;
            const uint4 v = (k0 + kc * 8 < K) ? rx[i] : uint4{0, 0, 0, 0};
            put16(Xs, BM, row, kc, v);
        }
    };
    auto sstore_w = [&](int buf, int k0) {
        uint16_t* Ws = lds + buf * STAGE;
#pragma unroll
        for (int i = 0; i < WP; ++i) {
            const int p = tid + NT * i;
            const int row = p >> 2, kc = p & 3;
            const uint4 w = (k0 + kc * 16 < K) ? rw[i] : uint4{0, 0, 0, 0};
            const uint2 d0 = e4m3x4_to_bf16(w.x), d1 = e4m3x4_to_bf16(w.y);
            const uint2 d2 = e4m3x4_to_bf16(w.z), d3 = e4m3x4_to_bf16(w.w);
            put16(Ws, BN, row, 2 * kc, uint4{d0.x, d0.y, d1.x, d1.y});
            put16(Ws, BN, row, 2 * kc + 1, uint4{d2.x, d2.y, d3.x, d3.y});
        }
    };
    auto sstore = [&](int buf, int k0) {
        sstore_x(buf, k0);
        sstore_w(buf, k0);
    };
    // Fragments of k step s (16 k = chunks 2s, 2s+1) from LDS stage `buf`.
    auto frags = [&](int buf, int s, bf16x8 (&af)[TN], bf16x8 (&bfr)[TM]) {
        const uint16_t* Ws = lds + buf * STAGE;
        const uint16_t* Xs = Ws + BN * BK;
        const int chunk = 2 * s + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TN; ++i) af[i] = get16(Ws, BN, wn * WTN + i * 32 + (lane & 31), chunk);
#pragma unroll
        for (int j = 0; j < TM; ++j) bfr[j] = get16(Xs, BM, wm * WTM + j * 32 + (lane & 31), chunk);
    };

    f32x16 acc[TN][TM];
    bf16x8 af0[TN], bf0[TM], af1[TN], bf1[TM];
    auto mfmas = [&](const bf16x8 (&af)[TN], const bf16x8 (&bfr)[TM]) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    };
    auto mfmas_half = [&](const bf16x8 (&af)[TN], const bf16x8 (&bfr)[TM], int h) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = h * (TM / 2); j < (h + 1) * (TM / 2); ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    };
    auto zero_acc = [&]() {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    };
    // acc += the K steps [kb, ke) of the tile at (m0, n0).
    auto run = [&](int kb, int ke) {
    gload(kb * BK);
    sstore(0, kb * BK);
    __syncthreads();
    frags(0, 0, af0, bf0);
    for (int kt = kb; kt < ke; ++kt) {
        const int buf = (kt - kb) & 1;
        const bool more = kt + 1 < ke;
        if (more) gload((kt + 1) * BK);
        // The next tile's LDS stage (buf ^ 1) was last read before the previous barrier, so its
        // stores go between this tile's MFMA groups: the matrix cores keep working while the x
        // tile and the converted W tile are written.
        static_assert(BK / 16 == 4, "four k steps per tile");
        // fragment reads of the next k step, then the MFMAs of this one (independent), one read
        // between every two MFMAs
        auto step = [&](int s_next, bf16x8 (&afn)[TN], bf16x8 (&bfn)[TM], const bf16x8 (&af)[TN],
                        const bf16x8 (&bfr)[TM]) {
            frags(buf, s_next, afn, bfn);
            mfmas(af, bfr);
#pragma unroll
            for (int q = 0; q < TN + TM; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // one LDS read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, TN * TM - (TN + TM), 0);
        };
        // k steps 0-2 with the reads of steps 1-3 under them; then k step 3 in two halves (m rows
        // j < TM/2, then the rest) with the x stores before the first and the converted W stores
        // before the second.
        static_assert(TM % 2 == 0, "k step 3 is split along m");
        step(1, af1, bf1, af0, bf0);
        step(2, af0, bf0, af1, bf1);
        step(3, af1, bf1, af0, bf0);
        if (more) sstore_x(buf ^ 1, (kt + 1) * BK);
        mfmas_half(af1, bf1, 0);
        if (more) sstore_w(buf ^ 1, (kt + 1) * BK);
        mfmas_half(af1, bf1, 1);
        __syncthreads();
        if (more) frags(buf ^ 1, 0, af0, bf0);
    }
    };

    // Epilogue: register r of lane l is n = 8 (r / 4) + 4 (l / 32) + r % 4, m = l % 32.
    // Residuals are loaded (clamped in bounds) before the first store.
    auto store = [&]() {
    uint2 rres[TN][4][TM];
    if (a.epi.kind == kEpiResidual) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq)
#pragma unroll
                for (int j = 0; j < TM; ++j) {
                    const int n = n0 + wn * WTN + i * 32 + 8 * gq + 4 * (lane >> 5);
                    const int m = min(m0 + wm * WTM + j * 32 + (lane & 31), M - 1);
                    const int64_t row = (int64_t)m * a.epi.ldres;
                    rres[i][gq][j] = load_res4(a.epi.res, row + min(n, N - 1), row + N - 1, a.vec_res && n + 3 < N);
                }
    }
#pragma unroll
    for (int i = 0; i < TN; ++i) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
            const int n = n0 + wn * WTN + i * 32 + 8 * gq + 4 * (lane >> 5);
            float sc[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[r] = a.s[min(n + r, N - 1)];
            const bool full = a.vec_store && (n + 3 < N);
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int m = m0 + wm * WTM + j * 32 + (lane & 31);
                if (m >= M) continue;
                uint16_t* yp = a.y + (int64_t)m * a.ldy + n;
                const uint2 rv = rres[i][gq][j];
                const uint16_t b0 = epilogue(acc[i][j][4 * gq + 0], sc[0], a.epi.kind, (uint16_t)rv.x);
                const uint16_t b1 = epilogue(acc[i][j][4 * gq + 1], sc[1], a.epi.kind, (uint16_t)(rv.x >> 16));
                const uint16_t b2 = epilogue(acc[i][j][4 * gq + 2], sc[2], a.epi.kind, (uint16_t)rv.y);
                const uint16_t b3 = epilogue(acc[i][j][4 * gq + 3], sc[3], a.epi.kind, (uint16_t)(rv.y >> 16));
                if (full) {
                    *reinterpret_cast<uint2*>(yp) = uint2{(uint32_t)b0 | ((uint32_t)b1 << 16),
                                                          (uint32_t)b2 | ((uint32_t)b3 << 16)};
                } else {
                    if (n < N) yp[0] = b0;
                    if (n + 1 < N) yp[1] = b1;
                    if (n + 2 < N) yp[2] = b2;
                    if (n + 3 < N) yp[3] = b3;
                }
            }
        }
    }
    };

    // One tile per workgroup, XCD-ordered: workgroup g runs on XCD g % 8, which takes the
    // consecutive tiles [x * per_xcd, (x + 1) * per_xcd).
    const int g = (int)blockIdx.x;
    const int local = g >> 3;
    const int tile = (g & 7) * a.per_xcd + local;
    if (local >= a.per_xcd || tile >= a.tiles_m * a.tiles_n) return;   // uniform
    const int tm = tile / a.tiles_n;
    m0 = tm * BM;
    n0 = (tile - tm * a.tiles_n) * BN;
    zero_acc();
    run(0, KT);
    store();
}

// ---------------------------------------------------------------------------------------
// DMA-fed 256 x 256 kernel: 4 waves (one per SIMD), each a 128 x 128 tile of 32 x 32 x 16
// MFMAs with the 256 fp32 accumulators per lane in AGPRs.  Both operands go global -> LDS
// with global_load_lds_dwordx4 (no register staging, no LDS store instructions): x as bf16,
// W as the raw e4m3 codes.  W fragments are converted to bf16 after the LDS read (one
// v_cvt_scalef32_pk_bf16_fp8 per 2 codes, one k step ahead of their MFMAs).  Three LDS stages
// of 48 KiB (W 256 x 64 codes, x 256 x 64 bf16); the DMA of k tile t + 2 is issued while
// tile t is multiplied, and one s_barrier per k tile publishes the next stage.
//
// k order inside a 64-wide k tile: the MFMA's 16-wide k step s, lane half h, element e
// (0..7) is k = 32 (s / 2) + 16 h + 8 (s % 2) + e.  A lane's 16 consecutive W codes
// (k = 32 j + 16 h .. + 15) then feed k steps 2 j and 2 j + 1, and its x fragment for step s is
// the 16-byte chunk 4 (s / 2) + 2 h + s % 2 of the row: one 16-byte LDS read each.  Both
// operands use the same order, so the sum over the tile is unchanged.
//
// LDS layouts (bank groups of 256 B, 16 lanes per ds_read_b128 pass): W rows are 64 B
// (four 16-byte chunks), chunk q of row r at q ^ ((r >> 2) & 3); x rows are 128 B, chunk c
// of row r at swz(r, c).  A fragment read (16 consecutive rows, one logical chunk) then hits
// 16 distinct bank groups, and every DMA instruction writes 1 KiB of consecutive LDS: lane l
// fetches the global chunk that belongs at LDS offset 16 l.
//
// Requirements (checked on the host): K % 64 == 0; x, W 16-byte aligned, ldx % 8 == 0,
// ldw % 16 == 0; M * ldx * 2 and N * ldw below 2^31 (32-bit DMA offsets).
constexpr int kDmaStage = 256 * 64 + 256 * 64 * 2;    // bytes per LDS stage
constexpr int kDmaStages = 3;
constexpr size_t kDmaPartialBytes = (size_t)256 * 256 * sizeof(float);   // one fp32 256 x 256 tile

// 16 bytes per lane from base + off to LDS [lds_addr + 16 lane].  Inline asm so that the
// compiler does not track the LDS write (it would wait for every outstanding DMA before any
// LDS read); completion is waited for with an explicit vmcnt before the barrier that
// publishes the stage.  m0 is set in the statement and listed as clobbered; the compiler warns
// that it may not preserve a reserved register across it, and no compiler-generated code of
// this file uses m0 (checked in its assembly), so nothing lives there to be lost.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_addr)
                 : "memory", "m0");
}

// Tile seq of the DMA-fed kernel's tile order -> (row band tm, column band tn): groups of gh row
// bands, column bands in order within a group, row bands fastest (the last group may be shorter).
// An XCD takes a contiguous run of seq, so gh sets its footprint: gh = tiles_m gives whole column
// bands (few W column bands, every x row band), gh = 1 whole row bands.  Every seq below
// tiles_m * tiles_n maps to one tile inside the grid.
__device__ __forceinline__ void tile_coords(int seq, int tiles_m, int tiles_n, int gh, int& tm, int& tn) {
    const int per = gh * tiles_n;
    const int rg = seq / per;
    const int r0 = rg * gh;
    const int h = min(gh, tiles_m - r0);
    const int loc = seq - rg * per;
    tn = loc / h;
    tm = r0 + (loc - tn * h);
}

template <bool SK, bool GROUPED, int BM = 256>
__global__ __launch_bounds__(256, 1) void gemm_fp8_w8a16_dma_kernel(const GemmArgs a) {
    // BM = 256: 256 x 256 tiles, each wave 128 x 128 (TM = 4 blocks of 32 x rows); BM = 128:
    // 128 x 256 tiles, each wave 64 x 128 (TM = 2), data-parallel only
    static_assert(BM == 256 || (BM == 128 && !SK), "tile rows");
    constexpr int NT = 256, BK = kBK, W_STAGE = 256 * 64, TN = 4, TM = BM / 64;
    constexpr int XI = BM / 32;                     // x DMA instructions per wave and k tile
    constexpr int STAGE = W_STAGE + BM * 128;       // bytes per LDS stage
    __shared__ int sk_up;                           // stream-K: the flag the finisher waited for came
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_u16[];      // one name for the dynamic LDS
    uint8_t* const lds = reinterpret_cast<uint8_t*>(lds_u16);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5, l32 = lane & 31;
    const int M = a.M, K = a.K, KT = K / BK;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)lds;
    int m0 = 0, n0 = 0;
    // the current tile's matrix: for a grouped launch chosen per tile (wave-uniform), otherwise
    // read straight from the kernel arguments wherever used (so nothing needs to stay live)
    const uint8_t* gW_ = a.grp[0].W;
    int64_t gldw_ = a.grp[0].ldw;
    const float* gs_ = a.grp[0].s;
    uint16_t* gy_ = a.grp[0].y;
    int64_t gldy_ = a.grp[0].ldy, gldres_ = a.grp[0].ldres;
    const uint16_t* gres_ = a.grp[0].res;
    int gN_ = a.grp[0].N, gepi_ = a.grp[0].epi, gvs_ = a.grp[0].vec_scale, gv16_ = a.grp[0].vec16,
        gv16r_ = a.grp[0].vec16_res;
#define NMI_G(field, var) (GROUPED ? var : a.grp[0].field)
#define gW NMI_G(W, gW_)
#define gldw NMI_G(ldw, gldw_)
#define gs NMI_G(s, gs_)
#define gy NMI_G(y, gy_)
#define gldy NMI_G(ldy, gldy_)
#define gldres NMI_G(ldres, gldres_)
#define gres NMI_G(res, gres_)
#define gN NMI_G(N, gN_)
#define gepi NMI_G(epi, gepi_)
#define gvs NMI_G(vec_scale, gvs_)
#define gv16 NMI_G(vec16, gv16_)
#define gv16r NMI_G(vec16_res, gv16r_)
    // column band tn of the launch -> its group's matrix and n0
    auto select = [&](const int tn) __attribute__((always_inline)) {
        if constexpr (GROUPED) {
            int gi = 0;
#pragma unroll
            for (int i = 1; i < kMaxGroups; ++i)
                if (i < a.ngroups && tn >= a.grp[i].tn_begin) gi = i;
            gi = __builtin_amdgcn_readfirstlane(gi);
            const GemmArgs::Group& G = a.grp[gi];
            gW_ = G.W; gldw_ = G.ldw; gs_ = G.s; gy_ = G.y; gldy_ = G.ldy; gres_ = G.res; gldres_ = G.ldres;
            gN_ = G.N; gepi_ = G.epi; gvs_ = G.vec_scale; gv16_ = G.vec16; gv16r_ = G.vec16_res;
            n0 = (tn - G.tn_begin) * 256;
        } else {
            n0 = tn * 256;
        }
    };

    f32x16 acc[TN][TM];
    auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    };

    // acc += k tiles [kb, ke) of the tile at (m0, n0).  Entered and left with no DMA in flight
    // and every wave past its last LDS read.
    auto run = [&](int kb, int ke) __attribute__((always_inline)) {
        // The lane-derived offsets below are recomputed per call from an opaque copy of the
        // thread id: hoisted to kernel scope, they stayed live across the stream-K bookkeeping
        // and were spilled, and their reloads put vmcnt waits inside the k loop.
        int tid_r;
        asm volatile("v_mov_b32 %0, %1" : "=v"(tid_r) : "v"(tid));
        const int lane = tid_r & 63, h = lane >> 5, l32 = lane & 31;
        // DMA sources, 32-bit byte offsets from the operand bases.  W instruction i of this wave:
        // rows (4 i + wave) * 16 + lane / 4, LDS chunk lane % 4; x instruction i: rows
        // (4 i + wave) * 8 + lane / 8, LDS chunk lane % 8.  Rows past M or gN are clamped (their
        // results are not stored).
        uint32_t woff[4], xoff[XI];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = (4 * i + wave) * 16 + (lane >> 2);
            const int q = (lane & 3) ^ ((r >> 2) & 3);
            woff[i] = (uint32_t)(min(n0 + r, gN - 1) * gldw + 16 * q);
        }
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int r = (4 * i + wave) * 8 + (lane >> 3);
            xoff[i] = (uint32_t)((min(m0 + r, M - 1) * a.ldx + 8 * swz(r, lane & 7)) * 2);
        }
        // LDS byte addresses of the stage being read, the next one and the one being filled
        // (rotated every k tile)
        uint32_t s_cur = lds0, s_nxt = lds0 + STAGE, s_dma = lds0 + 2 * STAGE;
        // DMA part 0: the W tile; parts 1 (, 2): the x tile (in halves at BM = 256)
        auto dma_to = [&](uint32_t base, int kt, int part, int k) {
            if (part == 0) {
                dma16(gW + (int64_t)kt * BK, woff[k], base + (4 * k + wave) * 16 * 64);
            } else {
                const int i = 4 * (part - 1) + k;
                dma16(reinterpret_cast<const uint8_t*>(a.x) + (int64_t)kt * BK * 2, xoff[i],
                      base + W_STAGE + (4 * i + wave) * 8 * 128);
            }
        };
        auto rd_x = [&](uint32_t sb, int s, int j) -> bf16x8 {
            const uint8_t* base = lds + (sb - lds0) + W_STAGE;
            const int c = 4 * (s >> 1) + 2 * h + (s & 1);
            const int r = wm * (BM / 2) + j * 32 + l32;
            return *reinterpret_cast<const bf16x8*>(base + r * 128 + swz(r, c) * 16);
        };
        auto rd_w = [&](uint32_t sb, int jp, int i) -> uint4 {
            const uint8_t* base = lds + (sb - lds0);
            const int r = wn * 128 + i * 32 + l32;
            return *reinterpret_cast<const uint4*>(base + r * 64 + (((2 * jp + h) ^ ((r >> 2) & 3)) * 16));
        };
        // conversion c (0..15) of a W code pair set, half t: fragment c / 4, 32-bit word c % 4
        auto cvt1 = [&](const uint4 (&wr)[4], int t, int c, u32x4 (&cf)[4]) {
            const int i = c >> 2, e = c & 3;
            const uint32_t w = (e >> 1) ? (t ? wr[i].w : wr[i].y) : (t ? wr[i].z : wr[i].x);
            const bf16x2 v = (e & 1) ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true)
                                     : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false);
            cf[i][e] = __builtin_bit_cast(uint32_t, v);
        };
        auto mf = [&](const u32x4 (&cf)[4], const bf16x8 (&xf)[TM], int q) {
            const int i = q / TM, j = q % TM;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, cf[i]), xf[j], acc[i][j], 0, 0, 0);
        };

        constexpr int NP = 1 + BM / 128;            // DMA parts per k tile (4 instructions each)
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int k = 0; k < 4; ++k) dma_to(s_cur, kb, p, k);
        if (kb + 1 < ke) {
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int k = 0; k < 4; ++k) dma_to(s_nxt, kb + 1, p, k);
            if constexpr (BM == 256) asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        }
        uint4 wr0[4], wr1[4];
        bf16x8 xa[TM], xb[TM];
        u32x4 cA[4], cB[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) wr0[i] = rd_w(s_cur, 0, i);
#pragma unroll
        for (int j = 0; j < TM; ++j) xa[j] = rd_x(s_cur, 0, j);
#pragma unroll
        for (int c = 0; c < 16; ++c) cvt1(wr0, 0, c, cA);

        // One k tile in an explicit order: every k step is 16 groups of one MFMA plus at most
        // one LDS read, one conversion and one DMA, fenced so that the compiler keeps them apart.
        auto iter = [&](int kt, auto pf_tag) {
            constexpr bool pf = decltype(pf_tag)::value;   // issue the DMA of k tile kt + 2
            const uint32_t st = s_cur, nst = s_nxt;
            const bool more = pf || kt + 1 < ke;
            if constexpr (BM == 128) {
                // 128 x 256 tiles: 8 MFMAs per k step (q: W block q / 2, x block q % 2), two
                // conversions per MFMA, the x and W reads of the next steps in the first slots,
                // DMA parts 0 (W) and 1 (x) in steps 0 and 1.  The next tile's step-0 operands
                // are read after the barrier of step 3; cA[0] is converted there and cA[1 .. 3]
                // in step 0, two slots ahead of their MFMAs.
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    mf(cA, xa, q);
                    if (q < 2) xb[q] = rd_x(st, 1, q);
                    else if (q < 6) wr1[q - 2] = rd_w(st, 1, q - 2);
                    if (pf && (q & 1)) dma_to(s_dma, kt + 2, 0, q >> 1);
                    cvt1(wr0, 1, 2 * q, cB);
                    cvt1(wr0, 1, 2 * q + 1, cB);
                    if (q < 6) {
                        cvt1(wr0, 0, 4 + 2 * q, cA);
                        cvt1(wr0, 0, 5 + 2 * q, cA);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    mf(cB, xb, q);
                    if (q < 2) xa[q] = rd_x(st, 2, q);
                    if (pf && (q & 1)) dma_to(s_dma, kt + 2, 1, q >> 1);
                    cvt1(wr1, 0, 2 * q, cA);
                    cvt1(wr1, 0, 2 * q + 1, cA);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    mf(cA, xa, q);
                    if (q < 2) xb[q] = rd_x(st, 3, q);
                    cvt1(wr1, 1, 2 * q, cB);
                    cvt1(wr1, 1, 2 * q + 1, cB);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    mf(cB, xb, q);
                    if (more) {
                        if (q == 1) {
                            if (pf) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                            else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                        }
                        if (q >= 2 && q < 6) wr0[q - 2] = rd_w(nst, 0, q - 2);
                        else if (q >= 6) xa[q - 6] = rd_x(nst, 0, q - 6);
                        if (q >= 6) {
                            cvt1(wr0, 0, 2 * (q - 6), cA);
                            cvt1(wr0, 0, 2 * (q - 6) + 1, cA);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
            // k step 0: MFMAs (cA, xa); reads x step 1 -> xb, W pair 1 -> wr1; DMA part 0;
            // cB <- wr0 half 1
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                mf(cA, xa, q);
                if (q < 4) xb[q] = rd_x(st, 1, q);
                else if (q < 8) wr1[q - 4] = rd_w(st, 1, q - 4);
                if (pf && (q & 3) == 2) dma_to(s_dma, kt + 2, 0, q >> 2);
                cvt1(wr0, 1, q, cB);
                __builtin_amdgcn_sched_barrier(0);
            }
            // k step 1: MFMAs (cB, xb); reads x step 2 -> xa; DMA part 1; cA <- wr1 half 0
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                mf(cB, xb, q);
                if (q < 4) xa[q] = rd_x(st, 2, q);
                if (pf && (q & 3) == 2) dma_to(s_dma, kt + 2, 1, q >> 2);
                cvt1(wr1, 0, q, cA);
                __builtin_amdgcn_sched_barrier(0);
            }
            // k step 2: MFMAs (cA, xa); reads x step 3 -> xb; DMA part 2; cB <- wr1 half 1
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                mf(cA, xa, q);
                if (q < 4) xb[q] = rd_x(st, 3, q);
                if (pf && (q & 3) == 2) dma_to(s_dma, kt + 2, 2, q >> 2);
                cvt1(wr1, 1, q, cB);
                __builtin_amdgcn_sched_barrier(0);
            }
            // k step 3: MFMAs (cB, xb); after two of them the barrier that publishes the next
            // stage (this wave's DMAs for it have landed: at most the 12 of k tile kt + 2 are
            // outstanding), then the next tile's W pair 0 and x step 0, and its step-0
            // conversions in the second half
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                mf(cB, xb, q);
                if (more) {
                    if (q == 1) {
                        if (pf) asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    }
                    if (q >= 2 && q < 6) wr0[q - 2] = rd_w(nst, 0, q - 2);
                    else if (q >= 6 && q < 10) xa[q - 6] = rd_x(nst, 0, q - 6);
                    if (q >= 8) {
                        cvt1(wr0, 0, 2 * (q - 8), cA);
                        cvt1(wr0, 0, 2 * (q - 8) + 1, cA);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            }
            const uint32_t t = s_cur;
            s_cur = s_nxt;
            s_nxt = s_dma;
            s_dma = t;
        };
        int kt = kb;
        for (; kt + 2 < ke; ++kt) iter(kt, std::true_type{});
        for (; kt < ke; ++kt) iter(kt, std::false_type{});
        // every wave past its last LDS read before the stages are refilled
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    // Epilogue through LDS (free after the k loop): each lane rounds v = bf16(acc * s[n]) and
    // writes it to a bf16 copy of the tile (rows of 256 padded to 520 bytes, so that the 32 rows
    // of one 8-byte write fall in distinct banks); then every thread takes 16-byte row pieces,
    // applies relu^2 or adds the residual (both act on the rounded v, as the separate bf16 steps
    // do), and stores them: full 512-byte row runs per wave instead of 16-byte pieces of 32 rows.
    // Register r of lane l is n = 8 (r / 4) + 4 (l / 32) + r % 4, m = l % 32.
    constexpr int PITCH = 520;                      // bytes per staged row
    auto store = [&]() __attribute__((always_inline)) {
        // tiles wholly inside gN take the branch-free path (one uniform test)
        const bool inner = n0 + 256 <= gN;
        // the lane's 64 scales: one batch of loads (data-parallel form), or one batch per
        // 32-column block i (stream-K form, which has fewer registers to spare)
        constexpr int SB = SK ? 1 : TN;
        auto load_scales = [&](int i0, float (&sc)[SB][4][4]) {
            if (inner && gvs) {
#pragma unroll
                for (int i = 0; i < SB; ++i)
#pragma unroll
                    for (int gq = 0; gq < 4; ++gq) {
                        const float4 s4 =
                            *reinterpret_cast<const float4*>(gs + n0 + wn * 128 + (i0 + i) * 32 + 8 * gq + 4 * h);
                        sc[i][gq][0] = s4.x; sc[i][gq][1] = s4.y; sc[i][gq][2] = s4.z; sc[i][gq][3] = s4.w;
                    }
            } else {
#pragma unroll
                for (int i = 0; i < SB; ++i)
#pragma unroll
                    for (int gq = 0; gq < 4; ++gq)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            sc[i][gq][r] = gs[min(n0 + wn * 128 + (i0 + i) * 32 + 8 * gq + 4 * h + r, gN - 1)];
            }
        };
        float sc[SB][4][4];
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            if (i % SB == 0) load_scales(i, sc);
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const int nl = wn * 128 + i * 32 + 8 * gq + 4 * h;           // n within the tile
                const float* sg = sc[i % SB][gq];
#pragma unroll
                for (int j = 0; j < TM; ++j) {
                    const int ml = wm * (BM / 2) + j * 32 + l32;
                    const uint32_t lo = pack_bf16(acc[i][j][4 * gq + 0] * sg[0], acc[i][j][4 * gq + 1] * sg[1]);
                    const uint32_t hi = pack_bf16(acc[i][j][4 * gq + 2] * sg[2], acc[i][j][4 * gq + 3] * sg[3]);
                    *reinterpret_cast<uint2*>(lds + ml * PITCH + nl * 2) = uint2{lo, hi};
                }
            }
        }
        __syncthreads();
        // 32 threads per row (16 bytes = 8 columns each), 8 rows per pass of the workgroup,
        // eight passes per batch: the batch's LDS reads are issued before its stores
        const int c8 = (tid & 31) * 8;
        const int n = n0 + c8;
        const int rows = min(BM, M - m0);
        const bool full = gv16 && (inner || n + 7 < gN);
        const bool res16 = gepi == kEpiResidual && full && gv16r;
#pragma unroll
        for (int batch = 0; batch < BM / 64; ++batch) {
            uint32_t w[8][4];
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const int row = (tid >> 5) + 8 * (8 * batch + p);
                const uint2* src = reinterpret_cast<const uint2*>(lds + row * PITCH + c8 * 2);   // 8-byte aligned
                const uint2 v0 = src[0], v1 = src[1];
                w[p][0] = v0.x; w[p][1] = v0.y; w[p][2] = v1.x; w[p][3] = v1.y;
            }
            if (gepi == kEpiResidual) {
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    const int row = (tid >> 5) + 8 * (8 * batch + p);
                    if (row >= rows) continue;
                    const uint16_t* rp = gres + (int64_t)(m0 + row) * gldres + n;
                    uint32_t rv[4];
                    if (res16) {
                        const uint4 r4 = *reinterpret_cast<const uint4*>(rp);
                        rv[0] = r4.x; rv[1] = r4.y; rv[2] = r4.z; rv[3] = r4.w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            rv[e] = (n + 2 * e < gN ? (uint32_t)rp[2 * e] : 0u) |
                                    ((n + 2 * e + 1 < gN ? (uint32_t)rp[2 * e + 1] : 0u) << 16);
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[p][e] = add_bf16x2(w[p][e], rv[e]);
                }
            } else if (gepi == kEpiRelu2) {
#pragma unroll
                for (int p = 0; p < 8; ++p)
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[p][e] = relu2_bf16x2(w[p][e]);
            }
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const int row = (tid >> 5) + 8 * (8 * batch + p);
                if (row >= rows) continue;
                uint16_t* yp = gy + (int64_t)(m0 + row) * gldy + n;
                if (full) {
                    // streaming store: the tile's output is not read again by this launch
                    // (measured on MI355X: q|k|v at M = 2048 74.7 -> 73.3 us, down_proj 161 -> 159)
                    __builtin_nontemporal_store(u32x4{w[p][0], w[p][1], w[p][2], w[p][3]}, reinterpret_cast<u32x4*>(yp));
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (n + e < gN) yp[e] = (uint16_t)(w[p][e >> 1] >> (16 * (e & 1)));
                }
            }
        }
        __syncthreads();                            // the staging area is the next run's LDS
    };

    if constexpr (!SK) {
        // One tile per workgroup, XCD-ordered: workgroup g runs on XCD g % 8, which takes the
        // consecutive tiles [x * per_xcd, (x + 1) * per_xcd) in column-band order (m fastest),
        // so an XCD's tiles share few W column bands and less of W, the larger operand at
        // these shapes, is fetched into each XCD's L2 (measured +2.5% on up_proj and q|k|v
        // against n-fastest order).
        const int g = (int)blockIdx.x;
        const int local = g >> 3;
        const int tile = (g & 7) * a.per_xcd + local;
        if (local >= a.per_xcd || tile >= a.tiles_m * a.tiles_n) return;   // uniform
        int tm, tn;
        tile_coords(tile, a.tiles_m, a.tiles_n, a.gh, tm, tn);
        m0 = tm * BM;
        select(tn);
        zero_acc();
        run(0, KT);
        store();
    } else {
        // Stream-K as in the 8-wave kernel: per-XCD problems, each workgroup a contiguous range
        // of (tile, k tile) steps walked backwards; the workgroup holding a tile's last k tile
        // finishes it with the partials of the others (slot = their workgroup id).
        const int g = (int)blockIdx.x;
        const int Gx = (int)gridDim.x >> 3;
        const int xcd = g & 7, v = g >> 3;
        const int T = a.tiles_m * a.tiles_n;
        const int xb = xcd * T / 8, te = (xcd + 1) * T / 8;
        // The XCD's full rounds of tiles go one per workgroup, as in the data-parallel form;
        // only the tiles of its last, partly filled round are split (stream-K over [tb, te)).
        const int rounds = (te - xb) / Gx;
        for (int r = 0; r < rounds; ++r) {
            const int tile = xb + r * Gx + v;
            int tm, tn;
            tile_coords(tile, a.tiles_m, a.tiles_n, a.gh, tm, tn);
            m0 = tm * 256;
            select(tn);
            zero_acc();
            run(0, KT);
            store();
        }
        const int tb = xb + rounds * Gx;
        const int total = (te - tb) * KT;
        const int start = __builtin_amdgcn_readfirstlane((int)((int64_t)v * total / Gx));
        const int end = __builtin_amdgcn_readfirstlane((int)((int64_t)(v + 1) * total / Gx));
        for (int it = end; it > start;) {
            const int tl = __builtin_amdgcn_readfirstlane((it - 1) / KT);
            const int tile = tb + tl;
            const int t0 = tl * KT;
            const int kb = max(start, t0) - t0, ke = it - t0;
            int tm, tn;
            tile_coords(tile, a.tiles_m, a.tiles_n, a.gh, tm, tn);
            m0 = tm * 256;
            select(tn);
            zero_acc();
            run(kb, ke);
            if (ke == KT && kb > 0) {
                // finisher: add the partials of the local workgroups holding k tiles [0, kb), in
                // decreasing workgroup order, to this workgroup's own sum.  Each contributor wrote
                // that partial first (ranges are walked backwards) and this is the finisher's
                // last segment, so the flags are normally up.  (Adding before the own k tiles
                // forced the accumulators through scratch around the k loop.)
                const int first = __builtin_amdgcn_readfirstlane((int)(((int64_t)(t0 + 1) * Gx - 1) / total));
                for (int cv = v - 1; cv >= first; --cv) {
                    if ((int64_t)cv * total / Gx == (int64_t)(cv + 1) * total / Gx) continue;   // empty range
                    const int c = 8 * cv + xcd;
                    // Bounded wait for the contributor's flag: relaxed polls, then an agent-scope
                    // acquire fence (paired with the contributor's release exchange of the flag,
                    // it makes the partial visible to this thread and, through the barrier, to the
                    // workgroup).  At the limit the wait gives up unless the flag comes up in the
                    // same instant: it marks the slot abandoned (2) with a compare-exchange from 0,
                    // leaves the partial out and sets the workspace's and the device's error words
                    // -- the tile is wrong, the kernel exits, and the contributor, finding the mark
                    // when it raises its flag, lowers it again, so every flag ends the launch at 0.
                    if (tid == 0) {
                        bool up = false;
                        for (int spin = 0;; ++spin) {
                            if (__hip_atomic_load(a.sk_flags + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1u) {
                                up = true;
                                break;
                            }
                            if (spin >= a.sk_spin) break;
                            __builtin_amdgcn_s_sleep(1);
                        }
                        if (!up) {
                            uint32_t expect = 0u;
                            up = !__hip_atomic_compare_exchange_strong(a.sk_flags + c, &expect, 2u, __ATOMIC_RELAXED,
                                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                        if (up) {
                            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                        } else {
                            __hip_atomic_store(a.sk_error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            __hip_atomic_store(a.sk_host_error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        }
                        sk_up = up ? 1 : 0;
                    }
                    __syncthreads();
                    if (sk_up) {
                        // slot c: 8-byte piece p of thread t at (p * 256 + t) * 8 (2 KiB per piece)
                        uint64_t slot_off = (uint64_t)c * kDmaPartialBytes;
                        asm volatile("" : "+s"(slot_off));  // derived addresses computed here, not hoisted
                        const char* slot = reinterpret_cast<const char*>(a.sk_part) + slot_off;
                        // a row of TM blocks per batch: 32 loads in flight, four memory round trips
                        // for the partial (one per block measured ~30 us per finished tile)
#pragma unroll
                        for (int i = 0; i < TN; ++i) {
                            uint64_t pr[TM][8];
#pragma unroll
                            for (int j = 0; j < TM; ++j)
#pragma unroll
                                for (int r = 0; r < 8; ++r)
                                    pr[j][r] = __hip_atomic_load(
                                        reinterpret_cast<const uint64_t*>(slot + (size_t)((i * TM + j) * 8 + r) * NT * 8) +
                                            tid,
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                            for (int j = 0; j < TM; ++j)
#pragma unroll
                                for (int r = 0; r < 8; ++r) {
                                    acc[i][j][2 * r] += __uint_as_float((uint32_t)pr[j][r]);
                                    acc[i][j][2 * r + 1] += __uint_as_float((uint32_t)(pr[j][r] >> 32));
                                }
                        }
                        __syncthreads();                // slot c has been read: re-arm its flag
                        if (tid == 0) __hip_atomic_store(a.sk_flags + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
            if (ke < KT) {
                // contributor: partial tile to slot g, then the flag
                uint64_t slot_off = (uint64_t)g * kDmaPartialBytes;
                asm volatile("" : "+s"(slot_off));      // derived addresses computed here, not hoisted
                char* slot = reinterpret_cast<char*>(a.sk_part) + slot_off;
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) {
#pragma unroll
                        for (int r = 0; r < 16; r += 2) {
                            const uint64_t pr = (uint64_t)__float_as_uint(acc[i][j][r]) |
                                                ((uint64_t)__float_as_uint(acc[i][j][r + 1]) << 32);
                            __hip_atomic_store(
                                reinterpret_cast<uint64_t*>(slot + (size_t)((i * TM + j) * 8 + r / 2) * NT * 8) + tid, pr,
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    }
                __builtin_amdgcn_s_waitcnt(0);          // the partial's stores have completed
                __syncthreads();
                // release at agent scope: the workgroup's partial (ordered before this exchange by
                // the barrier) is visible to whoever acquires the flag.  A finisher that gave up
                // left the mark 2: lower the flag again (the finisher no longer looks at it).
                if (tid == 0) {
                    if (a.sk_lostflag) {
                        // tests: raise the flag only once the finisher has given up (bounded)
                        for (int spin = 0; spin < (1 << 22); ++spin) {
                            if (__hip_atomic_load(a.sk_flags + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 2u) break;
                            __builtin_amdgcn_s_sleep(1);
                        }
                    }
                    if (__hip_atomic_exchange(a.sk_flags + g, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == 2u)
                        __hip_atomic_store(a.sk_flags + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                store();
            }
            it = t0 + kb;
        }
    }
}
#undef gN
#undef gW
#undef gldw
#undef gs
#undef gy
#undef gldy
#undef gldres
#undef gres
#undef N
#undef gepi
#undef gvs
#undef gv16
#undef gv16r

// Stream-K workspace: the flag slots share the 64 KiB counter region of the skinny kernel's
// workspace layout (zero at rest in both; the last 4 bytes are the error word, NMI_WS_ERROR_OFFSET),
// then one fp32 partial tile per workgroup.
constexpr size_t kSkFlagBytes = 64 * 1024;
static_assert(kSkFlagBytes - 4 == NMI_WS_ERROR_OFFSET, "error word position");

// The 8-wave 32 x 32 MFMA kernel, one tile per workgroup.
template <int BM, int BN>
hipError_t launch_m32(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, const float* s, uint16_t* y,
                      int64_t ldy, int M, int N, int K, hipStream_t stream, const Epi& epi) {
    constexpr int NW = 8;
    constexpr size_t lds = 2 * (size_t)(BM + BN) * kBK * sizeof(uint16_t);
    constexpr auto kernel = &gemm_fp8_w8a16_m32_kernel<BM, BN, NW>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    GemmArgs a{};
    a.x = x; a.ldx = ldx; a.W = W; a.ldw = ldw; a.s = s; a.y = y; a.ldy = ldy;
    a.M = M; a.N = N; a.K = K; a.epi = epi;
    a.tiles_m = (M + BM - 1) / BM;
    a.tiles_n = (N + BN - 1) / BN;
    const int T = a.tiles_m * a.tiles_n;
    a.per_xcd = (T + 7) / 8;
    a.vec_store = ((reinterpret_cast<uintptr_t>(y) & 7) == 0 && (ldy & 3) == 0) ? 1 : 0;
    a.vec_res = ((reinterpret_cast<uintptr_t>(epi.res) & 7) == 0 && (epi.ldres & 3) == 0) ? 1 : 0;
    hipLaunchKernelGGL(kernel, dim3(8 * a.per_xcd), dim3(NW * 64), lds, stream, a);
    return hipGetLastError();
}

// Whether the DMA-fed kernel can take the operands (16-byte aligned DMA sources with 32-bit
// offsets, whole 64-wide k tiles).
bool dma_supported(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, int M, int N, int K) {
    return K % kBK == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(W) & 15) == 0 &&
           ldx % 8 == 0 && ldw % 16 == 0 && (int64_t)M * ldx * 2 < ((int64_t)1 << 31) &&
           (int64_t)N * ldw < ((int64_t)1 << 31);
}

// The DMA-fed kernel: one tile per workgroup, or stream-K over all CUs when the tiles cover at
// most half of them and the workspace holds the flags and one partial tile per workgroup
// (tuning knob gemm.sk: 1 forces stream-K where the workspace allows, 2 forbids it).
// Measured on MI355X (config 3, steady state): stream-K 950 vs 792 TFLOP/s on down_proj (104
// tiles), but 955 vs 1002 on up_proj (392 tiles) and 879 vs 1050 on qkv (224 tiles): with every
// CU busy the clock drops (~1.85 vs ~2.3 GHz with 104 busy) and the partial tiles cost traffic,
// so filling a partly idle last round does not pay.
// ng > 1: matrices sharing x in one launch (their column bands follow one another in the
// launch's tile numbering, each tile looks up its matrix).  Measured on MI355X: the attention
// block's q | k | v at S = 2048 (160 + 32 + 32 tiles) as one launch took the block 496 -> 380 us.
hipError_t launch_dma_groups(const uint16_t* x, int64_t ldx, const GemvGroup* g, int ng, int M, int K,
                             hipStream_t stream, void* ws, size_t ws_bytes) {
    constexpr int lds = kDmaStages * kDmaStage;
    constexpr int lds128 = kDmaStages * (256 * 64 + 128 * 128);
    static const hipError_t attr = [] {
        hipError_t e = hipSuccess;
        for (const void* k : {reinterpret_cast<const void*>(&gemm_fp8_w8a16_dma_kernel<false, false>),
                              reinterpret_cast<const void*>(&gemm_fp8_w8a16_dma_kernel<true, false>),
                              reinterpret_cast<const void*>(&gemm_fp8_w8a16_dma_kernel<false, true>),
                              reinterpret_cast<const void*>(&gemm_fp8_w8a16_dma_kernel<true, true>)})
            if (e == hipSuccess) e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        for (const void* k : {reinterpret_cast<const void*>(&gemm_fp8_w8a16_dma_kernel<false, false, 128>),
                              reinterpret_cast<const void*>(&gemm_fp8_w8a16_dma_kernel<false, true, 128>)})
            if (e == hipSuccess) e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, lds128);
        return e;
    }();
    if (attr != hipSuccess) return attr;
    if (ng < 1 || ng > kMaxGroups) return hipErrorInvalidValue;
    const bool grouped = ng > 1;
    const auto dp_kernel = grouped ? &gemm_fp8_w8a16_dma_kernel<false, true> : &gemm_fp8_w8a16_dma_kernel<false, false>;
    const auto sk_kernel = grouped ? &gemm_fp8_w8a16_dma_kernel<true, true> : &gemm_fp8_w8a16_dma_kernel<true, false>;
    GemmArgs a{};
    a.x = x; a.ldx = ldx;
    a.M = M; a.K = K;
    a.tiles_m = (M + 255) / 256;
    a.ngroups = ng;
    int tn = 0;
    for (int i = 0; i < ng; ++i) {
        const GemvGroup& G = g[i];
        const Epi& e = G.epi;
        a.grp[i] = GemmArgs::Group{G.W, G.ldw, G.s, G.y, G.ldy, e.kind == kEpiResidual ? e.res : nullptr, e.ldres, G.N, tn,
                                   e.kind,
                                   (reinterpret_cast<uintptr_t>(G.s) & 15) == 0 ? 1 : 0,
                                   ((reinterpret_cast<uintptr_t>(G.y) & 15) == 0 && (G.ldy & 7) == 0) ? 1 : 0,
                                   ((reinterpret_cast<uintptr_t>(e.res) & 15) == 0 && (e.ldres & 7) == 0) ? 1 : 0};
        tn += (G.N + 255) / 256;
    }
    a.tiles_n = tn;
    const int T = a.tiles_m * a.tiles_n;
    a.per_xcd = (T + 7) / 8;
    const int G = device_info().num_cu;             // one 144 KiB workgroup per CU
    const int gh_knob = tuning().gemm_gh;
    // 128 x 256 tiles where they finish sooner: with one workgroup per CU a grid of t tiles takes
    // ceil(t / CUs) rounds, and a 128-row tile costs 0.525 of a 256-row one (its MFMA rate measured
    // 4-5% lower: down_proj at M = 2048 1152 against 1208 TFLOP/s).  That takes them where the
    // 256-row tiles cover at most half the CUs -- each workgroup then has a whole tile with the
    // same MFMA work as half a tile of the stream-K form, without its partial-tile exchange:
    // down_proj at M = 2048 (208 tiles) 146.3 against 168.8 us in stream-K form, attention block at
    // S = 2048 250 against 296 us, Mamba block at S = 512 336 against 376 us -- and where the
    // 256-row tiles leave a short last round: the Mamba in_proj at M = 2048 (552 tiles, 3 rounds,
    // against 1104 in 5) took the block 531 -> 524 us.  Tuning knob gemm.bm: 128 forces them, 256
    // forbids them; gemm.sk = 1 keeps stream-K.
    const int bm_knob = tuning().gemm_bm;
    const int64_t T128 = (int64_t)((M + 127) / 128) * a.tiles_n;
    const bool short_tiles = 21 * ((T128 + G - 1) / G) < 40 * (((int64_t)T + G - 1) / G);
    if (bm_knob != 256 && tuning().gemm_sk != 1 && (bm_knob == 128 || short_tiles)) {
        const auto kernel128 =
            grouped ? &gemm_fp8_w8a16_dma_kernel<false, true, 128> : &gemm_fp8_w8a16_dma_kernel<false, false, 128>;
        a.tiles_m = (M + 127) / 128;
        const int T128 = a.tiles_m * a.tiles_n;
        a.per_xcd = (T128 + 7) / 8;
        a.gh = gh_knob > 0 ? std::min(gh_knob, a.tiles_m) : a.tiles_m;
        hipLaunchKernelGGL(kernel128, dim3(8 * a.per_xcd), dim3(256), lds128, stream, a);
        return hipGetLastError();
    }
    const bool fits = ws && ws_bytes >= kSkFlagBytes + (size_t)G * kDmaPartialBytes && G % 8 == 0 &&
                      G * 4 <= (int)kSkFlagBytes && (int64_t)T * (K / kBK) < ((int64_t)1 << 31);
    const int knob = tuning().gemm_sk;
    uint32_t* host_error = nullptr;
    if (fits && knob != 2 && (knob == 1 || 2 * (int64_t)T <= G) && (host_error = async_error_word()) != nullptr) {
        a.sk_host_error = host_error;
        a.gh = gh_knob > 0 ? std::min(gh_knob, a.tiles_m) : 1;
        a.sk_total = (int64_t)T * (K / kBK);
        a.sk_flags = static_cast<uint32_t*>(ws);
        a.sk_part = reinterpret_cast<float*>(static_cast<char*>(ws) + kSkFlagBytes);
        a.sk_error = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + NMI_WS_ERROR_OFFSET);
        a.sk_spin = tuning().gemm_sk_spin > 0 ? tuning().gemm_sk_spin : (1 << 26);
        a.sk_lostflag = tuning().gemm_sk_lostflag == 1 ? 1 : 0;
        // at most two workgroups per tile of an XCD (tuning knob gemm.sk_cap: another cap; -1: one
        // workgroup per CU).  Measured on MI355X: down_proj at M = 2048 (104 tiles) 174.7 -> 160.0
        // us; the attention block's k and v projections (32 tiles each, cut 8 ways on all CUs)
        // took the block 618 -> 496 us at S = 2048; caps of 3 and 4 in between.
        int gx = G / 8;
        const int cap = tuning().gemm_sk_cap == 0 ? 2 : tuning().gemm_sk_cap;
        if (cap > 0) gx = std::min(gx, (T + 7) / 8 * cap);
        hipLaunchKernelGGL(sk_kernel, dim3(8 * gx), dim3(256), lds, stream, a);
        return hipGetLastError();
    }
    a.gh = gh_knob > 0 ? std::min(gh_knob, a.tiles_m) : a.tiles_m;
    hipLaunchKernelGGL(dp_kernel, dim3(8 * a.per_xcd), dim3(256), lds, stream, a);
    return hipGetLastError();
}

hipError_t launch_dma(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, const float* s, uint16_t* y,
                      int64_t ldy, int M, int N, int K, hipStream_t stream, const Epi& epi, void* ws, size_t ws_bytes) {
    const GemvGroup g{W, ldw, s, y, ldy, N, 0, 0, epi};
    return launch_dma_groups(x, ldx, &g, 1, M, K, stream, ws, ws_bytes);
}

}  // namespace

namespace {
__global__ __launch_bounds__(256) void sk_flags_clear_kernel(uint4* __restrict__ flags) {
#pragma unroll
    for (int i = 0; i < (int)(kSkFlagBytes / 16 / 256); ++i) flags[i * 256 + threadIdx.x] = uint4{0u, 0u, 0u, 0u};
}
}  // namespace

// Zeroes the whole 64 KiB flag region (the stream-K flags and the error word) with one workgroup
// of 16-byte stores.
hipError_t launch_sk_flags_clear(void* ws, hipStream_t stream) {
    hipLaunchKernelGGL(sk_flags_clear_kernel, dim3(1), dim3(256), 0, stream, static_cast<uint4*>(ws));
    return hipGetLastError();
}

// Only the stream-K form uses a workspace, and it runs only under gemm.sk = 1 (or with the
// 128-row tiles forbidden, gemm.bm = 256): otherwise none, so that the blocks neither reserve
// its 64 MiB nor clear its flags.
size_t gemm_workspace_bytes(int M) {
    const Tuning& t = tuning();
    if (M < 512 || t.gemm_sk == 2 || (t.gemm_sk != 1 && t.gemm_bm != 256)) return 0;
    return kSkFlagBytes + (size_t)device_info().num_cu * kDmaPartialBytes;
}

// A grouped GEMM (matrices sharing x) as one launch of the DMA-fed kernel where it takes every
// matrix (M >= 512, automatic tile choice); otherwise one launch per matrix.
hipError_t launch_gemm_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* g, int ng,
                               hipStream_t stream, void* ws, size_t ws_bytes) {
    bool one = ng > 1 && M >= 512 && tuning().gemm_tile == 0;
    for (int i = 0; one && i < ng; ++i) one = dma_supported(x, ldx, g[i].W, g[i].ldw, M, g[i].N, K);
    if (one) return launch_dma_groups(x, ldx, g, ng, M, K, stream, ws, ws_bytes);
    hipError_t e = hipSuccess;
    for (int i = 0; i < ng && e == hipSuccess; ++i)
        e = launch_gemm(x, ldx, g[i].W, g[i].ldw, g[i].s, g[i].y, g[i].ldy, M, g[i].N, K, stream, g[i].epi, ws,
                        ws_bytes);
    return e;
}

hipError_t launch_gemm(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw,
                       const float* s, uint16_t* y, int64_t ldy, int M, int N, int K,
                       hipStream_t stream, const Epi& epi, void* ws, size_t ws_bytes) {
    int tile = tuning().gemm_tile;
    if (tile != 1 && tile != 2 && tile != 20 && tile != 21 && tile != 24) {
        // M < 512: the short-prompt kernel (gemm_short.hip) where it can take the operands, else
        // the 128 x 128 16 x 16 x 32 kernel; otherwise the DMA-fed 256 x 256 kernel where it can
        // take the operands, else the 8-wave 32 x 32 kernel with 256 x 256 tiles where they fill
        // at least 3/4 of the CUs, 256 x 128 below that.  (Measured on MI355X, config 3; the other
        // tile shapes and schedules tried -- 16 x 16 x 32 MFMA at 256-wide tiles, 64-bit LDS reads,
        // 4-wave forms, raised issue priority -- were slower.)
        const DeviceInfo& dev = device_info();
        const int64_t big = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
        if (M < 512) tile = gemm_short_supported(x, ldx, W, ldw, M, N, K) ? 2 : 1;
        else if (dma_supported(x, ldx, W, ldw, M, N, K)) tile = 24;
        else tile = (4 * big >= 3 * (int64_t)dev.num_cu) ? 20 : 21;
    }
    if (tile == 24 && !dma_supported(x, ldx, W, ldw, M, N, K)) tile = 20;
    if (tile == 2 && !gemm_short_supported(x, ldx, W, ldw, M, N, K)) tile = 1;
    switch (tile) {
        case 2: return launch_gemm_short(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 24: return launch_dma(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 20: return launch_m32<256, 256>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi);
        case 21: return launch_m32<256, 128>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi);
        default: {
            constexpr int BM = 128, BN = 128;
            const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
            hipLaunchKernelGGL((gemm_fp8_w8a16_kernel<BM, BN>), grid, dim3(256), 0, stream,
                               x, ldx, W, ldw, s, y, ldy, M, N, K, epi);
            return hipGetLastError();
        }
    }
}

}  // namespace nmi

