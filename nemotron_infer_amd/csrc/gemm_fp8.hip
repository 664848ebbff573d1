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
#include "nmi_device.hpp"
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
    int vec_store;          // y 8-byte aligned and ldy % 4 == 0
    int vec_res;            // residual 8-byte aligned and ldres % 4 == 0
    Epi epi;
    // Stream-K (m32 kernels): sk_total = tiles * K steps (0: one tile per workgroup); the
    // workspace's flag slots (zero at rest) and fp32 partial tiles, one per workgroup.
    int64_t sk_total;
    uint32_t* sk_flags;
    float* sk_part;
};

template <int BM, int BN>
__global__ __launch_bounds__(256, 1) void gemm_fp8_w8a16_big_kernel(const GemmArgs a) {
    constexpr int BK = kBK;
    constexpr int WTM = BM / 2, WTN = BN / 2;      // wave tile (m x n)
    constexpr int TM = WTM / 16, TN = WTN / 16;    // 16 x 16 MFMA tiles per wave
    constexpr int XP = BM * (BK / 8) / 256;        // 16-byte x pieces per thread per K step
    constexpr int WP = BN * (BK / 16) / 256;       // 16-byte W pieces per thread per K step
    constexpr int STAGE = (BM + BN) * BK;          // bf16 elements per LDS stage
    static_assert(XP >= 1 && WP >= 1, "tile too small for 256 threads");
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];

    const int g = (int)blockIdx.x;
    const int local = g >> 3;
    const int tile = (g & 7) * a.per_xcd + local;
    if (local >= a.per_xcd || tile >= a.tiles_m * a.tiles_n) return;   // uniform
    const int tm = tile / a.tiles_n;
    const int tn = tile - tm * a.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = a.M, N = a.N, K = a.K;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wn = wave & 1, wm = wave >> 1;

    uint4 rx[XP], rw[WP];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int p = tid + 256 * i;
            const int row = p >> 3, kc = p & 7;
            const int gm = min(m0 + row, M - 1), gk = min(k0 + kc * 8, K - 8);
            rx[i] = load16(a.x + (int64_t)gm * a.ldx + gk);
        }
#pragma unroll
        for (int i = 0; i < WP; ++i) {
            const int p = tid + 256 * i;
            const int row = p >> 2, kc = p & 3;
            const int gn = min(n0 + row, N - 1), gk = min(k0 + kc * 16, K - 16);
            rw[i] = load16(a.W + (int64_t)gn * a.ldw + gk);
        }
    };
    auto sstore = [&](int buf, int k0) {
        uint16_t* Ws = lds + buf * STAGE;
        uint16_t* Xs = Ws + BN * BK;
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int p = tid + 256 * i;
            const int row = p >> 3, kc = p & 7;
            const uint4 v = (k0 + kc * 8 < K) ? rx[i] : uint4{0, 0, 0, 0};
            *reinterpret_cast<uint4*>(Xs + row * BK + (swz(row, kc) << 3)) = v;
        }
#pragma unroll
        for (int i = 0; i < WP; ++i) {
            const int p = tid + 256 * i;
            const int row = p >> 2, kc = p & 3;
            const uint4 w = (k0 + kc * 16 < K) ? rw[i] : uint4{0, 0, 0, 0};
            const uint2 d0 = e4m3x4_to_bf16(w.x), d1 = e4m3x4_to_bf16(w.y);
            const uint2 d2 = e4m3x4_to_bf16(w.z), d3 = e4m3x4_to_bf16(w.w);
            const int c0 = 2 * kc, c1 = 2 * kc + 1;
            *reinterpret_cast<uint4*>(Ws + row * BK + (swz(row, c0) << 3)) = uint4{d0.x, d0.y, d1.x, d1.y};
            *reinterpret_cast<uint4*>(Ws + row * BK + (swz(row, c1) << 3)) = uint4{d2.x, d2.y, d3.x, d3.y};
        }
    };

    f32x4 acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int KT = (K + BK - 1) / BK;
    gload(0);
    sstore(0, 0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
        const uint16_t* Ws = lds + buf * STAGE;
        const uint16_t* Xs = Ws + BN * BK;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int chunk = ks * 4 + (lane >> 4);
            bf16x8 af[TN], bfr[TM];
#pragma unroll
            for (int i = 0; i < TN; ++i) {
                const int row = wn * WTN + i * 16 + (lane & 15);
                af[i] = *reinterpret_cast<const bf16x8*>(Ws + row * BK + (swz(row, chunk) << 3));
            }
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int row = wm * WTM + j * 16 + (lane & 15);
                bfr[j] = *reinterpret_cast<const bf16x8*>(Xs + row * BK + (swz(row, chunk) << 3));
            }
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(buf ^ 1, (kt + 1) * BK);
        __syncthreads();
    }

    // Epilogue: lane holds D[n = 4 (lane / 16) + r][m = lane % 16] of each 16 x 16 tile.
    // Residuals are loaded (clamped in bounds) before the first store.
    uint2 rres[TN][TM];
    if (a.epi.kind == kEpiResidual) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int n = n0 + wn * WTN + i * 16 + 4 * (lane >> 4);
                const int m = min(m0 + wm * WTM + j * 16 + (lane & 15), M - 1);
                const int64_t row = (int64_t)m * a.epi.ldres;
                rres[i][j] = load_res4(a.epi.res, row + min(n, N - 1), row + N - 1, a.vec_res && n + 3 < N);
            }
    }
#pragma unroll
    for (int i = 0; i < TN; ++i) {
        const int n = n0 + wn * WTN + i * 16 + 4 * (lane >> 4);
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = a.s[min(n + r, N - 1)];
        const bool full = a.vec_store && (n + 3 < N);
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int m = m0 + wm * WTM + j * 16 + (lane & 15);
            if (m >= M) continue;
            uint16_t* yp = a.y + (int64_t)m * a.ldy + n;
            const uint2 rv = rres[i][j];
            const uint16_t b0 = epilogue(acc[i][j][0], sc[0], a.epi.kind, (uint16_t)rv.x);
            const uint16_t b1 = epilogue(acc[i][j][1], sc[1], a.epi.kind, (uint16_t)(rv.x >> 16));
            const uint16_t b2 = epilogue(acc[i][j][2], sc[2], a.epi.kind, (uint16_t)rv.y);
            const uint16_t b3 = epilogue(acc[i][j][3], sc[3], a.epi.kind, (uint16_t)(rv.y >> 16));
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

// ---------------------------------------------------------------------------------------
// 32 x 32 x 16 MFMA variant of the large-tile kernel: the same tiles, LDS layout, XCD order
// and epilogue, but v_mfma_f32_32x32x16_bf16 (half the fragment registers per k step of the
// 16 x 16 x 32 form), with the fragments of k step s+1 read from LDS while the MFMAs of
// step s run (two fragment register sets).  Operand layouts (gfx950): A lane l holds row
// l % 32, k 8 (l / 32) .. +7; B lane l holds column l % 32, the same k; D register r of lane l
// is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
// PIPE: 0 the next tile's LDS stores after the MFMAs; 1 between the MFMA groups; 2 also each
// group's fragment reads interleaved one by one with the previous group's MFMAs; 3 as 2 with the
// wave's issue priority raised while it issues MFMAs.
template <int BM, int BN, int NW, bool B64, int PIPE, bool SK>
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
    // LDS tile layouts.  B64 = false: rows of eight 16-byte chunks, chunk c of row r at
    // swz(r, c).  B64 = true: the low and high 8 bytes of every chunk in two planes of
    // 64-byte rows, chunk c of row r at c ^ ((r >> 2) & 7), so that fragments are read with
    // ds_read_b64 (measured on MI355X: ~1.6x the LDS read throughput of ds_read_b128) and
    // the 32 rows one read touches fall in distinct banks.
    auto put16 = [&](uint16_t* T, int rows, int row, int c, uint4 v) {
        if constexpr (B64) {
            const int off = row * 32 + ((c ^ ((row >> 2) & 7)) << 2);          // in bf16 elements
            *reinterpret_cast<uint2*>(T + off) = uint2{v.x, v.y};
            *reinterpret_cast<uint2*>(T + rows * 32 + off) = uint2{v.z, v.w};
        } else {
            *reinterpret_cast<uint4*>(T + row * BK + (swz(row, c) << 3)) = v;
        }
    };
    auto get16 = [&](const uint16_t* T, int rows, int row, int c) -> bf16x8 {
        if constexpr (B64) {
            const int off = row * 32 + ((c ^ ((row >> 2) & 7)) << 2);
            const uint2 lo = *reinterpret_cast<const uint2*>(T + off);
            const uint2 hi = *reinterpret_cast<const uint2*>(T + rows * 32 + off);
            typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
            return __builtin_bit_cast(bf16x8, u32x4_t{lo.x, lo.y, hi.x, hi.y});
        } else {
            return *reinterpret_cast<const bf16x8*>(T + row * BK + (swz(row, c) << 3));
        }
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
        if constexpr (PIPE) {
            // The next tile's LDS stage (buf ^ 1) was last read before the previous barrier, so
            // its stores go between this tile's MFMA groups: the matrix cores keep working
            // while the x tile and the converted W tile are written.
            static_assert(BK / 16 == 4, "four k steps per tile");
            // fragment reads of the next k step, then the MFMAs of this one (independent)
            auto step = [&](int s_next, bf16x8 (&afn)[TN], bf16x8 (&bfn)[TM], const bf16x8 (&af)[TN],
                            const bf16x8 (&bfr)[TM]) {
                frags(buf, s_next, afn, bfn);
                if constexpr (PIPE >= 3) __builtin_amdgcn_s_setprio(1);
                mfmas(af, bfr);
                if constexpr (PIPE >= 3) __builtin_amdgcn_s_setprio(0);
                if constexpr (PIPE >= 2) {
#pragma unroll
                    for (int q = 0; q < TN + TM; ++q) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // one LDS read
                    }
                    __builtin_amdgcn_sched_group_barrier(0x008, TN * TM - (TN + TM), 0);
                }
            };
            if constexpr (PIPE >= 2) {
                // k steps 0-2 with the reads of steps 1-3 under them; then k step 3 in two halves
                // (m rows j < TM/2, then the rest) with the x stores before the first and the
                // converted W stores before the second.
                static_assert(TM % 2 == 0, "k step 3 is split along m");
                step(1, af1, bf1, af0, bf0);
                step(2, af0, bf0, af1, bf1);
                step(3, af1, bf1, af0, bf0);
                if (more) sstore_x(buf ^ 1, (kt + 1) * BK);
                if constexpr (PIPE >= 3) __builtin_amdgcn_s_setprio(1);
                mfmas_half(af1, bf1, 0);
                if constexpr (PIPE >= 3) __builtin_amdgcn_s_setprio(0);
                if (more) sstore_w(buf ^ 1, (kt + 1) * BK);
                if constexpr (PIPE >= 3) __builtin_amdgcn_s_setprio(1);
                mfmas_half(af1, bf1, 1);
                if constexpr (PIPE >= 3) __builtin_amdgcn_s_setprio(0);
            } else {
                frags(buf, 1, af1, bf1);
                mfmas(af0, bf0);
                frags(buf, 2, af0, bf0);
                mfmas(af1, bf1);
                frags(buf, 3, af1, bf1);
                if (more) sstore_x(buf ^ 1, (kt + 1) * BK);
                mfmas(af0, bf0);
                if (more) sstore_w(buf ^ 1, (kt + 1) * BK);
                mfmas(af1, bf1);
            }
        } else {
#pragma unroll
            for (int s = 0; s < BK / 16; s += 2) {
                frags(buf, s + 1, af1, bf1);
                mfmas(af0, bf0);
                if (s + 2 < BK / 16) frags(buf, s + 2, af0, bf0);
                mfmas(af1, bf1);
            }
            if (more) sstore(buf ^ 1, (kt + 1) * BK);
        }
        __syncthreads();
        if (more) frags(buf ^ 1, 0, af0, bf0);
    }
    };

    // Epilogue: register r of lane l is n = 8 (r / 4) + 4 (l / 32) + r % 4, m = l % 32.
    // Residuals are loaded (clamped in bounds) before the first store.
    auto store = [&]() {
    uint2 rres[TN][4][TM];
    if (!SK && a.epi.kind == kEpiResidual) {     // (the stream-K kernel is not used with a residual)
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

    if constexpr (!SK) {
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
    } else {

    // Stream-K, one independent problem per XCD: workgroup g runs on XCD x = g % 8, which
    // owns the consecutive tiles [x T / 8, (x + 1) T / 8).  Their K steps, flattened
    // tile-major, are split evenly between the XCD's Gx = G / 8 workgroups: local workgroup
    // v = g / 8 owns [v total / Gx, (v + 1) total / Gx).  A tile cut between workgroups is
    // finished by the one holding its last K step: the others store fp32 partial tiles (slot =
    // their workgroup id) and raise a flag; the finisher starts from the partials, added in
    // decreasing workgroup order, then runs its own K steps and stores the output.  Each workgroup walks its range backwards, so its
    // partial (the head of its last tile) is written first and the tile it finishes (the tail of
    // its first) comes last.  A finisher only waits for workgroups g - 8, g - 16, ..., which are
    // dispatched before it and never wait on it: no co-residency is needed for progress.
    constexpr int ACC = TN * TM * 16;               // fp32 accumulators per thread
    // (All of this is wave-uniform and kept in scalar registers: the 256 x 256 kernel has no
    // vector registers to spare.  tiles * K steps < 2^31 is checked on the host.)
    const int g = (int)blockIdx.x;
    const int Gx = (int)gridDim.x >> 3;
    const int xcd = g & 7, v = g >> 3;
    const int T = a.tiles_m * a.tiles_n;
    const int tb = xcd * T / 8, te = (xcd + 1) * T / 8;
    const int total = (te - tb) * KT;
    const int start = __builtin_amdgcn_readfirstlane((int)((int64_t)v * total / Gx));
    const int end = __builtin_amdgcn_readfirstlane((int)((int64_t)(v + 1) * total / Gx));
    for (int it = end; it > start;) {
        const int tl = __builtin_amdgcn_readfirstlane((it - 1) / KT);     // tile within the XCD's range
        const int tile = tb + tl;
        const int t0 = tl * KT;
        const int kb = max(start, t0) - t0, ke = it - t0;
        const int tm = tile / a.tiles_n;
        m0 = tm * BM;
        n0 = (tile - tm * a.tiles_n) * BN;
        zero_acc();
        if (ke == KT && kb > 0) {
            // finisher: start from the partials of the local workgroups holding K steps
            // [0, kb), added in decreasing workgroup order, before this workgroup's own steps
            const int first = __builtin_amdgcn_readfirstlane((int)(((int64_t)(t0 + 1) * Gx - 1) / total));
            for (int cv = v - 1; cv >= first; --cv) {
                if ((int64_t)cv * total / Gx == (int64_t)(cv + 1) * total / Gx) continue;   // empty range
                const int c = 8 * cv + xcd;             // their workgroup id
                if (tid == 0) {
                    // bounded wait: the bound turns a lost flag into a wrong tile, not a hang
                    for (int spin = 0; spin < (1 << 26); ++spin) {
                        if (__hip_atomic_load(a.sk_flags + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1u)
                            break;
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
                __syncthreads();
                const uint64_t* part =
                    reinterpret_cast<const uint64_t*>(a.sk_part) + (size_t)c * (ACC / 2) * NT + tid;
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) {
                        uint64_t pr[8];
#pragma unroll
                        for (int r = 0; r < 8; ++r)
                            pr[r] = __hip_atomic_load(part + (size_t)((i * TM + j) * 8 + r) * NT, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                        for (int r = 0; r < 8; ++r) {
                            acc[i][j][2 * r] += __uint_as_float((uint32_t)pr[r]);
                            acc[i][j][2 * r + 1] += __uint_as_float((uint32_t)(pr[r] >> 32));
                        }
                    }
                __syncthreads();                        // slot c has been read: re-arm its flag
                if (tid == 0) __hip_atomic_store(a.sk_flags + c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        run(kb, ke);
        if (ke < KT) {
            // contributor (this workgroup's last K steps): partial tile to slot g, then the flag
            uint64_t* part = reinterpret_cast<uint64_t*>(a.sk_part) + (size_t)g * (ACC / 2) * NT + tid;
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j) {
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        const uint64_t pr = (uint64_t)__float_as_uint(acc[i][j][r]) |
                                            ((uint64_t)__float_as_uint(acc[i][j][r + 1]) << 32);
                        __hip_atomic_store(part + (size_t)(((i * TM + j) * 16 + r) / 2) * NT, pr, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    }
                    __builtin_amdgcn_sched_barrier(0);    // one 32 x 32 tile at a time (registers)
                }
            __builtin_amdgcn_s_waitcnt(0);              // the partial's stores have completed
            __syncthreads();
            if (tid == 0) __hip_atomic_store(a.sk_flags + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            store();
        }
        it = t0 + kb;
        __syncthreads();
    }
    }
}

// Stream-K workspace: the flag slots share the 64 KiB counter region of the skinny kernel's
// workspace layout (zero at rest in both), then one fp32 partial tile per workgroup.
constexpr size_t kSkFlagBytes = 64 * 1024;

template <int BM, int BN, int NW>
constexpr size_t sk_partial_bytes() {
    constexpr int WGN = NW == 8 ? 4 : 2;
    return (size_t)NW * 64 * ((BM / 2 / 32) * (BN / WGN / 32) * 16) * sizeof(float);
}

// sk: use the stream-K form when the workspace allows (tuning knob gemm.sk: 1 forces it, 2
// forbids it).
template <int BM, int BN, bool M32, int NW = 4, bool B64 = false, int PIPE = 0>
hipError_t launch_big(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, const float* s,
                      uint16_t* y, int64_t ldy, int M, int N, int K, hipStream_t stream, const Epi& epi,
                      void* ws, size_t ws_bytes, bool sk = false) {
    constexpr size_t lds = 2 * (size_t)(BM + BN) * kBK * sizeof(uint16_t);
    constexpr auto kernel =
        M32 ? &gemm_fp8_w8a16_m32_kernel<BM, BN, NW, B64, PIPE, false> : &gemm_fp8_w8a16_big_kernel<BM, BN>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    GemmArgs a{x, ldx, W, ldw, s, y, ldy, M, N, K, 0, 0, 0, 0, 0, epi, 0, nullptr, nullptr};
    a.tiles_m = (M + BM - 1) / BM;
    a.tiles_n = (N + BN - 1) / BN;
    const int T = a.tiles_m * a.tiles_n;
    a.per_xcd = (T + 7) / 8;
    a.vec_store = ((reinterpret_cast<uintptr_t>(y) & 7) == 0 && (ldy & 3) == 0) ? 1 : 0;
    a.vec_res = ((reinterpret_cast<uintptr_t>(epi.res) & 7) == 0 && (epi.ldres & 3) == 0) ? 1 : 0;
    if constexpr (M32 && PIPE != 0) {
        constexpr auto sk_kernel = &gemm_fp8_w8a16_m32_kernel<BM, BN, NW, B64, PIPE, true>;
        static const hipError_t sk_attr = hipFuncSetAttribute(reinterpret_cast<const void*>(sk_kernel),
                                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (sk_attr != hipSuccess) return sk_attr;
        static const int occ = [] {
            int o = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, reinterpret_cast<const void*>(sk_kernel), NW * 64,
                                                             lds) != hipSuccess ||
                o < 1)
                o = 1;
            return o;
        }();
        const int G = device_info().num_cu * occ;
        const int knob = tuning().gemm_sk;
        const bool fits = ws && ws_bytes >= kSkFlagBytes + (size_t)G * sk_partial_bytes<BM, BN, NW>() && G % 8 == 0 &&
                          G * 4 <= (int)kSkFlagBytes && (int64_t)T * ((K + kBK - 1) / kBK) < ((int64_t)1 << 31);
        if (fits && epi.kind != kEpiResidual && knob != 2 && (knob == 1 || sk)) {
            a.sk_total = (int64_t)T * ((K + kBK - 1) / kBK);
            a.sk_flags = static_cast<uint32_t*>(ws);
            a.sk_part = reinterpret_cast<float*>(static_cast<char*>(ws) + kSkFlagBytes);
            hipLaunchKernelGGL(sk_kernel, dim3(G), dim3(NW * 64), lds, stream, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL(kernel, dim3(8 * a.per_xcd), dim3(M32 ? NW * 64 : 256), lds, stream, a);
    return hipGetLastError();
}

}  // namespace

size_t gemm_workspace_bytes(int M) {
    if (M < 512 || tuning().gemm_sk != 1) return 0;
    return kSkFlagBytes + (size_t)device_info().num_cu * sk_partial_bytes<256, 256, 8>();
}

hipError_t launch_gemm(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw,
                       const float* s, uint16_t* y, int64_t ldy, int M, int N, int K,
                       hipStream_t stream, const Epi& epi, void* ws, size_t ws_bytes) {
    int tile = tuning().gemm_tile;
    if (tile < 1 || tile > 23) {
        // Measured on MI355X (config 3, steady state): the pipelined 8-wave kernels (32 x 32
        // MFMA, the next tile's LDS stores between the MFMA groups, each group's fragment reads
        // interleaved with the previous group's MFMAs: +2% over clustered); 256 x 256 tiles where there
        // are at least 3/4 as many as CUs (up_proj 392, qkv 224), else 256 x 128 (down_proj,
        // N = 3136: 104 tiles of 256 x 256); 128 x 128 for small M.  The stream-K form (knob
        // gemm.sk = 1) fills the idle CUs of a partial last round but measured no faster: the GEMM
        // runs power-limited (~1.5 GHz under load), so idle CUs cost less than they seem.
        const DeviceInfo& dev = device_info();
        const int64_t big = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
        if (M < 512) tile = 1;
        else tile = (4 * big >= 3 * (int64_t)dev.num_cu) ? 20 : 21;
    }
    switch (tile) {
        case 2: return launch_big<256, 256, false>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 3: return launch_big<256, 128, false>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 4: return launch_big<128, 256, false>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 5: return launch_big<256, 256, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 6: return launch_big<256, 128, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 7: return launch_big<128, 256, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 8: return launch_big<256, 256, true, 8>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 9: return launch_big<256, 128, true, 8>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 10: return launch_big<256, 256, true, 4, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 11: return launch_big<256, 256, true, 8, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 12: return launch_big<256, 128, true, 8, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 13: return launch_big<256, 128, true, 4, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 14: return launch_big<256, 256, true, 8, false, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 15: return launch_big<256, 128, true, 8, false, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 16: return launch_big<256, 256, true, 8, true, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 17: return launch_big<256, 128, true, 8, true, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 18: return launch_big<256, 256, true, 4, false, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 19: return launch_big<256, 128, true, 4, false, true>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 20: return launch_big<256, 256, true, 8, false, 2>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 21: return launch_big<256, 128, true, 8, false, 2>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 22: return launch_big<256, 256, true, 8, false, 3>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
        case 23: return launch_big<256, 128, true, 8, false, 3>(x, ldx, W, ldw, s, y, ldy, M, N, K, stream, epi, ws, ws_bytes);
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

