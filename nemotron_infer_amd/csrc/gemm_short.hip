// gemm_short.hip -- fp8-weight GEMM for short prompts (17 <= M < 512) on bf16 MFMA, gfx950.
//
//   y[m,n] = bf16_rne( (sum_k float(x[m,k]) * float(W[n,k])) * s[n] )   (+ relu^2 / residual)
//
// The reference runs these M through the same cuBLASLt fp8 GEMM as long prompts
// (nemotron_infer/csrc/include/ops/gemm.cuh:325-403).  Here short prompts get their own
// schedule: at M <= ~150 a linear is bound by its weight bytes (about 2M flop per byte, below
// MI355X's ~315 flop/B ridge), so the kernel is built to stream W at HBM rate while keeping the
// MFMA form of the large-tile kernel:
//
// * A workgroup owns BN = 128 TN weight rows (32 TN per wave) and BM = 32 TM rows of x; each wave
//   computes a 32 TN x BM block with v_mfma_f32_32x32x16_bf16 (W the A operand, x the B
//   operand).
// * W (raw e4m3 codes) and x (bf16) k tiles of 64 go global -> LDS by global_load_lds_dwordx4
//   (no register staging) through NS stages; NS - 1 k tiles are in flight while one is
//   multiplied, one barrier per k tile.  The codes are converted to bf16 with
//   v_cvt_scalef32_pk_bf16_fp8 (exact) as they are read from LDS.
// * K is split between workgroups when the tiles alone would leave the GPU short of loads in
//   flight: each split writes its float32 partial tile [M, N] to the workspace with plain
//   stores and a second kernel adds the splits in split order (deterministic), scales, rounds
//   and applies the epilogue.  The kernel boundary orders the partials: no flags, no waits.
//   Without a split the first kernel applies the epilogue itself.  The partials start after the
//   workspace's first 64 KiB: that region holds the counters and flags of the other kernels'
//   protocols (zero at rest, the error word at its end), which this kernel never touches.
// * LDS layouts as in the large-tile kernel: W rows of 64 B with chunk q at q ^ ((r >> 2) & 3),
//   x rows of 128 B with chunk c at c ^ ((r >> 1) & 7); the k order inside a tile is permuted
//   identically for both operands (k step s, lane half h, element e -> k = 32 (s / 2) + 16 h +
//   8 (s % 2) + e), so one 16-byte read of codes serves two k steps.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <algorithm>

namespace nmi {

namespace {

constexpr int kBK = 64;          // k per tile
constexpr int kWaves = 4;
constexpr size_t kFlagRegion = 64 * 1024;        // the workspace's counter / flag region, left alone

struct ShortArgs {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* W;
    int64_t ldw;
    const float* s;
    uint16_t* y;
    int64_t ldy;
    float* part;             // [splits][M][N] float32 (splits > 1)
    int M, N, K;
    int tiles_n, splits, kt_per;
    int part_vec;            // N % 4 == 0: 16-byte partial stores
    Epi epi;
};

// 16 bytes per lane from base + off to LDS [lds_addr + 16 lane] (LDS DMA).  Inline asm so that
// the compiler does not track the LDS write (it would wait for every outstanding DMA before any
// LDS read); completion is waited for with an explicit vmcnt before the barrier that publishes
// the stage.  m0 is set in the statement and listed as clobbered.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_addr)
                 : "memory", "m0");
}

// Waits until at most N of this wave's vector memory operations are outstanding, then the
// workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}
// wait_barrier<later * D>() for a run-time later in [0, L].
template <int D, int L>
__device__ __forceinline__ void wait_later(int later) {
    if constexpr (L == 0) {
        wait_barrier<0>();
    } else {
        if (later >= L) wait_barrier<L * D>();
        else wait_later<D, L - 1>(later);
    }
}

__device__ __forceinline__ int xswz(int row, int c) { return c ^ ((row >> 1) & 7); }
__device__ __forceinline__ int wswz(int row, int q) { return q ^ ((row >> 2) & 3); }

// The 4 waves form a WN x (4 / WN) grid; each wave computes TN 32-row blocks of W times TM
// 32-row blocks of x, so a workgroup covers BN = 32 TN WN weight rows and BM = 32 TM (4 / WN) x
// rows.  NS: LDS stages.
template <int TN, int TM, int WN, int NS, int OCC>
__global__ __launch_bounds__(256, OCC) void gemm_short_kernel(const ShortArgs a) {
    constexpr int WM = kWaves / WN;
    constexpr int BN = 32 * TN * WN, BM = 32 * TM * WM;
    constexpr int WI = BN / 16 / kWaves;            // W DMA instructions per wave per k tile
    constexpr int XI = BM / 8 / kWaves;             // x DMA instructions per wave per k tile
    static_assert(WI >= 1, "at least one W DMA per wave");
    constexpr int D = WI + XI;                      // DMA instructions per wave per k tile
    constexpr int WSTAGE = BN * kBK;
    constexpr int STAGE = WSTAGE + BM * kBK * 2;
    static_assert(XI >= 1, "at least one x DMA per wave");
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)lds;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, l32 = lane & 31;
    const int wn = wave % WN, wm = wave / WN;
    const int tn = (int)blockIdx.x / a.splits, sp = (int)blockIdx.x % a.splits;
    const int n0 = tn * BN, m0 = (int)blockIdx.y * BM;
    const int KT = a.K / kBK;
    const int kt0 = sp * a.kt_per, kt1 = min(KT, kt0 + a.kt_per);
    const int nk = kt1 - kt0;

    // DMA sources (byte offsets from the operand bases, k tile 0).  W instruction i: rows
    // (4 i + wave) * 16 + lane / 4; x instruction i: rows (4 i + wave) * 8 + lane / 8.  Rows
    // past N or M are clamped (their results are not stored).
    uint32_t woff[WI], xoff[XI];
#pragma unroll
    for (int i = 0; i < WI; ++i) {
        const int r = (4 * i + wave) * 16 + (lane >> 2);
        woff[i] = (uint32_t)(min(n0 + r, a.N - 1) * a.ldw + 16 * wswz(r, lane & 3));
    }
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int r = (4 * i + wave) * 8 + (lane >> 3);
        xoff[i] = (uint32_t)((min(m0 + r, a.M - 1) * a.ldx + 8 * xswz(r, lane & 7)) * 2);
    }
    auto issue = [&](int j) {                      // k tile kt0 + j into stage j % NS
        const uint32_t sb = lds0 + (uint32_t)((j % NS) * STAGE);
        const int kt = kt0 + j;
        const uint8_t* wb = a.W + (int64_t)kt * kBK;
        const uint8_t* xb = reinterpret_cast<const uint8_t*>(a.x) + (int64_t)kt * kBK * 2;
#pragma unroll
        for (int i = 0; i < WI; ++i) dma16(wb, woff[i], sb + (4 * i + wave) * 1024);
#pragma unroll
        for (int i = 0; i < XI; ++i) dma16(xb, xoff[i], sb + WSTAGE + (4 * i + wave) * 1024);
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int u = 0; u < TN; ++u)
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[u][t][r] = 0.f;

#pragma unroll
    for (int j = 0; j < NS - 1; ++j)
        if (j < nk) issue(j);

    for (int j = 0; j < nk; ++j) {
        // this wave's DMAs of k tile j have landed once at most min(NS - 2, nk - 1 - j) later
        // tiles' are outstanding; the barrier publishes every wave's and retires the reads of
        // the stage that the next issue overwrites
        wait_later<D, NS - 2>(min(NS - 2, nk - 1 - j));
        if (j + NS - 1 < nk) issue(j + NS - 1);
        const uint8_t* sw = lds + (j % NS) * STAGE;
        const uint8_t* sx = sw + WSTAGE;
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
            uint4 codes[TN];
#pragma unroll
            for (int u = 0; u < TN; ++u) {
                const int wr = (wn * TN + u) * 32 + l32;            // this lane's W row of block u
                codes[u] = *reinterpret_cast<const uint4*>(sw + wr * 64 + 16 * wswz(wr, 2 * jp + h));
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                bf16x8 af[TN];
#pragma unroll
                for (int u = 0; u < TN; ++u) {
                    const uint2 c0 = e4m3x4_to_bf16(half ? codes[u].z : codes[u].x);
                    const uint2 c1 = e4m3x4_to_bf16(half ? codes[u].w : codes[u].y);
                    af[u] = __builtin_bit_cast(bf16x8, uint4{c0.x, c0.y, c1.x, c1.y});
                }
                const int c = 4 * jp + 2 * h + half;
#pragma unroll
                for (int t = 0; t < TM; ++t) {
                    const int xr = (wm * TM + t) * 32 + l32;
                    const bf16x8 bf = *reinterpret_cast<const bf16x8*>(sx + xr * 128 + 16 * xswz(xr, c));
#pragma unroll
                    for (int u = 0; u < TN; ++u)
                        acc[u][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[u], bf, acc[u][t], 0, 0, 0);
                }
            }
        }
    }

    // Register r of lane l in block (u, t): n = n0 + 32 (TN wn + u) + 8 (r / 4) + 4 h + r % 4,
    // m = m0 + 32 (TM wm + t) + l32.
    if (a.splits > 1) {
        // partial tile of this split, raw sums (the reduce kernel scales)
        float* part = a.part + (size_t)sp * a.M * a.N;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int m = m0 + 32 * (TM * wm + t) + l32;
            if (m >= a.M) continue;
            float* row = part + (size_t)m * a.N;
#pragma unroll
            for (int u = 0; u < TN; ++u)
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    const int n = n0 + 32 * (TN * wn + u) + 4 * h + 8 * gq;
                    if (a.part_vec && n + 3 < a.N) {
                        *reinterpret_cast<float4*>(row + n) = float4{acc[u][t][4 * gq], acc[u][t][4 * gq + 1],
                                                                     acc[u][t][4 * gq + 2], acc[u][t][4 * gq + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < a.N) row[n + e] = acc[u][t][4 * gq + e];
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int u = 0; u < TN; ++u) {
        const int nb = n0 + 32 * (TN * wn + u) + 4 * h;
        float sc[4][4];
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[gq][e] = a.s[min(nb + 8 * gq + e, a.N - 1)];
        // residuals first (y may be the residual), then the stores
        uint16_t res[TM][4][4];
        if (a.epi.kind == kEpiResidual) {
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                const int m = min(m0 + 32 * (TM * wm + t) + l32, a.M - 1);
#pragma unroll
                for (int gq = 0; gq < 4; ++gq)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        res[t][gq][e] = a.epi.res[(int64_t)m * a.epi.ldres + min(nb + 8 * gq + e, a.N - 1)];
            }
        }
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int m = m0 + 32 * (TM * wm + t) + l32;
            if (m >= a.M) continue;
            uint16_t* yr = a.y + (int64_t)m * a.ldy;
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const int n = nb + 8 * gq;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < a.N)
                        yr[n + e] = epilogue(acc[u][t][4 * gq + e], sc[gq][e], a.epi.kind,
                                             a.epi.kind == kEpiResidual ? res[t][gq][e] : (uint16_t)0);
            }
        }
    }
}

// Sum of the splits' partials in split order, the scale, one rounding, the epilogue.  One
// thread per 4 consecutive outputs of a row (16-byte partial loads when N % 4 == 0); the partials
// of up to 8 splits are loaded before any is added (one memory round trip for them, not one per
// split), the scales and residuals before the partials.
__global__ __launch_bounds__(256) void gemm_short_reduce_kernel(const ShortArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int q_n = (a.N + 3) / 4;
    if (i >= (int64_t)a.M * q_n) return;
    const int m = (int)(i / q_n), n = 4 * (int)(i % q_n);
    const size_t stride = (size_t)a.M * a.N;
    const float* p = a.part + (size_t)m * a.N + n;
    const int cnt = min(4, a.N - n);
    float sc[4], v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) sc[e] = a.s[min(n + e, a.N - 1)];
    uint16_t r[4] = {0, 0, 0, 0};
    if (a.epi.kind == kEpiResidual)
        for (int e = 0; e < cnt; ++e) r[e] = a.epi.res[(int64_t)m * a.epi.ldres + n + e];
    if (a.part_vec) {
        for (int s0 = 0; s0 < a.splits; s0 += 8) {
            float4 f[8];
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (s0 + q < a.splits) f[q] = *reinterpret_cast<const float4*>(p + (size_t)(s0 + q) * stride);
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (s0 + q < a.splits) {
                    v[0] += f[q].x; v[1] += f[q].y; v[2] += f[q].z; v[3] += f[q].w;
                }
        }
    } else {
        for (int sp = 0; sp < a.splits; ++sp)
            for (int e = 0; e < cnt; ++e) v[e] += p[sp * stride + e];
    }
    uint16_t* yr = a.y + (int64_t)m * a.ldy + n;
    uint16_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = epilogue(v[e], sc[e], a.epi.kind, r[e]);
    if (cnt == 4 && (reinterpret_cast<uintptr_t>(yr) & 7) == 0) {
        *reinterpret_cast<uint2*>(yr) = uint2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
    } else {
        for (int e = 0; e < cnt; ++e) yr[e] = o[e];
    }
}

template <int TN, int TM, int WN, int NS, int OCC>
hipError_t launch_short_t(ShortArgs a, int tiles_m, hipStream_t stream) {
    constexpr int lds = NS * (32 * TN * WN * kBK + 32 * TM * (kWaves / WN) * kBK * 2);
    static_assert(lds * OCC <= 160 * 1024, "LDS of OCC workgroups per CU");
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_short_kernel<TN, TM, WN, NS, OCC>), hipFuncAttributeMaxDynamicSharedMemorySize,
        lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((gemm_short_kernel<TN, TM, WN, NS, OCC>), dim3(a.tiles_n * a.splits, tiles_m), dim3(256), lds,
                       stream, a);
    return hipGetLastError();
}

}  // namespace

bool gemm_short_supported(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, int M, int N, int K) {
    return M >= 1 && K % kBK == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(W) & 15) == 0 && ldx % 8 == 0 && ldw % 16 == 0 &&
           (int64_t)M * ldx * 2 < ((int64_t)1 << 31) && (int64_t)N * ldw < ((int64_t)1 << 31);
}

namespace {

// The kernel forms: W blocks per wave, x blocks per wave, waves along N (the rest along M), LDS
// stages, workgroups per CU.  Larger BN brings fewer x bytes along per weight byte (every
// workgroup reads its BM rows of x from L2) and fewer LDS reads per MFMA; smaller BN gives more
// workgroups without splitting K (whose partials cost 8 M bytes per weight row and split).
struct ShortCfg {
    int tn, tm, wn, ns, per_cu;
    int round;           // workgroups per CU that one round of the K split aims at
    int bn() const { return 32 * tn * wn; }
    int bm() const { return 32 * tm * (kWaves / wn); }
};
constexpr ShortCfg kForms[] = {
    {2, 1, 4, 7, 1, 1},   // 0: 256 x 32
    {1, 1, 4, 6, 2, 2},   // 1: 128 x 32
    {2, 2, 4, 6, 1, 1},   // 2: 256 x 64
    {1, 2, 4, 4, 2, 1},   // 3: 128 x 64
    {1, 1, 2, 6, 2, 2},   // 4: 64 x 64
    {2, 4, 4, 4, 1, 1},   // 5: 256 x 128
    {2, 2, 2, 4, 1, 1},   // 6: 128 x 128
    {1, 2, 2, 3, 2, 2},   // 7: 64 x 128
};
constexpr int kNumForms = sizeof(kForms) / sizeof(kForms[0]);

// The form for (M, N).  M <= 32: the widest of 256 x 32 and 128 x 32 whose tiles fill three
// quarters of the workgroup slots without a K split, else 128 x 32 (then K is split).  33 <= M
// <= 64: 128 x 64 with K split to about one workgroup per CU -- the best of every form and split
// count on each config-3 shape in a sweep (up / down / q|k|v at M = 64 19.7 / 17.7 / 14.2 us
// against 23.4 / 20.6 / 15.6 for 64 x 64 tiles split to two per CU).  Above M = 64 the 128 x 128
// form with a 64 x 64 block per wave (fewest LDS reads per MFMA; best or within 1% of the best at
// M = 128 and 256).  Tuning knob gemm.short = f + 1 forces form f.
int short_form(int M, int N) {
    const int forced = tuning().gemm_short;
    if (forced >= 1 && forced <= kNumForms) return forced - 1;
    int lo, hi;                                     // candidate forms, widest first
    if (M <= 32) { lo = 0; hi = 1; }
    else if (M <= 64) return 3;
    else { lo = 6; hi = 6; }
    const int cu = device_info().num_cu;
    for (int f = lo; f <= hi; ++f) {
        const ShortCfg& c = kForms[f];
        const int64_t tiles = (int64_t)((N + c.bn() - 1) / c.bn()) * ((M + c.bm() - 1) / c.bm());
        if (4 * tiles >= 3 * (int64_t)c.per_cu * cu) return f;
    }
    return hi;
}

}  // namespace

int gemm_short_splits(int M, int N, int K) {
    const ShortCfg& c = kForms[short_form(M, N)];
    const int bn = c.bn(), bm = c.bm();
    const int tiles = ((N + bn - 1) / bn) * ((M + bm - 1) / bm);
    const int KT = K / kBK;
    if (tuning().gemm_splits > 0) return std::min(tuning().gemm_splits, KT);
    // one round of the form's target workgroups per CU, at least 4 k tiles each, and the partials
    // (4 M bytes per weight row and split, written and read back) at most the weight bytes
    const int want = std::max(1, c.round * device_info().num_cu / tiles);
    const int by_k = std::max(1, KT / 4);
    const int by_bytes = std::max(1, (int)((int64_t)K / (4 * (int64_t)M)));
    return std::max(1, std::min(want, std::min(by_k, by_bytes)));
}

// Enough for any N' <= N (grouped launches share one workspace): splits x N' is at most
// min(splits by k and bytes) x N, and the one-round limit keeps it below the rows one round of
// workgroups covers.
size_t gemm_short_workspace_bytes(int M, int N, int K) {
    if (M < 1 || N < 1 || K < kBK) return 0;
    const int KT = K / kBK;
    int64_t rows;
    if (tuning().gemm_splits > 0) {
        const int sp = std::min(tuning().gemm_splits, KT);
        if (sp <= 1) return 0;
        rows = (int64_t)sp * N;
    } else {
        const int64_t cap = std::max(1, std::min(KT / 4, (int)((int64_t)K / (4 * (int64_t)M))));
        if (cap <= 1) return 0;
        // over the forms M can take: at most the rows one round of workgroups covers
        int64_t round_rows = 0;
        for (const ShortCfg& c : kForms) round_rows = std::max<int64_t>(round_rows, (int64_t)c.per_cu * c.bn());
        rows = std::min<int64_t>(cap * N, round_rows * device_info().num_cu);
    }
    return kFlagRegion + (size_t)rows * M * sizeof(float);
}

hipError_t launch_gemm_short(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw, const float* s,
                             uint16_t* y, int64_t ldy, int M, int N, int K, hipStream_t stream, const Epi& epi,
                             void* ws, size_t ws_bytes) {
    const int form = short_form(M, N);
    const ShortCfg& c = kForms[form];
    ShortArgs a{};
    a.x = x; a.ldx = ldx; a.W = W; a.ldw = ldw; a.s = s; a.y = y; a.ldy = ldy;
    a.M = M; a.N = N; a.K = K; a.epi = epi;
    a.tiles_n = (N + c.bn() - 1) / c.bn();
    const int KT = K / kBK;
    int splits = gemm_short_splits(M, N, K);
    if (splits > 1 && (!ws || ws_bytes < kFlagRegion + (size_t)splits * M * N * sizeof(float))) splits = 1;
    a.kt_per = (KT + splits - 1) / splits;
    a.splits = (KT + a.kt_per - 1) / a.kt_per;      // no empty split
    a.part = splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + kFlagRegion) : nullptr;
    a.part_vec = N % 4 == 0 ? 1 : 0;
    const int tiles_m = (M + c.bm() - 1) / c.bm();
    hipError_t e;
    switch (form) {
        case 0: e = launch_short_t<2, 1, 4, 7, 1>(a, tiles_m, stream); break;
        case 1: e = launch_short_t<1, 1, 4, 6, 2>(a, tiles_m, stream); break;
        case 2: e = launch_short_t<2, 2, 4, 6, 1>(a, tiles_m, stream); break;
        case 3: e = launch_short_t<1, 2, 4, 4, 2>(a, tiles_m, stream); break;
        case 4: e = launch_short_t<1, 1, 2, 6, 2>(a, tiles_m, stream); break;
        case 5: e = launch_short_t<2, 4, 4, 4, 1>(a, tiles_m, stream); break;
        case 6: e = launch_short_t<2, 2, 2, 4, 1>(a, tiles_m, stream); break;
        default: e = launch_short_t<1, 2, 2, 3, 2>(a, tiles_m, stream); break;
    }
    if (e != hipSuccess || a.splits == 1) return e;
    const int64_t n4 = (int64_t)M * ((N + 3) / 4);
    hipLaunchKernelGGL(gemm_short_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace nmi
