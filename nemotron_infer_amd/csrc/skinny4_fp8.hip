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
// * x [M, window] is staged per workgroup in LDS as [m][k group (4)][chunk] 8-byte words.
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
    GemvGroup g[kMaxGroups];
};

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x4 as_bf16x4(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(bf16x4, uint2{lo, hi});
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

template <int KS, int T, int U, int G>
hipError_t launch_cfg(Skinny4Args& a, hipStream_t stream) {
    constexpr int rows_per_wg = (kWaves / KS) * 4 * T;
    int wgs = 0;
    for (int i = 0; i < a.ngroups; ++i) {
        a.g[i].wg_begin = wgs;
        wgs += (a.g[i].N + rows_per_wg - 1) / rows_per_wg;
    }
    const size_t lds = ((size_t)a.M * 4 * a.xs_stride + 1) * sizeof(uint2);
    hipLaunchKernelGGL((skinny4_fp8_kernel<KS, T, U, G>), dim3(wgs), dim3(256), lds, stream, a);
    return hipGetLastError();
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
        default: return launch_g<KS, T, 8>(M, a, stream);
    }
}

template <int KS>
hipError_t launch_t(int t, int u, int M, Skinny4Args& a, hipStream_t stream) {
    return t == 2 ? launch_u<KS, 2>(u, M, a, stream) : launch_u<KS, 1>(u, M, a, stream);
}

}  // namespace

hipError_t launch_skinny4_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                                  int ngroups, hipStream_t stream) {
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
    // x window: 2 M w 16-byte pieces <= 2048 (8 per thread) and M x 32 w bytes <= 32 KiB.
    const int wmax = kStageBytes / (32 * M);
    a.window = C < wmax ? C : wmax;
    // (m, kg) rows padded to a stride of 2 mod 8 words: the 4 activation rows one read touches
    // start in different 64-byte bank groups.
    a.xs_stride = ((a.window + 5) & ~7) + 2;
    const Tuning& tn = tuning();
    // K split inside the workgroup so that a lane has 2-8 chunks per window; T = 2 when there
    // are enough rows to keep ~3 workgroups per CU.
    const int slice = a.window;
    int ks = slice >= 16 * 8 * 4 ? 4 : (slice >= 16 * 8 * 2 ? 2 : 1);
    if (tn.s4_ks == 1 || tn.s4_ks == 2 || tn.s4_ks == 4) ks = tn.s4_ks;
    const int64_t wg_t1 = (rows + (int64_t)(kWaves / ks) * 4 - 1) / ((int64_t)(kWaves / ks) * 4);
    int t = (wg_t1 >= 6 * (int64_t)dev.num_cu) ? 2 : 1;
    if (tn.s4_t == 1 || tn.s4_t == 2) t = tn.s4_t;
    const int per_lane = (slice / ks + 15) / 16;
    int u = per_lane <= 2 ? 2 : (per_lane <= 4 ? 4 : 8);
    if (tn.s4_u == 2 || tn.s4_u == 4 || tn.s4_u == 8) u = tn.s4_u;
    switch (ks) {
        case 1: return launch_t<1>(t, u, M, a, stream);
        case 2: return launch_t<2>(t, u, M, a, stream);
        default: return launch_t<4>(t, u, M, a, stream);
    }
}

}  // namespace nmi
