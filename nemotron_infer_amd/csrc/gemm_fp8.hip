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
// * LDS rows are 64 bf16 (eight 16-byte chunks); chunk c of row r is stored at c ^ (r & 7),
//   which spreads the 16 rows an MFMA operand read touches over all banks.
// * Epilogue: acc * s[n] in float32, one bf16 RNE rounding, masked for ragged M and N.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kBK = 64;

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_fp8_w8a16_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ W, int64_t ldw,
    const float* __restrict__ s, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K) {
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
            *reinterpret_cast<uint4*>(A + row * kBK + ((kc ^ (row & 7)) << 3)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int id = tid + 256 * i;
            const int row = id >> 2, kc = id & 3;
            const uint2 d0 = e4m3x4_to_bf16(rb[i].x), d1 = e4m3x4_to_bf16(rb[i].y);
            const uint2 d2 = e4m3x4_to_bf16(rb[i].z), d3 = e4m3x4_to_bf16(rb[i].w);
            const int c0 = 2 * kc, c1 = 2 * kc + 1;
            *reinterpret_cast<uint4*>(B + row * kBK + ((c0 ^ (row & 7)) << 3)) = uint4{d0.x, d0.y, d1.x, d1.y};
            *reinterpret_cast<uint4*>(B + row * kBK + ((c1 ^ (row & 7)) << 3)) = uint4{d2.x, d2.y, d3.x, d3.y};
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
                af[i] = *reinterpret_cast<const bf16x8*>(A + row * kBK + ((chunk ^ (row & 7)) << 3));
            }
#pragma unroll
            for (int jn = 0; jn < TN; ++jn) {
                const int row = wn * WN + jn * 16 + (lane & 15);
                bfr[jn] = *reinterpret_cast<const bf16x8*>(B + row * kBK + ((chunk ^ (row & 7)) << 3));
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

    // Epilogue: lane holds D[(lane>>4)*4 + t][lane & 15] of each 16x16 tile.
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
                if (m < M) y[(int64_t)m * ldy + n] = f32_to_bf16_rne(acc[i][jn][t] * sc);
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw,
                       const float* s, uint16_t* y, int64_t ldy, int M, int N, int K,
                       hipStream_t stream) {
    constexpr int BM = 128, BN = 128;
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL((gemm_fp8_w8a16_kernel<BM, BN>), grid, dim3(256), 0, stream,
                       x, ldx, W, ldw, s, y, ldy, M, N, K);
    return hipGetLastError();
}

}  // namespace nmi

