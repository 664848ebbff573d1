// gemv_fp8.hip -- M = 1 fp8 (OCP e4m3) W8A16 GEMV for gfx950.
//
//   y[n] = bf16_rne( (sum_k float(W[n,k]) * float(x[k])) * s[n] )
//
// Same result contract as the reference's gemv_fp8_kernel
// (nemotron_infer/csrc/include/ops/gemv.cuh:48-89, formula :19-20, epilogue :87-88); the
// schedule is designed for CDNA4 instead:
//
// * Wave64, one DPP row (16 lanes) per weight row: a wave covers 4 rows, a workgroup of
//   4 waves covers 16 / 8 / 4 rows when KS = 1 / 2 / 4 of its waves split K between them.
//   Lane j of a row reads the 16-byte chunks j, j+16, j+32, ... of that row, so one load
//   instruction of a wave fetches 4 rows x 256 contiguous bytes.
// * UNROLL 16-byte non-temporal loads per lane are issued before any of them is consumed
//   (memory-level parallelism: the kernel is HBM-bound, 2 flop per weight byte).
// * x is staged once per workgroup in LDS as float32, quarter-major (float4 quarter p of
//   chunk c at [p][c]) so that the 16 lanes of a row read 16 consecutive float4 -- no bank
//   conflicts -- and the 4 rows of a wave share them by broadcast.  K is processed in LDS
//   windows of at most 1008 chunks (63 KiB).
// * e4m3 -> f32 with v_cvt_pk_f32_fp8, float32 FMA accumulation, a DPP 16-lane reduction,
//   then (KS > 1) an ordered sum of the K-slice partials through LDS, and the per-row scale
//   and the single bf16 RNE rounding in the epilogue.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kWaves = 4;
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerWave = 64 / kLanesPerRow;
constexpr int kMaxWindowChunks = 1008;   // 1008 chunks * 64 B = 63 KiB, + the static partials < 64 KiB

__device__ __forceinline__ float dot16(const uint4 w, const float* __restrict__ xq,
                                       int qstride, float acc) {
    // xq points at quarter 0 of the chunk; quarter p lives at xq + p * qstride.
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const f32x4 wf = e4m3x4_to_f32(words[p]);
        const float4 xv = *reinterpret_cast<const float4*>(xq + p * qstride);
        acc = __builtin_fmaf(wf.x, xv.x, acc);
        acc = __builtin_fmaf(wf.y, xv.y, acc);
        acc = __builtin_fmaf(wf.z, xv.z, acc);
        acc = __builtin_fmaf(wf.w, xv.w, acc);
    }
    return acc;
}

template <int KS, int UNROLL>
__global__ __launch_bounds__(256) void gemv_fp8_m1_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ W, int64_t ldw,
    const float* __restrict__ s, uint16_t* __restrict__ y, int N, int K, int window_chunks) {
    extern __shared__ float xs[];                       // [4][window_chunks][4] floats
    constexpr int kRowGroups = kWaves / KS;
    constexpr int kRowsPerWG = kRowGroups * kRowsPerWave;
    __shared__ float partial[KS > 1 ? KS : 1][kRowsPerWG];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane >> 4;                // row within the wave
    const int j = lane & 15;                // lane within the row
    const int g = wave / KS;                // row group of this wave
    const int q = wave % KS;                // K slice of this wave
    const int row = blockIdx.x * kRowsPerWG + g * kRowsPerWave + r;
    const bool active = row < N;
    const uint8_t* __restrict__ wrow = W + (int64_t)(active ? row : 0) * ldw;
    const int C = K >> 4;                   // 16-byte chunks per row
    const int qstride = window_chunks * 4;  // floats between quarters

    float acc = 0.f;
    for (int w0 = 0; w0 < C; w0 += window_chunks) {
        const int wc = min(window_chunks, C - w0);
        if (w0 != 0) __syncthreads();       // previous window fully consumed
        // Stage x[w0*16 : (w0+wc)*16) as float32; each thread converts 8 bf16 (half a chunk).
        for (int e = tid; e < wc * 2; e += 256) {
            const uint4 v = load16(x + (int64_t)(w0 * 16 + e * 8));
            const int c = e >> 1, h = e & 1;
            float* dst0 = xs + (2 * h) * qstride + c * 4;
            float* dst1 = xs + (2 * h + 1) * qstride + c * 4;
            *reinterpret_cast<float4*>(dst0) =
                float4{bf16lo_to_f32(v.x), bf16hi_to_f32(v.x), bf16lo_to_f32(v.y), bf16hi_to_f32(v.y)};
            *reinterpret_cast<float4*>(dst1) =
                float4{bf16lo_to_f32(v.z), bf16hi_to_f32(v.z), bf16lo_to_f32(v.w), bf16hi_to_f32(v.w)};
        }
        __syncthreads();

        const int cb = (q * wc) / KS;
        const int ce = ((q + 1) * wc) / KS;
        if (active) {
            const uint8_t* __restrict__ wwin = wrow + (int64_t)w0 * 16;
            for (int c0 = cb + j; c0 < ce; c0 += UNROLL * kLanesPerRow) {
                uint4 wv[UNROLL];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    const int c = c0 + u * kLanesPerRow;
                    wv[u] = (c < ce) ? load_stream16(wwin + (int64_t)c * 16) : uint4{0, 0, 0, 0};
                }
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    const int c = c0 + u * kLanesPerRow;
                    if (c < ce) acc = dot16(wv[u], xs + c * 4, qstride, acc);
                }
            }
        }
    }

    acc = dpp_row_sum16(acc);
    if constexpr (KS == 1) {
        if (active && j == 0) y[row] = f32_to_bf16_rne(acc * s[row]);
    } else {
        if (j == 0) partial[q][g * kRowsPerWave + r] = acc;
        __syncthreads();
        if (q == 0 && j == 0 && active) {
            float t = partial[0][g * kRowsPerWave + r];
#pragma unroll
            for (int qq = 1; qq < KS; ++qq) t += partial[qq][g * kRowsPerWave + r];
            y[row] = f32_to_bf16_rne(t * s[row]);
        }
    }
}

template <int KS, int UNROLL>
hipError_t launch_ks(const uint16_t* x, const uint8_t* W, int64_t ldw, const float* s,
                     uint16_t* y, int N, int K, hipStream_t stream) {
    constexpr int rows_per_wg = (kWaves / KS) * kRowsPerWave;
    const int C = K >> 4;
    const int window = C < kMaxWindowChunks ? C : kMaxWindowChunks;
    const dim3 grid((N + rows_per_wg - 1) / rows_per_wg);
    const size_t lds = (size_t)window * 16 * sizeof(float);
    hipLaunchKernelGGL((gemv_fp8_m1_kernel<KS, UNROLL>), grid, dim3(256), lds, stream,
                       x, W, ldw, s, y, N, K, window);
    return hipGetLastError();
}

template <int UNROLL>
hipError_t launch_unroll(int ks, const uint16_t* x, const uint8_t* W, int64_t ldw,
                         const float* s, uint16_t* y, int N, int K, hipStream_t stream) {
    switch (ks) {
        case 1: return launch_ks<1, UNROLL>(x, W, ldw, s, y, N, K, stream);
        case 2: return launch_ks<2, UNROLL>(x, W, ldw, s, y, N, K, stream);
        default: return launch_ks<4, UNROLL>(x, W, ldw, s, y, N, K, stream);
    }
}

}  // namespace

hipError_t launch_gemv_m1(const uint16_t* x, const uint8_t* W, int64_t ldw, const float* s,
                          uint16_t* y, int N, int K, hipStream_t stream) {
    const DeviceInfo& dev = device_info();
    // Fewest K-splitting waves that still give every CU at least two workgroups.
    int ks = tuning().gemv_ks;
    if (ks != 1 && ks != 2 && ks != 4) {
        const int target = 2 * dev.num_cu;
        ks = 4;
        for (int cand : {1, 2, 4}) {
            const int rows_per_wg = (kWaves / cand) * kRowsPerWave;
            if ((N + rows_per_wg - 1) / rows_per_wg >= target) { ks = cand; break; }
        }
    }
    switch (tuning().gemv_unroll) {
        case 4: return launch_unroll<4>(ks, x, W, ldw, s, y, N, K, stream);
        case 16: return launch_unroll<16>(ks, x, W, ldw, s, y, N, K, stream);
        default: return launch_unroll<8>(ks, x, W, ldw, s, y, N, K, stream);
    }
}

}  // namespace nmi
