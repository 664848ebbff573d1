// rmsnorm.hip -- RMSNorm of bf16 activation rows for gfx950 (the normalisation that opens
// every fp8 block: model/mlp_block.cuh:140, attention_block.cuh and mamba_block.cuh alike;
// reference kernel ops/reduce.cuh:135-244).
//
//   y[m, k] = bf16_rne(x[m, k] * (r_m * w[k])),  r_m = 1 / sqrt(sum_k x[m, k]^2 / K + eps)
//
// One 256-thread workgroup per row.  Thread t owns the 16-byte pieces t, t + 256, ... (8
// activations each); its float32 sum of squares runs over them in that order (sumsq8), then
// the wave sum (16-lane DPP rows, then (r0 + r1) + (r2 + r3)), then the four waves
// (0 + 1) + (2 + 3).  The GEMV kernel's fused form (NORM in gemv_fp8.hip) uses the same
// pieces and order, so the two give bit-identical activations.  Used where the first linear
// of a block does not run on the GEMV kernel (M > 2), and by tests.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

__global__ __launch_bounds__(256) void rmsnorm_bf16_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           const float* __restrict__ w, float eps,
                                                           uint16_t* __restrict__ y, int64_t ldy, int K) {
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int pieces = K >> 3;
    const uint16_t* __restrict__ xr = x + (int64_t)blockIdx.x * ldx;
    uint16_t* __restrict__ yr = y + (int64_t)blockIdx.x * ldy;

    float ss = 0.f;
    for (int e = tid; e < pieces; e += 256) ss = sumsq8(load16(xr + (int64_t)e * 8), ss);
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float r = rms_factor((red[0] + red[1]) + (red[2] + red[3]), K, eps);
    for (int e = tid; e < pieces; e += 256) {
        const uint4 v = load16(xr + (int64_t)e * 8);
        const float4 g0 = *reinterpret_cast<const float4*>(w + (int64_t)e * 8);
        const float4 g1 = *reinterpret_cast<const float4*>(w + (int64_t)e * 8 + 4);
        *reinterpret_cast<uint4*>(yr + (int64_t)e * 8) = rms_scale8(v, g0, g1, r);
    }
}

}  // namespace

hipError_t launch_rmsnorm(const uint16_t* x, int64_t ldx, const Norm& norm, uint16_t* y, int64_t ldy,
                          int M, int K, hipStream_t stream) {
    if (M < 1 || K < 8 || K % 8 != 0 || !norm.w) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_bf16_kernel, dim3(M), dim3(256), 0, stream, x, ldx, norm.w, norm.eps, y, ldy, K);
    return hipGetLastError();
}

}  // namespace nmi
