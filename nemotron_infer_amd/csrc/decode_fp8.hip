// decode_fp8.hip -- device-side e4m3 decode through the kernels' own conversion helpers.
//
// Test entry for the 256-code bit-exact check: every code goes through e4m3x4_to_bf16
// (v_cvt_scalef32_pk_bf16_fp8, the decode of every GEMV and MFMA kernel here), with the code at
// each of the four byte positions of a dword as the kernels see it; out_f32 is that bf16 value
// widened (exact).  out_scaled = decode * scale is the float32 product of the reference's GEMV
// epilogue (ops/gemv.cuh:87-88).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

__global__ __launch_bounds__(256) void decode_e4m3_kernel(const uint32_t* __restrict__ codes,
                                                          float* __restrict__ out_f32,
                                                          float* __restrict__ out_scaled,
                                                          uint16_t* __restrict__ out_bf16,
                                                          float scale, int nwords) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nwords) return;
    const uint32_t w = codes[i];
    const uint2 b = e4m3x4_to_bf16(w);
    const float4 f{bf16lo_to_f32(b.x), bf16hi_to_f32(b.x), bf16lo_to_f32(b.y), bf16hi_to_f32(b.y)};
    reinterpret_cast<float4*>(out_f32)[i] = f;
    reinterpret_cast<float4*>(out_scaled)[i] = float4{f.x * scale, f.y * scale, f.z * scale, f.w * scale};
    reinterpret_cast<uint2*>(out_bf16)[i] = b;
}

}  // namespace

hipError_t launch_decode(const uint8_t* codes, float* out_f32, float* out_scaled,
                         uint16_t* out_bf16, float scale, int n, hipStream_t stream) {
    const int nwords = n / 4;
    const dim3 grid((nwords + 255) / 256);
    hipLaunchKernelGGL(decode_e4m3_kernel, grid, dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(codes), out_f32, out_scaled, out_bf16,
                       scale, nwords);
    return hipGetLastError();
}

}  // namespace nmi
