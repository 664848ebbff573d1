// nmi_launch.hpp -- host-side launchers of the gfx950 kernels (internal to libnmi.so).
//
// The C ABI (capi.cpp) validates arguments, then calls these.  Each launcher assumes its
// arguments were validated (shapes, strides, alignment) and returns the hipError_t of the
// launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nmi {

struct DeviceInfo {
    int device = -1;
    int num_cu = 256;
    int num_xcd = 8;
};

// Records the calling thread's last error message (returned by nmi_last_error()).
void set_last_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// Per-device properties, queried once per device (thread-safe).
const DeviceInfo& device_info();

// Tuning knobs (0 = automatic).  Set through nmi_tuning_set() for sweeps; never needed for
// correctness.
struct Tuning {
    int gemv_ks = 0;       // waves of a workgroup that split K: 1, 2 or 4
    int gemv_unroll = 0;   // 16-byte weight loads in flight per lane: 4, 8 or 16
    int gemm_tile = 0;     // GEMM tile variant id (see gemm_fp8.hip)
    int skinny_ks = 0;     // skinny-M kernel: waves of a workgroup that split K
};
Tuning& tuning();

hipError_t launch_gemv_m1(const uint16_t* x, const uint8_t* W, int64_t ldw, const float* s,
                          uint16_t* y, int N, int K, hipStream_t stream);

hipError_t launch_gemv_skinny(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw,
                              const float* s, uint16_t* y, int64_t ldy, int M, int N, int K,
                              hipStream_t stream);

hipError_t launch_gemm(const uint16_t* x, int64_t ldx, const uint8_t* W, int64_t ldw,
                       const float* s, uint16_t* y, int64_t ldy, int M, int N, int K,
                       hipStream_t stream);

hipError_t launch_decode(const uint8_t* codes, float* out_f32, float* out_scaled,
                         uint16_t* out_bf16, float scale, int n, hipStream_t stream);

}  // namespace nmi
