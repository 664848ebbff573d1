// noalloc.hip -- nmi_mlp_forward_fp8_noalloc: the fp8 MLP block with no allocation at all.
//
// nmi_mlp_forward_fp8 needs transient device memory: the relu^2 activations [M, inter] and, for
// M > 2, the RMSNorm-ed input [M, hidden].  It takes them from a caller workspace or, without
// one, from the bump allocator, which may hipMalloc a slab.  Callers that cannot allocate (code
// under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc) use this entry
// point instead: the transient buffers live in `scratch`, a file-scope device array of
// kNoAllocScratchBytes that every GPU the library runs on holds until the process ends.  For
// 17 <= M < 512 the block's GEMMs run without their K split here (its partials would not fit),
// so results equal nmi_mlp_forward_fp8's up to float32 summation order there, and bit for bit
// at every other M (and with tuning knob gemm.splits = 1).
//
// Host code never passes `scratch` itself (its name is a host-side stand-in, not a device
// address): the first call on a device, with that device current, resolves the array's address
// on that device with hipGetSymbolAddress and keeps it per device.  The block's kernels fully
// write these buffers before reading them, so nothing in the array needs clearing between calls.
// Every call on a GPU shares that GPU's array: calls that may overlap in time on one GPU (other
// streams) race on it.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "nmi_fp8_linear.h"
#include "nmi_launch.hpp"

namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;     // 4 MiB on every device
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// The array's address on the current device (resolved once per device).
hipError_t scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return hipSuccess;
}

}  // namespace

extern "C" {

size_t nmi_mlp_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int nmi_mlp_forward_fp8_noalloc(const void* input_bf16, const float* norm_w, const void* up_w_e4m3,
                                const float* up_scale, const void* down_w_e4m3, const float* down_scale,
                                void* out_bf16, int M, int hidden, int inter, float eps, void* stream) {
    const char* fn = "nmi_mlp_forward_fp8_noalloc";
    const size_t need = nmi::mlp_workspace_bytes(M, hidden, inter, false);
    if (need == 0) {
        nmi::set_last_error("%s: M=%d hidden=%d inter=%d (need M >= 1, hidden and inter >= 16)", fn, M, hidden,
                            inter);
        return NMI_ERR_INVALID_ARG;
    }
    if (need > kNoAllocScratchBytes) {
        nmi::set_last_error("%s: M=%d hidden=%d inter=%d needs %zu bytes of transient buffers, more than the "
                            "%zu-byte scratch array (at hidden = 3136, inter = 12544: M <= 133)",
                            fn, M, hidden, inter, need, kNoAllocScratchBytes);
        return NMI_ERR_WORKSPACE;
    }
    void* ptr = nullptr;
    const hipError_t e = scratch_ptr(&ptr);
    if (e != hipSuccess) {
        nmi::set_last_error("%s: hipGetSymbolAddress of the scratch array: %s (hipError %d)", fn,
                            hipGetErrorString(e), (int)e);
        return (int)e;
    }
    return nmi::mlp_forward_fp8(input_bf16, norm_w, up_w_e4m3, up_scale, down_w_e4m3, down_scale, out_bf16, M, hidden,
                                inter, eps, ptr, kNoAllocScratchBytes, stream, false, fn);
}

}  // extern "C"
