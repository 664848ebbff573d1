// block.cpp -- extern "C" entries of the fp8 block layer above the linear: the RMSNorm and
// the MLP block (declared in include/nmi_fp8_linear.h).
//
// The reference's MLP block (nemotron_infer/csrc/include/model/mlp_block.cuh:121-176) runs at
// M = 1 five launches over four bump-allocated buffers: rmsnorm_bf16 -> normed, gemv_fp8 ->
// up, relu^2 -> act, gemv_fp8 -> down, residual add -> out.  Here the element-wise steps
// ride on the linears: relu^2 and the residual add are output epilogues of the up and down
// projections, and where the up projection runs on the GEMV kernel (M = 1, and M = 2 where the
// 16x16x32 skinny kernel does not take it) the RMSNorm is applied while that kernel stages its
// activations -- two launches and one [M, inter] buffer.  Otherwise the RMSNorm is its own
// launch (rmsnorm.hip) into a second buffer.  On the GEMM
// path (M > 16) the workspace also holds the GEMMs' region: below M = 512 the short-prompt
// kernel's K-split partials (which need no initialisation); from M = 512 nothing unless the
// stream-K form is forced (tuning knob gemm.sk = 1 or gemm.bm = 256), whose flags and partial
// tiles one small kernel zeroes at the start of every call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "nmi_fp8_linear.h"
#include "nmi_launch.hpp"

using namespace nmi;

namespace {

int fail(int code, const char* msg) {
    set_last_error("%s", msg);
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return NMI_OK;
    set_last_error("%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
    return (int)e;
}

int fail2(int code, const char* fn, const char* msg) {
    set_last_error("%s: %s", fn, msg);
    return code;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace layout: the prefill GEMM's stream-K region (M >= 512: flags, then partial tiles),
// act [M, inter] bf16, then normed [M, hidden] bf16 when the RMSNorm is not fused into the up
// projection.
bool norm_fused(int M, int hidden) { return gemv_fuses_norm(M, hidden); }

// split = false leaves the short-prompt GEMMs unsplit (no partial region): the allocation-free
// form, whose buffers must fit a fixed array
size_t gemm_region(int M, int hidden, int inter, bool split) {
    if (choose_path(M) != Path::Gemm || (!split && !gemm_workspace_has_flags(M))) return 0;
    return round256(std::max(linear_workspace_bytes(M, inter, hidden), linear_workspace_bytes(M, hidden, inter)));
}

size_t mlp_bytes(int M, int hidden, int inter, bool split) {
    size_t b = gemm_region(M, hidden, inter, split) + round256((size_t)M * inter * 2);
    if (!norm_fused(M, hidden)) b += round256((size_t)M * hidden * 2);
    return b;
}

}  // namespace

extern "C" {

int nmi_rmsnorm_bf16(const void* x_bf16, const float* w, void* y_bf16, int M, int K, float eps, void* stream) {
    const char* fn = "nmi_rmsnorm_bf16";
    if (!x_bf16 || !w || !y_bf16) return fail(NMI_ERR_INVALID_ARG, "nmi_rmsnorm_bf16: NULL pointer argument");
    if (M < 1 || K < 8 || K % 8 != 0) {
        set_last_error("%s: M=%d K=%d (need M >= 1, K a positive multiple of 8)", fn, M, K);
        return NMI_ERR_INVALID_ARG;
    }
    if (!aligned(x_bf16, 16) || !aligned(y_bf16, 16) || !aligned(w, 16))
        return fail(NMI_ERR_ALIGNMENT, "nmi_rmsnorm_bf16: x, y and w must be 16-byte aligned");
    return hip_status(launch_rmsnorm(static_cast<const uint16_t*>(x_bf16), K, Norm{w, eps},
                                     static_cast<uint16_t*>(y_bf16), K, M, K, static_cast<hipStream_t>(stream)),
                      fn);
}

size_t nmi_mlp_workspace_bytes(int M, int hidden, int inter) {
    if (M < 1 || hidden < 16 || inter < 16) return 0;
    return mlp_bytes(M, hidden, inter, true);
}

int nmi_mlp_forward_fp8(const void* input_bf16, const float* norm_w, const void* up_w_e4m3, const float* up_scale,
                        const void* down_w_e4m3, const float* down_scale, void* out_bf16, int M, int hidden,
                        int inter, float eps, void* workspace, size_t workspace_bytes, void* stream) {
    return mlp_forward_fp8(input_bf16, norm_w, up_w_e4m3, up_scale, down_w_e4m3, down_scale, out_bf16, M, hidden,
                           inter, eps, workspace, workspace_bytes, stream, true, "nmi_mlp_forward_fp8");
}

}  // extern "C"

namespace nmi {

size_t mlp_workspace_bytes(int M, int hidden, int inter, bool split) {
    if (M < 1 || hidden < 16 || inter < 16) return 0;
    return mlp_bytes(M, hidden, inter, split);
}

int mlp_forward_fp8(const void* input_bf16, const float* norm_w, const void* up_w_e4m3, const float* up_scale,
                    const void* down_w_e4m3, const float* down_scale, void* out_bf16, int M, int hidden, int inter,
                    float eps, void* workspace, size_t workspace_bytes, void* stream, bool split, const char* fn) {
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    if (!input_bf16 || !norm_w || !up_w_e4m3 || !up_scale || !down_w_e4m3 || !down_scale || !out_bf16)
        return fail2(NMI_ERR_INVALID_ARG, fn, "NULL pointer argument");
    if (M < 1 || hidden < 16 || hidden % 16 != 0 || inter < 16 || inter % 16 != 0) {
        set_last_error("%s: M=%d hidden=%d inter=%d (need M >= 1, hidden and inter positive multiples of 16)",
                       fn, M, hidden, inter);
        return NMI_ERR_INVALID_ARG;
    }
    if (!aligned(input_bf16, 16) || !aligned(norm_w, 16) || !aligned(up_w_e4m3, 16) || !aligned(down_w_e4m3, 16))
        return fail2(NMI_ERR_ALIGNMENT, fn, "input, norm_w and the weights must be 16-byte aligned");
    if (!aligned(up_scale, 4) || !aligned(down_scale, 4) || !aligned(out_bf16, 2))
        return fail2(NMI_ERR_ALIGNMENT, fn, "misaligned scale or output");
    const size_t need = mlp_bytes(M, hidden, inter, split);
    if (workspace) {
        if (!aligned(workspace, 16))
            return fail2(NMI_ERR_ALIGNMENT, fn, "workspace must be 16-byte aligned");
        if (workspace_bytes < need) {
            set_last_error("%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, need);
            return NMI_ERR_WORKSPACE;
        }
    } else {
        const int rc = nmi_alloc(need, &workspace);   // as the reference's allocate_tensor calls
        if (rc != NMI_OK) return rc;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint16_t* in = static_cast<const uint16_t*>(input_bf16);
    uint16_t* out = static_cast<uint16_t*>(out_bf16);
    char* base = static_cast<char*>(workspace);
    const size_t gws = gemm_region(M, hidden, inter, split);
    void* gemm_ws = gws ? base : nullptr;        // the GEMMs' stream-K region or K-split partials
    uint16_t* act = reinterpret_cast<uint16_t*>(base + gws);
    const Norm norm{norm_w, eps};
    if (gws && gemm_workspace_has_flags(M)) {
        // the workspace may hold anything (bump-allocated or reused): zero the flag region
        const hipError_t ez = launch_sk_flags_clear(gemm_ws, st);
        if (ez != hipSuccess) return hip_status(ez, fn);
    }

    // up projection with relu^2: act = bf16(relu(bf16(h . up^T * s))^2)
    GemvGroup up{static_cast<const uint8_t*>(up_w_e4m3), hidden, up_scale, act, inter, inter, 0, 0,
                 Epi{kEpiRelu2, nullptr, 0}};
    hipError_t e;
    if (norm_fused(M, hidden)) {
        e = dispatch_linear(in, hidden, M, hidden, &up, 1, nullptr, 0, st, norm);
    } else {
        uint16_t* normed = reinterpret_cast<uint16_t*>(base + gws + round256((size_t)M * inter * 2));
        e = launch_rmsnorm(in, hidden, norm, normed, hidden, M, hidden, st);
        if (e == hipSuccess) e = dispatch_linear(normed, hidden, M, hidden, &up, 1, gemm_ws, gws, st);
    }
    if (e != hipSuccess) return hip_status(e, fn);
    // down projection with the residual: out = bf16(input + bf16(act . down^T * s))
    GemvGroup down{static_cast<const uint8_t*>(down_w_e4m3), inter, down_scale, out, hidden, hidden, 0, 0,
                   Epi{kEpiResidual, in, hidden}};
    return hip_status(dispatch_linear(act, inter, M, inter, &down, 1, gemm_ws, gws, st), fn);
}

}  // namespace nmi
