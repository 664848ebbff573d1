// mamba.cpp -- extern "C" entry of the fp8 Mamba-2 block at decode (declared in
// include/nmi_fp8_linear.h).
//
// The reference's mamba_block_decode_fp8 (nemotron_infer/csrc/include/model/mamba_block.cuh:
// 436-515) runs twelve launches over bump-allocated buffers: rmsnorm, three gemv_fp8 on the
// in_proj row slices (z, xBC, dt), the conv1d step, three 2-D copies splitting x | B | C, the SSM
// step, the gated RMSNorm, gemv_fp8 (out_proj) and the residual add.  Here four: in_proj as one
// GEMV over all its rows (the slices are consecutive rows, so one launch writes [z | xBC | dt]
// exactly as the three would) with the RMSNorm applied while staging; the conv + SSM kernel
// (which reads x, B and C where the conv leaves them, no split copies); the gated RMSNorm; and
// out_proj with the residual add in its stores.
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

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// proj_ld: the row stride of proj in the block's workspace, proj rounded up to 8 elements so
// that every row starts 16-byte aligned.
struct MambaDims {
    int inter, conv_dim, proj, proj_ld;
};

MambaDims dims(int H, int P, int G, int N) {
    const int inter = H * P, conv_dim = inter + 2 * G * N, proj = inter + conv_dim + H;
    return MambaDims{inter, conv_dim, proj, (proj + 7) & ~7};
}

// Workspace: proj [B, PROJ], y [B, INTER], g [B, INTER] (bf16), normed [B, hidden] when the
// RMSNorm is not fused into the in_proj GEMV.
struct MambaLayout {
    size_t proj, y, g, normed, total;
};

MambaLayout mamba_layout(int batch, int hidden, const MambaDims& d) {
    MambaLayout L{};
    L.proj = 0;
    L.y = L.proj + round256((size_t)batch * d.proj_ld * 2);
    L.g = L.y + round256((size_t)batch * d.inter * 2);
    L.normed = L.g + round256((size_t)batch * d.inter * 2);
    L.total = L.normed + round256((size_t)batch * hidden * 2);
    return L;
}

// Prefill workspace: the GEMMs' stream-K region (M = batch * S >= 512), normed [M, hidden],
// proj [M, proj_ld], xc [M, conv_dim rounded to 8], y [M, INTER], g [M, INTER].
struct FwdLayout {
    size_t gemm, normed, proj, xc, y, g, total;
    int64_t xc_ld;
};

// The GEMMs' region (the short-prompt kernel's K-split partials below M = 512; from 512 the
// stream-K flags and partials where that form is forced by tuning knob, else nothing):
// the larger of the in_proj and out_proj needs.
size_t gemm_region(int M, int hidden, const MambaDims& d) {
    if (choose_path(M) != Path::Gemm) return 0;
    return round256(std::max(linear_workspace_bytes(M, d.proj, hidden), linear_workspace_bytes(M, hidden, d.inter)));
}

FwdLayout fwd_layout(int M, int hidden, const MambaDims& d) {
    FwdLayout L{};
    L.xc_ld = (d.conv_dim + 7) & ~7;
    L.gemm = 0;
    L.normed = L.gemm + gemm_region(M, hidden, d);
    L.proj = L.normed + round256((size_t)M * hidden * 2);
    L.xc = L.proj + round256((size_t)M * d.proj_ld * 2);
    L.y = L.xc + round256((size_t)M * L.xc_ld * 2);
    L.g = L.y + round256((size_t)M * d.inter * 2);
    L.total = L.g + round256((size_t)M * d.inter * 2);
    return L;
}

}  // namespace

extern "C" {

size_t nmi_mamba_forward_workspace_bytes(int batch, int S, int hidden, int n_heads, int head_dim, int n_groups,
                                         int d_state) {
    if (batch < 1 || S < 1 || hidden < 16 || n_heads < 1 || head_dim < 1 || n_groups < 1 || d_state < 1) return 0;
    return fwd_layout(batch * S, hidden, dims(n_heads, head_dim, n_groups, d_state)).total;
}

int nmi_mamba_forward_fp8(const void* input_bf16, const float* norm_w, const void* in_proj_w_e4m3,
                          const float* in_proj_scale, const float* conv_w, const float* conv_b, const float* A_log,
                          const float* D, const float* dt_bias, const float* gnorm_w, const void* out_proj_w_e4m3,
                          const float* out_proj_scale, void* out_bf16, int batch, int S, float* conv_state_out,
                          float* ssm_state_out, int hidden, int n_heads, int head_dim, int n_groups, int d_state,
                          int conv_k, float eps, void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_mamba_forward_fp8";
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    if (!input_bf16 || !norm_w || !in_proj_w_e4m3 || !in_proj_scale || !conv_w || !conv_b || !A_log || !D ||
        !dt_bias || !gnorm_w || !out_proj_w_e4m3 || !out_proj_scale || !out_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_mamba_forward_fp8: NULL pointer argument");
    if (batch < 1 || S < 1 || hidden < 16 || hidden % 16 != 0 || (int64_t)batch * S > (1 << 30)) {
        set_last_error("%s: batch=%d S=%d hidden=%d (need batch, S >= 1, hidden a positive multiple of 16)", fn,
                       batch, S, hidden);
        return NMI_ERR_INVALID_ARG;
    }
    if (!mamba_decode_supported(n_heads, head_dim, n_groups, d_state, conv_k)) {
        set_last_error("%s: n_heads=%d head_dim=%d n_groups=%d d_state=%d conv_k=%d (supported: d_state %d, conv_k "
                       "%d, n_groups dividing n_heads, groups of at most 2048 values, head_dim <= 128, n_heads * "
                       "head_dim a multiple of 8 * n_groups)",
                       fn, n_heads, head_dim, n_groups, d_state, conv_k, kMambaDState, kMambaConvK);
        return NMI_ERR_INVALID_ARG;
    }
    const MambaDims d = dims(n_heads, head_dim, n_groups, d_state);
    if (d.inter % 16 != 0) {
        set_last_error("%s: n_heads * head_dim = %d must be a multiple of 16 (out_proj's K)", fn, d.inter);
        return NMI_ERR_INVALID_ARG;
    }
    if (!aligned(input_bf16, 16) || !aligned(norm_w, 16) || !aligned(in_proj_w_e4m3, 16) ||
        !aligned(out_proj_w_e4m3, 16) || !aligned(conv_w, 16) || !aligned(gnorm_w, 16) ||
        (ssm_state_out && !aligned(ssm_state_out, 16)))
        return fail(NMI_ERR_ALIGNMENT,
                    "nmi_mamba_forward_fp8: input, norm_w, the weights, conv_w, gnorm_w and ssm_state_out must be "
                    "16-byte aligned");
    if (!aligned(in_proj_scale, 4) || !aligned(out_proj_scale, 4) || !aligned(conv_b, 4) || !aligned(A_log, 4) ||
        !aligned(D, 4) || !aligned(dt_bias, 4) || (conv_state_out && !aligned(conv_state_out, 4)) ||
        !aligned(out_bf16, 2))
        return fail(NMI_ERR_ALIGNMENT, "nmi_mamba_forward_fp8: misaligned scale, parameter, state or output");
    const int M = batch * S;
    const FwdLayout lay = fwd_layout(M, hidden, d);
    if (workspace) {
        if (!aligned(workspace, 256))
            return fail(NMI_ERR_ALIGNMENT, "nmi_mamba_forward_fp8: workspace must be 256-byte aligned");
        if (workspace_bytes < lay.total) {
            set_last_error("%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, lay.total);
            return NMI_ERR_WORKSPACE;
        }
    } else {
        const int rc = nmi_alloc(lay.total, &workspace);   // as the reference's allocate_tensor calls
        if (rc != NMI_OK) return rc;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    char* base = static_cast<char*>(workspace);
    const size_t gws = lay.normed - lay.gemm;
    void* gemm_ws = gws ? base + lay.gemm : nullptr;
    uint16_t* proj = reinterpret_cast<uint16_t*>(base + lay.proj);
    const uint16_t* in = static_cast<const uint16_t*>(input_bf16);
    hipError_t e = hipSuccess;
    if (gws && gemm_workspace_has_flags(M)) e = launch_sk_flags_clear(gemm_ws, st);   // the workspace may hold anything
    if (e != hipSuccess) return hip_status(e, fn);
    // in_proj over all rows: proj = [z | xBC | dt]
    GemvGroup ip{static_cast<const uint8_t*>(in_proj_w_e4m3), hidden, in_proj_scale, proj, d.proj_ld, d.proj, 0, 0,
                 Epi{}};
    const Norm norm{norm_w, eps};
    if (gemv_fuses_norm(M, hidden)) {
        e = dispatch_linear(in, hidden, M, hidden, &ip, 1, nullptr, 0, st, norm);
    } else {
        uint16_t* normed = reinterpret_cast<uint16_t*>(base + lay.normed);
        e = launch_rmsnorm(in, hidden, norm, normed, hidden, M, hidden, st);
        if (e == hipSuccess) e = dispatch_linear(normed, hidden, M, hidden, &ip, 1, gemm_ws, gws, st);
    }
    if (e != hipSuccess) return hip_status(e, fn);
    // conv over each sequence, SSM scan
    MambaPrefillArgs pa{};
    pa.proj = proj;
    pa.proj_ld = d.proj_ld;
    pa.xc = reinterpret_cast<uint16_t*>(base + lay.xc);
    pa.xc_ld = lay.xc_ld;
    pa.conv_w = conv_w;
    pa.conv_b = conv_b;
    pa.A_log = A_log;
    pa.D = D;
    pa.dt_bias = dt_bias;
    pa.conv_state = conv_state_out;
    pa.ssm_state = ssm_state_out;
    pa.y = reinterpret_cast<uint16_t*>(base + lay.y);
    pa.y_ld = d.inter;
    pa.S = S;
    pa.H = n_heads;
    pa.P = head_dim;
    pa.G = n_groups;
    pa.inter = d.inter;
    pa.conv_dim = d.conv_dim;
    pa.x_vec = (head_dim % 8 == 0 && pa.xc_ld % 8 == 0) ? 1 : 0;
    pa.y_vec = (head_dim % 8 == 0 && pa.y_ld % 8 == 0) ? 1 : 0;
    e = launch_mamba_prefill_mixer(pa, batch, st);
    if (e != hipSuccess) return hip_status(e, fn);
    // gated RMSNorm of every row
    MambaDecodeArgs ga{};
    ga.proj = proj;
    ga.proj_ld = d.proj_ld;
    ga.y = pa.y;
    ga.g = reinterpret_cast<uint16_t*>(base + lay.g);
    ga.gnorm_w = gnorm_w;
    ga.H = n_heads;
    ga.P = head_dim;
    ga.G = n_groups;
    ga.inter = d.inter;
    ga.conv_dim = d.conv_dim;
    ga.eps = eps;
    ga.bc_state = 0;
    e = launch_mamba_gated_norm(ga, M, st);
    if (e != hipSuccess) return hip_status(e, fn);
    // out = bf16(input + bf16(out_proj(g)))
    GemvGroup op{static_cast<const uint8_t*>(out_proj_w_e4m3), d.inter, out_proj_scale, static_cast<uint16_t*>(out_bf16),
                 hidden, hidden, 0, 0, Epi{kEpiResidual, in, hidden}};
    return hip_status(dispatch_linear(ga.g, d.inter, M, d.inter, &op, 1, gemm_ws, gws, st), fn);
}

int nmi_mamba_mixer_decode(const void* proj_bf16, int64_t proj_ld, const float* conv_w, const float* conv_b,
                           const float* A_log, const float* D, const float* dt_bias, const float* gnorm_w,
                           float* conv_state, float* ssm_state, void* y_bf16, void* g_bf16, int batch, int n_heads,
                           int head_dim, int n_groups, int d_state, int conv_k, float eps, void* stream) {
    const char* fn = "nmi_mamba_mixer_decode";
    if (!proj_bf16 || !conv_w || !conv_b || !A_log || !D || !dt_bias || !gnorm_w || !conv_state || !ssm_state ||
        !y_bf16 || !g_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_mamba_mixer_decode: NULL pointer argument");
    if (batch < 1 || !mamba_decode_supported(n_heads, head_dim, n_groups, d_state, conv_k)) {
        set_last_error("%s: batch=%d n_heads=%d head_dim=%d n_groups=%d d_state=%d conv_k=%d (supported: batch >= 1, "
                       "d_state %d, conv_k %d, n_groups dividing n_heads, groups of at most 2048 values, "
                       "head_dim <= 128, n_heads * head_dim a multiple of 8 * n_groups)",
                       fn, batch, n_heads, head_dim, n_groups, d_state, conv_k, kMambaDState, kMambaConvK);
        return NMI_ERR_INVALID_ARG;
    }
    const MambaDims d = dims(n_heads, head_dim, n_groups, d_state);
    if (proj_ld < d.proj || (proj_ld * 2) % 16 != 0) {
        set_last_error("%s: proj_ld=%lld (need >= %d and a multiple of 8)", fn, (long long)proj_ld, d.proj);
        return NMI_ERR_INVALID_ARG;
    }
    if (!aligned(proj_bf16, 16) || !aligned(conv_w, 16) || !aligned(gnorm_w, 16) || !aligned(ssm_state, 16) ||
        !aligned(y_bf16, 16) || !aligned(g_bf16, 16))
        return fail(NMI_ERR_ALIGNMENT,
                    "nmi_mamba_mixer_decode: proj, conv_w, gnorm_w, ssm_state, y and g must be 16-byte aligned");
    if (!aligned(conv_b, 4) || !aligned(A_log, 4) || !aligned(D, 4) || !aligned(dt_bias, 4) || !aligned(conv_state, 4))
        return fail(NMI_ERR_ALIGNMENT, "nmi_mamba_mixer_decode: misaligned parameter or state");
    MambaDecodeArgs a{};
    a.proj = static_cast<const uint16_t*>(proj_bf16);
    a.proj_ld = proj_ld;
    a.conv_w = conv_w;
    a.conv_b = conv_b;
    a.A_log = A_log;
    a.D = D;
    a.dt_bias = dt_bias;
    a.gnorm_w = gnorm_w;
    a.conv_state = conv_state;
    a.ssm_state = ssm_state;
    a.y = static_cast<uint16_t*>(y_bf16);
    a.g = static_cast<uint16_t*>(g_bf16);
    a.H = n_heads;
    a.P = head_dim;
    a.G = n_groups;
    a.inter = d.inter;
    a.conv_dim = d.conv_dim;
    a.eps = eps;
    a.bc_state = 1;
    return hip_status(launch_mamba_decode_mixer(a, batch, static_cast<hipStream_t>(stream)), fn);
}

size_t nmi_mamba_decode_workspace_bytes(int batch, int hidden, int n_heads, int head_dim, int n_groups,
                                        int d_state) {
    if (batch < 1 || hidden < 16 || n_heads < 1 || head_dim < 1 || n_groups < 1 || d_state < 1) return 0;
    return mamba_layout(batch, hidden, dims(n_heads, head_dim, n_groups, d_state)).total;
}

int nmi_mamba_decode_fp8(const void* input_bf16, const float* norm_w, const void* in_proj_w_e4m3,
                         const float* in_proj_scale, const float* conv_w, const float* conv_b, const float* A_log,
                         const float* D, const float* dt_bias, const float* gnorm_w, const void* out_proj_w_e4m3,
                         const float* out_proj_scale, float* conv_state, float* ssm_state, void* out_bf16, int batch,
                         int hidden, int n_heads, int head_dim, int n_groups, int d_state, int conv_k, float eps,
                         void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_mamba_decode_fp8";
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    if (!input_bf16 || !norm_w || !in_proj_w_e4m3 || !in_proj_scale || !conv_w || !conv_b || !A_log || !D ||
        !dt_bias || !gnorm_w || !out_proj_w_e4m3 || !out_proj_scale || !conv_state || !ssm_state || !out_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_mamba_decode_fp8: NULL pointer argument");
    if (batch < 1 || hidden < 16 || hidden % 16 != 0) {
        set_last_error("%s: batch=%d hidden=%d (need batch >= 1, hidden a positive multiple of 16)", fn, batch,
                       hidden);
        return NMI_ERR_INVALID_ARG;
    }
    if (!mamba_decode_supported(n_heads, head_dim, n_groups, d_state, conv_k)) {
        set_last_error("%s: n_heads=%d head_dim=%d n_groups=%d d_state=%d conv_k=%d (supported: d_state %d, conv_k "
                       "%d, n_groups dividing n_heads, groups of at most 2048 values, head_dim <= 128, n_heads * "
                       "head_dim a multiple of 8 * n_groups)",
                       fn, n_heads, head_dim, n_groups, d_state, conv_k, kMambaDState, kMambaConvK);
        return NMI_ERR_INVALID_ARG;
    }
    const MambaDims d = dims(n_heads, head_dim, n_groups, d_state);
    if (d.inter % 16 != 0) {
        set_last_error("%s: n_heads * head_dim = %d must be a multiple of 16 (out_proj's K)", fn, d.inter);
        return NMI_ERR_INVALID_ARG;
    }
    if (!aligned(input_bf16, 16) || !aligned(norm_w, 16) || !aligned(in_proj_w_e4m3, 16) ||
        !aligned(out_proj_w_e4m3, 16) || !aligned(conv_w, 16) || !aligned(gnorm_w, 16) || !aligned(ssm_state, 16))
        return fail(NMI_ERR_ALIGNMENT,
                    "nmi_mamba_decode_fp8: input, norm_w, the weights, conv_w, gnorm_w and ssm_state must be "
                    "16-byte aligned");
    if (!aligned(in_proj_scale, 4) || !aligned(out_proj_scale, 4) || !aligned(conv_b, 4) || !aligned(A_log, 4) ||
        !aligned(D, 4) || !aligned(dt_bias, 4) || !aligned(conv_state, 4) || !aligned(out_bf16, 2))
        return fail(NMI_ERR_ALIGNMENT, "nmi_mamba_decode_fp8: misaligned scale, parameter, state or output");
    const MambaLayout lay = mamba_layout(batch, hidden, d);
    if (workspace) {
        if (!aligned(workspace, 16))
            return fail(NMI_ERR_ALIGNMENT, "nmi_mamba_decode_fp8: workspace must be 16-byte aligned");
        if (workspace_bytes < lay.total) {
            set_last_error("%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, lay.total);
            return NMI_ERR_WORKSPACE;
        }
    } else {
        const int rc = nmi_alloc(lay.total, &workspace);   // as the reference's allocate_tensor calls
        if (rc != NMI_OK) return rc;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    char* base = static_cast<char*>(workspace);
    uint16_t* proj = reinterpret_cast<uint16_t*>(base + lay.proj);
    const uint16_t* in = static_cast<const uint16_t*>(input_bf16);
    const Norm norm{norm_w, eps};

    // in_proj over all rows: proj = [z | xBC | dt]
    GemvGroup ip{static_cast<const uint8_t*>(in_proj_w_e4m3), hidden, in_proj_scale, proj, d.proj_ld, d.proj, 0, 0,
                 Epi{}};
    hipError_t e;
    if (gemv_fuses_norm(batch, hidden)) {
        e = dispatch_linear(in, hidden, batch, hidden, &ip, 1, nullptr, 0, st, norm);
    } else {
        uint16_t* normed = reinterpret_cast<uint16_t*>(base + lay.normed);
        e = launch_rmsnorm(in, hidden, norm, normed, hidden, batch, hidden, st);
        if (e == hipSuccess) e = dispatch_linear(normed, hidden, batch, hidden, &ip, 1, nullptr, 0, st);
    }
    if (e != hipSuccess) return hip_status(e, fn);
    // conv step + SSM step + gated RMSNorm
    MambaDecodeArgs a{};
    a.proj = proj;
    a.proj_ld = d.proj_ld;
    a.conv_w = conv_w;
    a.conv_b = conv_b;
    a.A_log = A_log;
    a.D = D;
    a.dt_bias = dt_bias;
    a.gnorm_w = gnorm_w;
    a.conv_state = conv_state;
    a.ssm_state = ssm_state;
    a.y = reinterpret_cast<uint16_t*>(base + lay.y);
    a.g = reinterpret_cast<uint16_t*>(base + lay.g);
    a.H = n_heads;
    a.P = head_dim;
    a.G = n_groups;
    a.inter = d.inter;
    a.conv_dim = d.conv_dim;
    a.eps = eps;
    a.bc_state = 1;
    e = launch_mamba_decode_mixer(a, batch, st);
    if (e != hipSuccess) return hip_status(e, fn);
    // out = bf16(input + bf16(out_proj(g)))
    GemvGroup op{static_cast<const uint8_t*>(out_proj_w_e4m3), d.inter, out_proj_scale, static_cast<uint16_t*>(out_bf16),
                 hidden, hidden, 0, 0, Epi{kEpiResidual, in, hidden}};
    return hip_status(dispatch_linear(a.g, d.inter, batch, d.inter, &op, 1, nullptr, 0, st), fn);
}

}  // extern "C"
