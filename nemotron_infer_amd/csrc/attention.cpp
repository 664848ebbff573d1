// attention.cpp -- extern "C" entries of the attention decode path (declared in
// include/nmi_fp8_linear.h): the SDPA decode op and the fp8 attention decode block.
//
// The reference's attention_block_decode_fp8 (nemotron_infer/csrc/include/model/
// attention_block.cuh:371-414) runs eight launches over bump-allocated buffers: rmsnorm, three
// gemv_fp8 (q, k, v), the two kernels of sdpa_decode_bf16, gemv_fp8 (o) and a residual add.
// Here: one grouped q|k|v GEMV that applies the RMSNorm while staging its input, the SDPA split
// kernel (which also appends K/V to the caches), its combine kernel when the positions are
// split, and the o GEMV with the residual add in its stores -- three or four launches.
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

// Shape checks shared by the op and the block; 0 or an NMI_ERR_* with the message set.
int check_sdpa_shape(const char* fn, int S_cache, int cache_cap, int n_heads, int n_kv) {
    if (n_kv < 1 || n_heads < n_kv || n_heads % n_kv != 0 || n_heads / n_kv > kSdpaMaxGroup) {
        set_last_error("%s: n_heads=%d n_kv_heads=%d (need n_heads a multiple of n_kv_heads, at most %d query "
                       "heads per KV head)",
                       fn, n_heads, n_kv, kSdpaMaxGroup);
        return NMI_ERR_INVALID_ARG;
    }
    if (S_cache < 0 || cache_cap <= S_cache) {
        set_last_error("%s: S_cache=%d cache_cap=%d (need 0 <= S_cache < cache_cap: the new token is stored at "
                       "position S_cache)",
                       fn, S_cache, cache_cap);
        return NMI_ERR_INVALID_ARG;
    }
    return NMI_OK;
}

// Block workspace: q [H*128], k_new, v_new [H_KV*128], o [H*128], normed [hidden] (when the
// RMSNorm is not fused into the q|k|v GEMV), then the SDPA partials.
struct AttnLayout {
    size_t q, k, v, o, normed, part, total;
};

AttnLayout attn_layout(int hidden, int n_heads, int n_kv, int S_cache) {
    AttnLayout L{};
    const size_t qb = round256((size_t)n_heads * kSdpaHead * 2), kb = round256((size_t)n_kv * kSdpaHead * 2);
    L.q = 0;
    L.k = L.q + qb;
    L.v = L.k + kb;
    L.o = L.v + kb;
    L.normed = L.o + qb;
    L.part = L.normed + round256((size_t)hidden * 2);
    L.total = L.part + round256(sdpa_decode_workspace_bytes(n_heads, S_cache, n_kv));
    return L;
}

// Prefill block workspace: the GEMMs' stream-K region (S >= 512), normed [S, hidden], q
// [S, H*128], k and v [S, H_KV*128], o [S, H*128].
struct FwdLayout {
    size_t gemm, normed, q, k, v, o, total;
};

// The GEMMs' region (the short-prompt kernel's K-split partials below M = 512; from 512 the
// stream-K flags and partials where that form is forced by tuning knob, else nothing):
// the largest of the q, k, v (launched one by one on the GEMM path) and o needs.
size_t gemm_region(int M, int hidden, int QD, int KD) {
    if (choose_path(M) != Path::Gemm) return 0;
    const size_t qkv = std::max(linear_workspace_bytes(M, (int64_t)QD + 2 * (int64_t)KD, hidden),
                                std::max(linear_workspace_bytes(M, QD, hidden), linear_workspace_bytes(M, KD, hidden)));
    return round256(std::max(qkv, linear_workspace_bytes(M, hidden, QD)));
}

FwdLayout fwd_layout(int S, int hidden, int n_heads, int n_kv) {
    FwdLayout L{};
    const size_t QD = (size_t)n_heads * kSdpaHead, KD = (size_t)n_kv * kSdpaHead;
    L.gemm = 0;
    L.normed = L.gemm + gemm_region(S, hidden, (int)QD, (int)KD);
    L.q = L.normed + round256((size_t)S * hidden * 2);
    L.k = L.q + round256((size_t)S * QD * 2);
    L.v = L.k + round256((size_t)S * KD * 2);
    L.o = L.v + round256((size_t)S * KD * 2);
    L.total = L.o + round256((size_t)S * QD * 2);
    return L;
}

bool heads_ok(int n_heads, int n_kv) { return n_kv >= 1 && n_heads >= n_kv && n_heads % n_kv == 0; }

}  // namespace

extern "C" {

size_t nmi_sdpa_prefill_workspace_bytes(int n_kv_heads, int S) {
    (void)n_kv_heads;
    (void)S;
    return 0;                                  // the kernel reads q, k and v as they are
}

int nmi_sdpa_prefill_bf16(const void* q_bf16, int64_t ldq, const void* k_bf16, int64_t ldk, const void* v_bf16,
                          int64_t ldv, void* o_bf16, int64_t ldo, int S, int n_heads, int n_kv_heads, void* workspace,
                          size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_sdpa_prefill_bf16";
    if (!q_bf16 || !k_bf16 || !v_bf16 || !o_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_sdpa_prefill_bf16: NULL pointer argument");
    if (S < 1 || !heads_ok(n_heads, n_kv_heads) || ldq < (int64_t)n_heads * kSdpaHead ||
        ldo < (int64_t)n_heads * kSdpaHead || ldk < (int64_t)n_kv_heads * kSdpaHead ||
        ldv < (int64_t)n_kv_heads * kSdpaHead) {
        set_last_error("%s: S=%d n_heads=%d n_kv_heads=%d ldq=%lld ldk=%lld ldv=%lld ldo=%lld (need S >= 1, n_heads a "
                       "multiple of n_kv_heads, row strides of at least the heads' 128 columns)",
                       fn, S, n_heads, n_kv_heads, (long long)ldq, (long long)ldk, (long long)ldv, (long long)ldo);
        return NMI_ERR_INVALID_ARG;
    }
    if (!aligned(q_bf16, 16) || !aligned(k_bf16, 16) || !aligned(v_bf16, 16) || !aligned(o_bf16, 8) || ldq % 8 ||
        ldk % 8 || ldv % 8 || ldo % 4)
        return fail(NMI_ERR_ALIGNMENT,
                    "nmi_sdpa_prefill_bf16: q, k, v must be 16-byte aligned with row strides multiple of 8 elements; "
                    "o 8-byte aligned with a row stride multiple of 4");
    (void)workspace;                           // no workspace: nmi_sdpa_prefill_workspace_bytes is 0
    (void)workspace_bytes;
    const hipError_t e = launch_sdpa_prefill(static_cast<const uint16_t*>(q_bf16), ldq,
                                             static_cast<const uint16_t*>(k_bf16), ldk,
                                             static_cast<const uint16_t*>(v_bf16), ldv, static_cast<uint16_t*>(o_bf16),
                                             ldo, S, n_heads, n_kv_heads, static_cast<hipStream_t>(stream));
    return hip_status(e, fn);
}

size_t nmi_attn_forward_workspace_bytes(int S, int hidden, int n_heads, int n_kv_heads) {
    if (S < 1 || hidden < 16 || !heads_ok(n_heads, n_kv_heads)) return 0;
    return fwd_layout(S, hidden, n_heads, n_kv_heads).total;
}

int nmi_attn_forward_fp8(const void* input_bf16, const float* norm_w, const void* q_w_e4m3, const float* q_scale,
                         const void* k_w_e4m3, const float* k_scale, const void* v_w_e4m3, const float* v_scale,
                         const void* o_w_e4m3, const float* o_scale, void* out_bf16, int S, void* k_cache_bf16,
                         void* v_cache_bf16, int cache_cap, int hidden, int n_heads, int n_kv_heads, float eps,
                         void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_attn_forward_fp8";
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    if (!input_bf16 || !norm_w || !q_w_e4m3 || !q_scale || !k_w_e4m3 || !k_scale || !v_w_e4m3 || !v_scale ||
        !o_w_e4m3 || !o_scale || !out_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_attn_forward_fp8: NULL pointer argument");
    if (S < 1 || hidden < 16 || hidden % 16 != 0 || !heads_ok(n_heads, n_kv_heads)) {
        set_last_error("%s: S=%d hidden=%d n_heads=%d n_kv_heads=%d (need S >= 1, hidden a positive multiple of 16, "
                       "n_heads a multiple of n_kv_heads)",
                       fn, S, hidden, n_heads, n_kv_heads);
        return NMI_ERR_INVALID_ARG;
    }
    const bool caches = k_cache_bf16 && v_cache_bf16;
    const int cap = cache_cap > 0 ? cache_cap : S;
    if (caches && cap < S) {
        set_last_error("%s: cache_cap=%d < S=%d", fn, cache_cap, S);
        return NMI_ERR_INVALID_ARG;
    }
    if (!aligned(input_bf16, 16) || !aligned(norm_w, 16) || !aligned(q_w_e4m3, 16) || !aligned(k_w_e4m3, 16) ||
        !aligned(v_w_e4m3, 16) || !aligned(o_w_e4m3, 16) ||
        (caches && (!aligned(k_cache_bf16, 16) || !aligned(v_cache_bf16, 16))))
        return fail(NMI_ERR_ALIGNMENT,
                    "nmi_attn_forward_fp8: input, norm_w, the weights and the caches must be 16-byte aligned");
    if (!aligned(q_scale, 4) || !aligned(k_scale, 4) || !aligned(v_scale, 4) || !aligned(o_scale, 4) ||
        !aligned(out_bf16, 2))
        return fail(NMI_ERR_ALIGNMENT, "nmi_attn_forward_fp8: misaligned scale or output");
    const FwdLayout lay = fwd_layout(S, hidden, n_heads, n_kv_heads);
    if (workspace) {
        if (!aligned(workspace, 256))
            return fail(NMI_ERR_ALIGNMENT, "nmi_attn_forward_fp8: workspace must be 256-byte aligned");
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
    const int QD = n_heads * kSdpaHead, KD = n_kv_heads * kSdpaHead;
    const uint16_t* in = static_cast<const uint16_t*>(input_bf16);
    uint16_t* q = reinterpret_cast<uint16_t*>(base + lay.q);
    uint16_t* k = reinterpret_cast<uint16_t*>(base + lay.k);
    uint16_t* v = reinterpret_cast<uint16_t*>(base + lay.v);
    uint16_t* o = reinterpret_cast<uint16_t*>(base + lay.o);
    hipError_t e = hipSuccess;
    if (gws && gemm_workspace_has_flags(S)) e = launch_sk_flags_clear(gemm_ws, st);   // the workspace may hold anything
    if (e != hipSuccess) return hip_status(e, fn);
    // q, k, v of the normed input
    GemvGroup qkv[3] = {
        {static_cast<const uint8_t*>(q_w_e4m3), hidden, q_scale, q, QD, QD, 0, 0, Epi{}},
        {static_cast<const uint8_t*>(k_w_e4m3), hidden, k_scale, k, KD, KD, 0, 0, Epi{}},
        {static_cast<const uint8_t*>(v_w_e4m3), hidden, v_scale, v, KD, KD, 0, 0, Epi{}},
    };
    const Norm norm{norm_w, eps};
    if (gemv_fuses_norm(S, hidden)) {
        e = dispatch_linear(in, hidden, S, hidden, qkv, 3, nullptr, 0, st, norm);
    } else {
        uint16_t* normed = reinterpret_cast<uint16_t*>(base + lay.normed);
        e = launch_rmsnorm(in, hidden, norm, normed, hidden, S, hidden, st);
        if (e == hipSuccess) e = dispatch_linear(normed, hidden, S, hidden, qkv, 3, gemm_ws, gws, st);
    }
    if (e != hipSuccess) return hip_status(e, fn);
    // the caches, causal attention
    if (caches)
        e = launch_kv_cache(k, KD, v, KD, S, n_kv_heads, static_cast<uint16_t*>(k_cache_bf16),
                            static_cast<uint16_t*>(v_cache_bf16), cap, st);
    if (e == hipSuccess) e = launch_sdpa_prefill(q, QD, k, KD, v, KD, o, QD, S, n_heads, n_kv_heads, st);
    if (e != hipSuccess) return hip_status(e, fn);
    // out = bf16(input + bf16(o_proj(o)))
    GemvGroup og{static_cast<const uint8_t*>(o_w_e4m3), QD, o_scale, static_cast<uint16_t*>(out_bf16), hidden, hidden,
                 0, 0, Epi{kEpiResidual, in, hidden}};
    return hip_status(dispatch_linear(o, QD, S, QD, &og, 1, gemm_ws, gws, st), fn);
}

size_t nmi_sdpa_decode_workspace_bytes(int n_heads, int n_kv_heads, int S_cache) {
    if (n_kv_heads < 1 || n_heads < 1 || S_cache < 0) return 0;
    return sdpa_decode_workspace_bytes(n_heads, S_cache, n_kv_heads);
}

int nmi_sdpa_decode_bf16(const void* q_bf16, void* k_cache_bf16, void* v_cache_bf16, void* o_bf16,
                         const void* k_new_bf16, const void* v_new_bf16, int S_cache, int cache_cap, int n_heads,
                         int n_kv_heads, void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_sdpa_decode_bf16";
    if (!q_bf16 || !k_cache_bf16 || !v_cache_bf16 || !o_bf16 || !k_new_bf16 || !v_new_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_sdpa_decode_bf16: NULL pointer argument");
    int rc = check_sdpa_shape(fn, S_cache, cache_cap, n_heads, n_kv_heads);
    if (rc != NMI_OK) return rc;
    if (!aligned(q_bf16, 16) || !aligned(k_cache_bf16, 16) || !aligned(v_cache_bf16, 16) || !aligned(k_new_bf16, 16) ||
        !aligned(v_new_bf16, 16) || !aligned(o_bf16, 4))
        return fail(NMI_ERR_ALIGNMENT,
                    "nmi_sdpa_decode_bf16: q, the caches, k_new and v_new must be 16-byte aligned, o 4-byte aligned");
    const size_t need = sdpa_decode_workspace_bytes(n_heads, S_cache, n_kv_heads);
    if (need) {
        if (workspace) {
            if (!aligned(workspace, 16))
                return fail(NMI_ERR_ALIGNMENT, "nmi_sdpa_decode_bf16: workspace must be 16-byte aligned");
            if (workspace_bytes < need) {
                set_last_error("%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, need);
                return NMI_ERR_WORKSPACE;
            }
        } else {
            rc = nmi_alloc(need, &workspace);
            if (rc != NMI_OK) return rc;
        }
    }
    return hip_status(launch_sdpa_decode(static_cast<const uint16_t*>(q_bf16), static_cast<uint16_t*>(k_cache_bf16),
                                         static_cast<uint16_t*>(v_cache_bf16), static_cast<const uint16_t*>(k_new_bf16),
                                         static_cast<const uint16_t*>(v_new_bf16), static_cast<uint16_t*>(o_bf16),
                                         S_cache, cache_cap, n_heads, n_kv_heads, workspace,
                                         static_cast<hipStream_t>(stream)),
                      fn);
}

size_t nmi_attn_decode_workspace_bytes(int hidden, int n_heads, int n_kv_heads, int S_cache) {
    if (hidden < 16 || n_heads < 1 || n_kv_heads < 1 || S_cache < 0) return 0;
    return attn_layout(hidden, n_heads, n_kv_heads, S_cache).total;
}

int nmi_attn_decode_fp8(const void* input_bf16, const float* norm_w, const void* q_w_e4m3, const float* q_scale,
                        const void* k_w_e4m3, const float* k_scale, const void* v_w_e4m3, const float* v_scale,
                        const void* o_w_e4m3, const float* o_scale, void* k_cache_bf16, void* v_cache_bf16,
                        int S_cache, int cache_cap, void* out_bf16, int hidden, int n_heads, int n_kv_heads,
                        float eps, void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "nmi_attn_decode_fp8";
    if (take_async_error(fn)) return NMI_ERR_ASYNC;
    if (!input_bf16 || !norm_w || !q_w_e4m3 || !q_scale || !k_w_e4m3 || !k_scale || !v_w_e4m3 || !v_scale ||
        !o_w_e4m3 || !o_scale || !k_cache_bf16 || !v_cache_bf16 || !out_bf16)
        return fail(NMI_ERR_INVALID_ARG, "nmi_attn_decode_fp8: NULL pointer argument");
    if (hidden < 16 || hidden % 16 != 0) {
        set_last_error("%s: hidden=%d (need a positive multiple of 16)", fn, hidden);
        return NMI_ERR_INVALID_ARG;
    }
    int rc = check_sdpa_shape(fn, S_cache, cache_cap, n_heads, n_kv_heads);
    if (rc != NMI_OK) return rc;
    if (!aligned(input_bf16, 16) || !aligned(norm_w, 16) || !aligned(q_w_e4m3, 16) || !aligned(k_w_e4m3, 16) ||
        !aligned(v_w_e4m3, 16) || !aligned(o_w_e4m3, 16) || !aligned(k_cache_bf16, 16) || !aligned(v_cache_bf16, 16))
        return fail(NMI_ERR_ALIGNMENT,
                    "nmi_attn_decode_fp8: input, norm_w, the weights and the caches must be 16-byte aligned");
    if (!aligned(q_scale, 4) || !aligned(k_scale, 4) || !aligned(v_scale, 4) || !aligned(o_scale, 4) ||
        !aligned(out_bf16, 2))
        return fail(NMI_ERR_ALIGNMENT, "nmi_attn_decode_fp8: misaligned scale or output");
    const AttnLayout lay = attn_layout(hidden, n_heads, n_kv_heads, S_cache);
    if (workspace) {
        if (!aligned(workspace, 16))
            return fail(NMI_ERR_ALIGNMENT, "nmi_attn_decode_fp8: workspace must be 16-byte aligned");
        if (workspace_bytes < lay.total) {
            set_last_error("%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, lay.total);
            return NMI_ERR_WORKSPACE;
        }
    } else {
        rc = nmi_alloc(lay.total, &workspace);   // as the reference's allocate_tensor calls
        if (rc != NMI_OK) return rc;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    char* base = static_cast<char*>(workspace);
    uint16_t* q = reinterpret_cast<uint16_t*>(base + lay.q);
    uint16_t* kn = reinterpret_cast<uint16_t*>(base + lay.k);
    uint16_t* vn = reinterpret_cast<uint16_t*>(base + lay.v);
    uint16_t* ot = reinterpret_cast<uint16_t*>(base + lay.o);
    const uint16_t* in = static_cast<const uint16_t*>(input_bf16);
    const int QD = n_heads * kSdpaHead, KD = n_kv_heads * kSdpaHead;

    // q|k|v of the normed input, one grouped launch
    GemvGroup qkv[3] = {
        {static_cast<const uint8_t*>(q_w_e4m3), hidden, q_scale, q, QD, QD, 0, 0, Epi{}},
        {static_cast<const uint8_t*>(k_w_e4m3), hidden, k_scale, kn, KD, KD, 0, 0, Epi{}},
        {static_cast<const uint8_t*>(v_w_e4m3), hidden, v_scale, vn, KD, KD, 0, 0, Epi{}},
    };
    const Norm norm{norm_w, eps};
    hipError_t e;
    if (gemv_fuses_norm(1, hidden)) {
        e = dispatch_linear(in, hidden, 1, hidden, qkv, 3, nullptr, 0, st, norm);
    } else {
        uint16_t* normed = reinterpret_cast<uint16_t*>(base + lay.normed);
        e = launch_rmsnorm(in, hidden, norm, normed, hidden, 1, hidden, st);
        if (e == hipSuccess) e = dispatch_linear(normed, hidden, 1, hidden, qkv, 3, nullptr, 0, st);
    }
    if (e != hipSuccess) return hip_status(e, fn);
    // attention over the cached positions, then K/V of this token appended at S_cache
    e = launch_sdpa_decode(q, static_cast<uint16_t*>(k_cache_bf16), static_cast<uint16_t*>(v_cache_bf16), kn, vn, ot,
                           S_cache, cache_cap, n_heads, n_kv_heads, base + lay.part, st);
    if (e != hipSuccess) return hip_status(e, fn);
    // out = bf16(input + bf16(o_proj(ot)))
    GemvGroup og{static_cast<const uint8_t*>(o_w_e4m3), QD, o_scale, static_cast<uint16_t*>(out_bf16), hidden, hidden,
                 0, 0, Epi{kEpiResidual, in, hidden}};
    return hip_status(dispatch_linear(ot, QD, 1, QD, &og, 1, nullptr, 0, st), fn);
}

}  // extern "C"
