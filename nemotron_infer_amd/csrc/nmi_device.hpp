// nmi_device.hpp -- gfx950 (CDNA4) device helpers shared by the fp8 W8A16 kernels.
//
// * e4m3 -> bf16 decode through v_cvt_scalef32_pk_bf16_fp8 with scale 1.0 (OCP E4M3 on gfx950),
//   four codes per dword, byte b -> element b.  Every e4m3 value is exactly representable in
//   bf16, so this is the value static_cast<float>(__nv_fp8_e4m3) gives in the reference
//   (nemotron_infer/csrc/include/ops/gemv.cuh:40-42) and the only decode the kernels use: the
//   GEMVs feed the pairs to v_dot2_f32_bf16, the MFMA kernels to their bf16 operands.
// * bf16 -> f32 by shifting the bit pattern; f32 -> bf16 round-to-nearest-even through
//   v_cvt_pk_bf16_f32 (the conversion __float2bfloat16_rn performs in gemv.cuh:88).
// * a 16-lane sum that uses DPP row operations (quad_perm, row_half_mirror, row_mirror), and
//   a 64-lane sum built on it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nmi_launch.hpp"

namespace nmi {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Four e4m3 codes -> four bf16 (two packed dwords), exact.
__device__ __forceinline__ uint2 e4m3x4_to_bf16(uint32_t w) {
    const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, false);
    const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, true);
    return uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

// c + a.lo * b.lo + a.hi * b.hi, a and b two packed bf16 each (v_dot2_f32_bf16; the
// bf16 x bf16 products are exact in float32).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                          false);
}

// Two bf16 packed in a dword -> two floats (element 0 is the low half).
__device__ __forceinline__ float bf16lo_to_f32(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float bf16hi_to_f32(uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); }

// f32 -> bf16 bits, round to nearest even (hardware v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Output epilogues fused into the stores of the linear kernels.  The linear's own result is
// v = bf16_rne(acc * s); kEpiRelu2 stores bf16_rne(max(v, 0)^2) and kEpiResidual stores
// bf16_rne(res + v).  A bf16 x bf16 product is exact in float32, and a float32 sum of two bf16
// is either exact or within 2^-24 relative of an operand that is itself the nearest bf16, so
// both round to the bf16 the reference's bf16 arithmetic gives on the rounded linear output
// (relu^2 as __hfma2_relu then __hmul2, ops/elementwise.cuh:256-272; residual as __hadd2,
// :241-244; used at model/mlp_block.cuh:145-147, 163-165 and 173-175).  relu keeps NaN
// (NaN < 0 is false).  `res` is the residual's bf16 bits (used only for kEpiResidual).
// Kernels load the residual before their first store: y may be the residual itself (in place),
// so a load issued after a store to y could not be moved ahead of it and would wait on memory
// once per store.
__device__ __forceinline__ uint16_t epilogue(float acc, float s, int epi, uint16_t res) {
    const uint16_t v = f32_to_bf16_rne(acc * s);
    if (epi == kEpiRelu2) {
        float f = bf16_to_f32(v);
        f = f < 0.f ? 0.f : f;
        return f32_to_bf16_rne(f * f);
    }
    if (epi == kEpiResidual) return f32_to_bf16_rne(bf16_to_f32(res) + bf16_to_f32(v));
    return v;
}

// Residual elements off .. off + 3 of one row (clamped to its last element `last`), packed as
// four bf16; one 8-byte load when `vec` (then all four are in bounds and 8-byte aligned).
__device__ __forceinline__ uint2 load_res4(const uint16_t* res, int64_t off, int64_t last, bool vec) {
    if (vec) return *reinterpret_cast<const uint2*>(res + off);
    return uint2{(uint32_t)res[min(off, last)] | ((uint32_t)res[min(off + 1, last)] << 16),
                 (uint32_t)res[min(off + 2, last)] | ((uint32_t)res[min(off + 3, last)] << 16)};
}

// RMSNorm pieces: 8 consecutive bf16 activations in 16 bytes.  sumsq8 continues a float32
// fma chain over the 8 elements in order; rms_scale8 returns bf16_rne(x * (r * g)) for each
// element (the reference's order of operations, ops/reduce.cuh:190-206).
__device__ __forceinline__ float sumsq8(const uint4 v, float acc) {
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = bf16lo_to_f32(d[i]), hi = bf16hi_to_f32(d[i]);
        acc = __builtin_fmaf(lo, lo, acc);
        acc = __builtin_fmaf(hi, hi, acc);
    }
    return acc;
}

// Two f32 -> two bf16 (lo in the low half), round to nearest even: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// epilogue()'s relu^2 and residual steps on two packed bf16 (low half first) that are already
// the rounded linear outputs v.
__device__ __forceinline__ uint32_t relu2_bf16x2(uint32_t w) {
    float lo = bf16lo_to_f32(w), hi = bf16hi_to_f32(w);
    lo = lo < 0.f ? 0.f : lo;
    hi = hi < 0.f ? 0.f : hi;
    return pack_bf16(lo * lo, hi * hi);
}
__device__ __forceinline__ uint32_t add_bf16x2(uint32_t v, uint32_t res) {
    return pack_bf16(bf16lo_to_f32(res) + bf16lo_to_f32(v), bf16hi_to_f32(res) + bf16hi_to_f32(v));
}

__device__ __forceinline__ uint4 rms_scale8(const uint4 v, const float4 g0, const float4 g1, float r) {
    return uint4{pack_bf16(bf16lo_to_f32(v.x) * (r * g0.x), bf16hi_to_f32(v.x) * (r * g0.y)),
                 pack_bf16(bf16lo_to_f32(v.y) * (r * g0.z), bf16hi_to_f32(v.y) * (r * g0.w)),
                 pack_bf16(bf16lo_to_f32(v.z) * (r * g1.x), bf16hi_to_f32(v.z) * (r * g1.y)),
                 pack_bf16(bf16lo_to_f32(v.w) * (r * g1.z), bf16hi_to_f32(v.w) * (r * g1.w))};
}

// 1 / sqrt(mean + eps) with correctly rounded float32 division and square root (HIP's default
// for '/' and sqrtf); the reference uses rsqrtf (ops/reduce.cuh:174).
__device__ __forceinline__ float rms_factor(float sumsq, int K, float eps) {
    return 1.0f / sqrtf(sumsq / (float)K + eps);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of each DPP row; every lane of the row receives the row total.
__device__ __forceinline__ float dpp_row_sum16(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]: pairs
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]: quads
    v += dpp_f32<0x141>(v);  // row_half_mirror: 8 lanes
    v += dpp_f32<0x140>(v);  // row_mirror: 16 lanes
    return v;
}

// Sum over all 64 lanes in a fixed order: 16-lane DPP row sums, then (r0 + r1) + (r2 + r3).
// Every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_row_sum16(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// 16-byte global load that bypasses the caches' retention policy (streamed weights).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return uint4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ uint4 load16(const void* p) {
    return *reinterpret_cast<const uint4*>(p);
}

// 16 bytes per lane from global memory straight into LDS (64 lanes: 1 KiB at lds_addr, in lane
// order), with no register staging; the plain form, or at device scope (sc1) for an earlier
// phase's output.  The compiler does not track these loads: completion is waited for with an
// explicit vmcnt.  m0 is set in the statement and listed as clobbered; the compiler warns that it
// may not preserve a reserved register across it, and no compiler-generated code of the files that
// use it uses m0 (checked in their assembly), so nothing lives there to be lost.
__device__ __forceinline__ void dma16_lds(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_addr)
                 : "memory", "m0");
}
// The same with the non-temporal hint (streamed weights: read once per launch).
__device__ __forceinline__ void dma16_lds_nt(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "s"(lds_addr)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma16_lds_device(const void* base, uint32_t off, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 sc1" ::"v"(off), "s"(base), "s"(lds_addr)
                 : "memory", "m0");
}

}  // namespace nmi
