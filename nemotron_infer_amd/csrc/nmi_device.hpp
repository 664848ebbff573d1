// nmi_device.hpp -- gfx950 (CDNA4) device helpers shared by the fp8 W8A16 kernels.
//
// * e4m3 -> f32 decode through v_cvt_pk_f32_fp8 (OCP E4M3 on gfx950), four codes per dword,
//   byte b of the dword -> element b.  This is the value static_cast<float>(__nv_fp8_e4m3)
//   gives in the reference (nemotron_infer/csrc/include/ops/gemv.cuh:40-42).
// * e4m3 -> bf16 decode through v_cvt_scalef32_pk_bf16_fp8 with scale 1.0; every e4m3 value is
//   exactly representable in bf16, so this is exact (used to stage weight tiles for MFMA).
// * bf16 -> f32 by shifting the bit pattern; f32 -> bf16 round-to-nearest-even through
//   v_cvt_pk_bf16_f32 (the conversion __float2bfloat16_rn performs in gemv.cuh:88).
// * a 16-lane sum that uses DPP row operations (quad_perm, row_half_mirror, row_mirror), and
//   a 64-lane sum built on it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nmi {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Four e4m3 codes packed little-endian in `w` -> four floats.
__device__ __forceinline__ f32x4 e4m3x4_to_f32(uint32_t w) {
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);  // bytes 0, 1
    const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);   // bytes 2, 3
    return f32x4{lo.x, lo.y, hi.x, hi.y};
}

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

}  // namespace nmi
