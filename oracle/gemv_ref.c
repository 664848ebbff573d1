/*
 * gemv_ref.c -- plain-C restatement of the reference's CPU GEMV checker.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and by bench.py's cpu_baseline leg through
 * oracle/cref.py; never linked into the product library.
 *
 *   oracle_e4m3_decode   closed-form OCP E4M3 decode (bias 7, subnormal m*2^-9,
 *                        NaN at S.1111.111, no inf); the value the reference obtains from
 *                        static_cast<float>(__nv_fp8_e4m3) (ops/gemv.cuh:40-42).
 *   oracle_gemv_fp8_seq  tests/ops/test_gemm.cu:505-513: for every row n,
 *                        sum += float(W[n,k]) * float(x[k]) in k order (float32, no FMA
 *                        contraction), then y[n] = sum * w_scale[n]; repeated per M row.
 *   oracle_bf16_rne      __float2bfloat16_rn (ops/gemv.cuh:88): round to nearest even.
 *
 * Built with -ffp-contract=off so that the multiply and the add round separately, as the
 * reference's host loop does.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stddef.h>

float oracle_e4m3_decode(uint8_t b) {
    const int sign = (b >> 7) & 1;
    const int e = (b >> 3) & 0xF;
    const int m = b & 0x7;
    float v;
    if (e == 0xF && m == 0x7) {
        uint32_t bits = sign ? 0xFFC00000u : 0x7FC00000u;
        memcpy(&v, &bits, 4);
        return v;
    }
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sign ? -v : v;
}

void oracle_e4m3_lut(float* out256) {
    for (int b = 0; b < 256; ++b) out256[b] = oracle_e4m3_decode((uint8_t)b);
}

static float bf16_bits_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void oracle_gemv_fp8_seq(const uint16_t* x, const uint8_t* W, const float* w_scale,
                         float* y, int M, int N, int K) {
    float lut[256];
    oracle_e4m3_lut(lut);
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (size_t)m * K;
        for (int n = 0; n < N; ++n) {
            const uint8_t* wr = W + (size_t)n * K;
            float sum = 0.f;
            for (int k = 0; k < K; ++k) {
                float prod = lut[wr[k]] * bf16_bits_to_f32(xr[k]);
                sum = sum + prod;
            }
            y[(size_t)m * N + n] = sum * w_scale[n];
        }
    }
}

void oracle_bf16_rne(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &in[i], 4);
        if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) {
            out[i] = (uint16_t)(0x7FC0u | ((u >> 16) & 0x8000u));
            continue;
        }
        u = u + 0x7FFFu + ((u >> 16) & 1u);
        out[i] = (uint16_t)(u >> 16);
    }
}
