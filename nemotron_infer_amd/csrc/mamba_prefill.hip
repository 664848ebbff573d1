// mamba_prefill.hip -- the Mamba-2 mixer over a prompt (prefill) for gfx950: the causal conv1d
// with SiLU over the sequence, and the SSM scan, each sequence starting from a zero state and
// leaving its final conv / SSM state for decode.
//
// Contract of the reference's prefill path (nemotron_infer/csrc/include/model/
// mamba_block.cuh:346-425): with xBC the in_proj columns [INTER, INTER + CONV_DIM) (bf16),
//   conv:  c[t] = bf16(silu(b + w0 x[t-3] + w1 x[t-2] + w2 x[t-1] + w3 x[t])), x[t < 0] = 0;
//          final state [x[S-3], x[S-2], x[S-1]]   (ops/mamba2/causal_conv1d.cuh:30-90, 300-360)
//   scan:  dt_t = softplus(dt[t] + dt_bias) (20 / -20 cut-offs), S_t = S_{t-1} exp(-exp(A_log) dt_t)
//          + dt_t B_t x_t (S_{-1} = 0), y_t = bf16(S_t . C_t + D x_t); final state S_{S-1}
//          (ops/mamba2/ssd_scan_chunked.cuh:16-322: the same recurrence in chunked matrix form,
//          its matrix products in TF32).
// The scan runs in that chunked form by default (mamba_ssd_kernel, on bf16 MFMA with two-part
// operands; described at the kernel), or as the recurrence itself in float32 (mamba_scan_kernel,
// tuning knob mamba.scan = 1): one workgroup per (sequence, head, 8 rows of P), a 32-lane
// half-wave per row holding the row's N = 128 states (4 per lane), tokens in chunks staged in LDS
// (B and C of the head's group, x, dt and the decay), the next chunk's loads issued before the
// current chunk is scanned; per token and row 4 state FMAs, 4 output FMAs and a 32-lane sum.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <cfloat>
#include <type_traits>

namespace nmi {

namespace {

constexpr int kN = kMambaDState;       // 128
constexpr int kConvK = kMambaConvK;    // 4
constexpr int kRowsPerWg = 8;          // SSM rows (p) per workgroup: 4 waves x 2 half-waves
constexpr int kTC = 32;                // tokens per staged chunk
constexpr int kConvT = 16;             // tokens per conv thread

__device__ __forceinline__ float silu(float v) { return v / (1.f + expf(-v)); }

// One thread per (channel, 16-token run): the conv with a 3-value window, SiLU, bf16.  The run's
// 19 inputs (3 before it) are all loaded before the first output is formed, so a thread waits for
// one memory round trip rather than one per token.
__global__ __launch_bounds__(256) void mamba_conv_prefill_kernel(const MambaPrefillArgs a) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int t0 = blockIdx.y * kConvT;
    const int b = blockIdx.z;
    if (c >= a.conv_dim || t0 >= a.S) return;
    const int n = min(kConvT, a.S - t0);
    const uint16_t* xin = a.proj + (size_t)b * a.S * a.proj_ld + a.inter + c;   // column c of xBC
    uint16_t* out = a.xc + (size_t)b * a.S * a.xc_ld + c;
    const float4 w = *reinterpret_cast<const float4*>(a.conv_w + (size_t)c * kConvK);
    const float bias = a.conv_b[c];
    float v[kConvT + 3];                                        // tokens t0 - 3 .. t0 + kConvT - 1
#pragma unroll
    for (int k = 0; k < kConvT + 3; ++k) {
        const int t = t0 - 3 + k;
        v[k] = (t >= 0 && k < n + 3) ? bf16_to_f32(xin[(size_t)t * a.proj_ld]) : 0.f;
    }
#pragma unroll
    for (int k = 0; k < kConvT; ++k) {
        if (k >= n) break;
        float acc = bias;
        acc = __builtin_fmaf(w.x, v[k], acc);
        acc = __builtin_fmaf(w.y, v[k + 1], acc);
        acc = __builtin_fmaf(w.z, v[k + 2], acc);
        acc = __builtin_fmaf(w.w, v[k + 3], acc);
        out[(size_t)(t0 + k) * a.xc_ld] = f32_to_bf16_rne(silu(acc));
    }
    if (t0 + n == a.S && a.conv_state) {
        float* st = a.conv_state + ((size_t)b * a.conv_dim + c) * (kConvK - 1);
        // the last three inputs: tokens S - 3 .. S - 1 (zero before the sequence)
#pragma unroll
        for (int e = 0; e < 3; ++e) {
            float val = 0.f;
#pragma unroll
            for (int k = 0; k < kConvT + 3; ++k)
                if (k == n + e) val = v[k];
            st[e] = val;
        }
    }
}

// SiLU from the hardware exp2 and reciprocal (a few float32 ulp from v / (1 + exp(-v)); the
// result is rounded to bf16): -inf and +inf limits hold (exp2 overflows to inf, its reciprocal to 0).
__device__ __forceinline__ float silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * v));
}

// Vector form (row strides and the xBC column offset 16-byte aligned): one thread per (8
// channels, 16-token run), 16-byte loads and stores of 8 channels; the run's 19 input rows are
// all loaded before the first output is formed.
__global__ __launch_bounds__(256) void mamba_conv_prefill_vec_kernel(const MambaPrefillArgs a) {
    const int c0 = 8 * (int)(blockIdx.x * 256 + threadIdx.x);
    const int t0 = blockIdx.y * kConvT;
    const int b = blockIdx.z;
    if (c0 >= a.conv_dim || t0 >= a.S) return;
    const int n = min(kConvT, a.S - t0);
    const uint16_t* xin = a.proj + (size_t)b * a.S * a.proj_ld + a.inter + c0;
    uint16_t* out = a.xc + (size_t)b * a.S * a.xc_ld + c0;
    uint4 v[kConvT + 3];                                        // tokens t0 - 3 .. t0 + kConvT - 1
#pragma unroll
    for (int k = 0; k < kConvT + 3; ++k) {
        const int t = t0 - 3 + k;
        v[k] = (t >= 0 && k < n + 3) ? load16(xin + (size_t)t * a.proj_ld) : uint4{0u, 0u, 0u, 0u};
    }
    float w[8][4], bias[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float4 wv = *reinterpret_cast<const float4*>(a.conv_w + (size_t)(c0 + e) * kConvK);
        w[e][0] = wv.x; w[e][1] = wv.y; w[e][2] = wv.z; w[e][3] = wv.w;
        bias[e] = a.conv_b[c0 + e];
    }
    auto ch = [](const uint4& q, int e) {                       // channel e of a row of 8
        const uint32_t d = e < 2 ? q.x : e < 4 ? q.y : e < 6 ? q.z : q.w;
        return e & 1 ? bf16hi_to_f32(d) : bf16lo_to_f32(d);
    };
#pragma unroll
    for (int k = 0; k < kConvT; ++k) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float acc = bias[e];
            acc = __builtin_fmaf(w[e][0], ch(v[k], e), acc);
            acc = __builtin_fmaf(w[e][1], ch(v[k + 1], e), acc);
            acc = __builtin_fmaf(w[e][2], ch(v[k + 2], e), acc);
            acc = __builtin_fmaf(w[e][3], ch(v[k + 3], e), acc);
            o[e] = silu_fast(acc);
        }
        if (k < n)
            *reinterpret_cast<uint4*>(out + (size_t)(t0 + k) * a.xc_ld) =
                uint4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])};
    }
    if (t0 + n == a.S && a.conv_state) {
        // the last three inputs of each channel: tokens S - 3 .. S - 1 (zero before the sequence),
        // read again (picking them from v by a run-time index would put v in scratch memory)
        uint4 last[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int t = a.S - 3 + j;
            last[j] = t >= 0 ? load16(xin + (size_t)t * a.proj_ld) : uint4{0u, 0u, 0u, 0u};
        }
        float* st = a.conv_state + ((size_t)b * a.conv_dim + c0) * (kConvK - 1);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int j = 0; j < 3; ++j) st[3 * e + j] = ch(last[j], e);
    }
}

// Scan: one workgroup per (sequence, head, 8 rows of P), a 32-lane half-wave per row with the
// row's N = 128 float32 states (4 per lane).  Tokens go in chunks of kTC = 32 staged in LDS: dt
// (softplus) and the decay per token, then dt.B and C in float32 (each computed once per chunk
// for all 8 rows, not per row and token), x per row; the next chunk's loads are in flight during
// the scan.  Per token a lane updates its 4 states, s = fma(s, dA, (dt B) x), and forms its
// 4-state part of y = S . C, summed over the half-wave (16-lane DPP sum, then lane 16 apart).
__global__ __launch_bounds__(256, 4) void mamba_scan_kernel(const MambaPrefillArgs a) {
    __shared__ __attribute__((aligned(16))) float sdtB[kTC][kN];
    __shared__ __attribute__((aligned(16))) float sC[kTC][kN];
    __shared__ __attribute__((aligned(16))) uint16_t sx[kTC][kRowsPerWg];
    __shared__ float sdt[kTC], sdA[kTC];
    __shared__ float sy[kTC][kRowsPerWg];

    const int splits = (a.P + kRowsPerWg - 1) / kRowsPerWg;
    const int h = blockIdx.x / splits, p0 = (blockIdx.x % splits) * kRowsPerWg;
    const int b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hw = lane >> 5, l = lane & 31;
    const int r = 2 * wave + hw;                                // this half-wave's row
    const int grp = h / (a.H / a.G);
    const int S = a.S;
    const size_t xrow0 = (size_t)b * S;                         // first token row of the sequence
    const float nA = -expf(a.A_log[h]);
    const float bias = a.dt_bias[h];
    const float Dh = a.D[h];
    const bool row_ok = p0 + r < a.P;
    const int nrows_wg = min(kRowsPerWg, a.P - p0);

    // chunk staging: B and C rows of kTC tokens (16 chunks of 16 B per token: 512 per chunk, 2 per
    // thread each), x (threads < kTC: 8 values, or fewer at the last split), dt (threads < kTC)
    uint4 rb[2], rc[2], rx;
    uint16_t rdt;
    auto gload = [&](int t0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = tid + 256 * u;
            const int t = min(t0 + (i >> 4), S - 1), c = i & 15;
            const uint16_t* row = a.xc + (xrow0 + t) * a.xc_ld + a.inter;
            rb[u] = load16(row + grp * kN + 8 * c);
            rc[u] = load16(row + a.G * kN + grp * kN + 8 * c);
        }
        if (tid < kTC) {
            const int t = min(t0 + tid, S - 1);
            const uint16_t* xr = a.xc + (xrow0 + t) * a.xc_ld + h * a.P + p0;
            if (nrows_wg == kRowsPerWg && a.x_vec) {
                rx = load16(xr);
            } else {
                uint16_t v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = e < nrows_wg ? xr[e] : 0;
                rx = uint4{v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16), v[4] | ((uint32_t)v[5] << 16),
                           v[6] | ((uint32_t)v[7] << 16)};
            }
            rdt = a.proj[(xrow0 + t) * a.proj_ld + a.inter + a.conv_dim + h];
        }
    };
    // Tokens past the end of the sequence get dt = 0, decay 1 and x = 0: their updates leave the
    // states exactly as they are (fma(s, 1, 0) = s).
    auto sstore = [&](int nt) {
        if (tid < kTC) {
            const bool live = tid < nt;
            *reinterpret_cast<uint4*>(&sx[tid][0]) = live ? rx : uint4{0u, 0u, 0u, 0u};
            float dt = bf16_to_f32(rdt) + bias;
            dt = dt > 20.f ? dt : (dt < -20.f ? 0.f : logf(1.f + expf(dt)));
            dt = fminf(FLT_MAX, fmaxf(0.f, dt));
            sdt[tid] = live ? dt : 0.f;
            sdA[tid] = live ? expf(nA * dt) : 1.f;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int i = tid + 256 * u;
            const int t = i >> 4, c = i & 15;
            const float dt = sdt[t];
            const uint32_t bw[4] = {rb[u].x, rb[u].y, rb[u].z, rb[u].w};
            const uint32_t cw[4] = {rc[u].x, rc[u].y, rc[u].z, rc[u].w};
            float db[8], cf[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                db[2 * e] = dt * bf16lo_to_f32(bw[e]);
                db[2 * e + 1] = dt * bf16hi_to_f32(bw[e]);
                cf[2 * e] = bf16lo_to_f32(cw[e]);
                cf[2 * e + 1] = bf16hi_to_f32(cw[e]);
            }
            *reinterpret_cast<f32x4*>(&sdtB[t][8 * c]) = f32x4{db[0], db[1], db[2], db[3]};
            *reinterpret_cast<f32x4*>(&sdtB[t][8 * c + 4]) = f32x4{db[4], db[5], db[6], db[7]};
            *reinterpret_cast<f32x4*>(&sC[t][8 * c]) = f32x4{cf[0], cf[1], cf[2], cf[3]};
            *reinterpret_cast<f32x4*>(&sC[t][8 * c + 4]) = f32x4{cf[4], cf[5], cf[6], cf[7]};
        }
    };

    float s[4] = {0.f, 0.f, 0.f, 0.f};
    gload(0);
    for (int t0 = 0; t0 < S; t0 += kTC) {
        const int nt = min(kTC, S - t0);
        sstore(nt);
        __syncthreads();
        if (t0 + kTC < S) gload(t0 + kTC);                     // the next chunk, in flight during the scan
#pragma unroll 4
        for (int t = 0; t < kTC; ++t) {
            const f32x4 db = *reinterpret_cast<const f32x4*>(&sdtB[t][4 * l]);
            const f32x4 c = *reinterpret_cast<const f32x4*>(&sC[t][4 * l]);
            const float x = bf16_to_f32(sx[t][r]);
            const float dA = sdA[t];
            float y = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                s[i] = __builtin_fmaf(s[i], dA, db[i] * x);
                y = __builtin_fmaf(s[i], c[i], y);
            }
            y = dpp_row_sum16(y);
            y += __shfl_xor(y, 16);
            if (l == 0) sy[t][r] = __builtin_fmaf(Dh, x, y);
        }
        __syncthreads();
        // the chunk's outputs: token t, rows p0 .. p0 + 7 (contiguous in y)
        if (tid < nt) {
            uint16_t* yr = a.y + (xrow0 + t0 + tid) * a.y_ld + h * a.P + p0;
            if (nrows_wg == kRowsPerWg && a.y_vec) {
                const float* vv = sy[tid];
                *reinterpret_cast<uint4*>(yr) = uint4{pack_bf16(vv[0], vv[1]), pack_bf16(vv[2], vv[3]),
                                                      pack_bf16(vv[4], vv[5]), pack_bf16(vv[6], vv[7])};
            } else {
                for (int e = 0; e < nrows_wg; ++e) yr[e] = f32_to_bf16_rne(sy[tid][e]);
            }
        }
    }
    if (a.ssm_state && row_ok) {
        float* st = a.ssm_state + (((size_t)b * a.H + h) * a.P + p0 + r) * kN + 4 * l;
        *reinterpret_cast<float4*>(st) = float4{s[0], s[1], s[2], s[3]};
    }
}

// Chunked scan (the default): the same recurrence in the chunked matrix form of the reference's
// ssd_scan_chunked.cuh, on bf16 MFMA.  One workgroup per (sequence, head, 16 rows of P), 64-token
// chunks in order; with c_i = sum_{k <= i} dt_k A over the chunk (A = -exp(A_log); kept in log2
// units), S0 the state entering it (rows p, columns n) and w_j = exp(c_63 - c_j) dt_j:
//   y_i  = exp(c_i) (C_i . S0[p, :]) + sum_{j <= i} G_ij x_j + D x_i,
//          G_ij = (C_i . B_j) exp(c_i - c_j) dt_j
//   S    = exp(c_63) S0 + sum_j (w_j x_j) B_j^T.
// All products on v_mfma_f32_16x16x32_bf16: C B^T exact bf16 products with float32 sums; G, S0
// and w x enter their products in two bf16 parts (hi = bf16(v), lo = bf16(v - hi): about 16
// significant bits, finer than the reference's TF32 products) against exact bf16 x, C and B; the
// state accumulates in float32 MFMA registers across chunks.  Each wave forms the G rows of its
// own 16 tokens and uses them straight from the MFMA output registers, so per chunk only the
// staging of B, C and x and the state's two-part copy go through a barrier.
// Each SIMD issues a wave64 VALU instruction over 4 cycles, so the per-element work is kept on
// MFMA: what remains on VALU per chunk is the decay weights, the G mask and the two-part splits.
// Tokens past the end of the sequence get dt = 0 and x = 0: no weight, no decay.
constexpr int kQ = 64;                 // tokens per chunk
constexpr int kPW = 16;                // rows of P per workgroup

// LDS (bytes): B and C chunks [64][128] bf16 (256-byte rows, 16-byte chunk c at c ^ (row & 15));
// the x chunk [64][16] bf16 (32-byte rows); S0 hi / lo [16][128] bf16 (chunk at c ^ (p & 15)), two
// buffers (chunk parity); two sets (chunk parity) of the per-token float32 arrays cum, ecum, w,
// dt.
constexpr int kOffB = 0, kOffC = 16384, kOffX = 32768, kOffS = 34816, kSBuf = 8192, kOffDec = kOffS + 2 * kSBuf,
              kDecSet = 4 * 256, kSsdLds = kOffDec + 2 * kDecSet;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
// v shifted right by K lanes within each row of 16 (0 where the source lies before the row)
template <int K>
__device__ __forceinline__ float row_shr(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x110 + K, 0xf, 0xf, true));
}
// Inclusive prefix sum over the 64 lanes: a scan within each row of 16 by DPP row shifts, then
// the totals of the rows before (read from lanes 15, 31, 47).
__device__ __forceinline__ float wave_incl_sum(float v) {
    v += row_shr<1>(v);
    v += row_shr<2>(v);
    v += row_shr<4>(v);
    v += row_shr<8>(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 47));
    const int row = (threadIdx.x & 63) >> 4;
    const float add = row == 0 ? 0.f : row == 1 ? r0 : row == 2 ? r0 + r1 : r0 + r1 + r2;
    return v + add;
}
__device__ __forceinline__ int bc_off(int row, int c) { return row * 256 + ((c ^ (row & 15)) << 4); }
__device__ __forceinline__ int t_off(int row, int c) { return row * 128 + ((c ^ ((row >> 1) & 7)) << 4); }
__device__ __forceinline__ int s_off(int p, int c) { return p * 256 + ((c ^ (p & 15)) << 4); }

__global__ __launch_bounds__(256, 2) void mamba_ssd_kernel(const MambaPrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int slices = (a.P + kPW - 1) / kPW;
    const int h = blockIdx.x / slices, p0 = (blockIdx.x % slices) * kPW;
    const int b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g4 = lane >> 4;                  // 16x16x32 operand layout
    const int grp = h / (a.H / a.G);
    const int S = a.S;
    const int pw = min(kPW, a.P - p0);
    const size_t xrow0 = (size_t)b * S;
    const float nA2 = -expf(a.A_log[h]) * 1.4426950408889634f;   // A in log2 units
    const float bias = a.dt_bias[h];
    const float Dh = a.D[h];
    // the decay arrays of set k (chunk parity): cum = c_j (log2 units), ecum = exp(c_j), wj =
    // exp(c_63 - c_j) dt_j, dts = dt_j
    auto dec_arr = [&](int k, int i) __attribute__((always_inline)) { return reinterpret_cast<float*>(lds + kOffDec + k * kDecSet + i * 256); };

    // chunk staging in registers (the next chunk's loads are in flight during this one): B and C
    // rows (1024 chunks of 16 B each: 4 per thread), x (threads < 128: token tid / 2, P columns
    // 8 (tid % 2) .. + 7 of the slice)
    uint4 rb[4], rc[4], rx = uint4{0u, 0u, 0u, 0u};
    auto gload = [&](int t0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = tid + 256 * u;
            const int t = min(t0 + (q >> 4), S - 1), c = q & 15;
            const uint16_t* row = a.xc + (xrow0 + t) * a.xc_ld + a.inter;
            rb[u] = load16(row + grp * kN + 8 * c);
            rc[u] = load16(row + a.G * kN + grp * kN + 8 * c);
        }
        if (tid < 2 * kQ) {
            const int t = min(t0 + (tid >> 1), S - 1), pc = 8 * (tid & 1);
            const uint16_t* xr = a.xc + (xrow0 + t) * a.xc_ld + h * a.P + p0 + pc;
            if (a.x_vec && pc + 8 <= pw) {
                rx = load16(xr);
            } else {
                uint16_t v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = pc + e < pw ? xr[e] : 0;
                rx = uint4{v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16), v[4] | ((uint32_t)v[5] << 16),
                           v[6] | ((uint32_t)v[7] << 16)};
            }
        }
    };
    // dt of the chunk at t0 (wave 1 scans it one chunk ahead of its use)
    auto load_dt = [&](int t0) __attribute__((always_inline)) {
        return a.proj[(xrow0 + min(t0 + lane, S - 1)) * a.proj_ld + a.inter + a.conv_dim + h];
    };
    // Wave 1: softplus(dt + bias) (the reference's cut-offs) and the chunk's inclusive cumulative
    // log2-decay (finite even where dt saturates: a decay that small is a reset either way), into
    // decay set k; tokens at or past nt get dt = 0.
    auto scan = [&](uint16_t dtb, int nt, int k) __attribute__((always_inline)) {
        float dt = bf16_to_f32(dtb) + bias;
        dt = dt > 20.f ? dt : (dt < -20.f ? 0.f : logf(1.f + expf(dt)));
        dt = fminf(FLT_MAX, fmaxf(0.f, dt));
        if (lane >= nt) dt = 0.f;
        const float v = wave_incl_sum(fmaxf(nA2 * dt, -1e30f));
        const float last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
        dec_arr(k, 0)[lane] = v;
        dec_arr(k, 1)[lane] = fexp2(v);
        dec_arr(k, 2)[lane] = fexp2(last - v) * dt;
        dec_arr(k, 3)[lane] = dt;
    };
    // Transposing LDS reads (ds_read_b64_tr_b16: in each 16-lane group, output lane 4 a + b, element
    // e is element b of source lane 4 e + a's 8 bytes).  B^T as the A operand: rows n = n0 + l16,
    // tokens 32 ks + 8 g4 + {0..7} (source lane s reads token row 32 ks + 8 g4 + 4 q + s / 4,
    // columns n0 + 4 (s % 4) .. + 3).
    auto bt_frag = [&](int n0, int ks) __attribute__((always_inline)) {
        v4i16 v[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int j = 32 * ks + 8 * g4 + 4 * q + (l16 >> 2);
            const int n = n0 + 4 * (l16 & 3);
            v[q] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lds + kOffB + bc_off(j, n >> 3) + 2 * (n & 7)));
        }
        return __builtin_bit_cast(bf16x8, __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // x^T: the four tokens j0 .. j0 + 3 of column p = l16 (j0 a multiple of 4) from the row-major
    // x chunk (32-byte rows; source lane s reads row j0 + s / 4, columns 4 (s % 4) .. + 3)
    auto xt4 = [&](int j0) __attribute__((always_inline)) {
        return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(lds + kOffX + (j0 + (l16 >> 2)) * 32 + 8 * (l16 & 3)));
    };
    auto split = [&](const float (&v)[8], bf16x8& hi, bf16x8& lo) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const uint32_t w = pack_bf16(v[e], v[e + 1]);
            hw[e >> 1] = w;
            lw[e >> 1] = pack_bf16(v[e] - __uint_as_float(w << 16), v[e + 1] - __uint_as_float(w & 0xffff0000u));
        }
        hi = __builtin_bit_cast(bf16x8, uint4{hw[0], hw[1], hw[2], hw[3]});
        lo = __builtin_bit_cast(bf16x8, uint4{lw[0], lw[1], lw[2], lw[3]});
    };

    // the state, transposed, as two 16 x 16 MFMA accumulator blocks per wave: rows n = 16 (2 wave +
    // nb) + 4 g4 + r, columns p = l16
    f32x4 st[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) st[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // S0 hi / lo of the first chunk (buffer 0): zero (thread t clears 16 bytes of each)
    *reinterpret_cast<uint4*>(lds + kOffS + 16 * tid) = uint4{0u, 0u, 0u, 0u};
    *reinterpret_cast<uint4*>(lds + kOffS + 4096 + 16 * tid) = uint4{0u, 0u, 0u, 0u};

    gload(0);
    // dt two chunks ahead (wave 1): chunk 0 scanned here, chunk c + 1 during chunk c
    uint16_t rdt1 = 0, rdt2 = 0;
    if (wave == 1) {
        const uint16_t rdt0 = load_dt(0);
        rdt1 = load_dt(kQ);
        scan(rdt0, min(kQ, S), 0);
    }
    // One chunk: (a) the staged chunk into LDS (B, C row-major; x row-major, zero past the
    // sequence), the next chunk's loads, barrier; then each wave on its own (no barrier): rows
    // i = 16 wave + l16 of G and y, rows n = 32 wave .. + 31 of the state; the new state's two-part
    // copy into the other S0 buffer; barrier.  rcur holds the next chunk's dt (wave 1), rnext
    // receives the one after it (register roles alternate between calls: no copy waits on a load).
    auto chunk = [&](auto W, int t0, uint16_t& rcur, uint16_t& rnext) __attribute__((always_inline)) {
        constexpr int w = decltype(W)::value;                    // this wave (a constant per instantiation)
        const int par = (t0 / kQ) & 1;
        const float* cum = dec_arr(par, 0);
        const float* ecum = dec_arr(par, 1);
        const float* wj = dec_arr(par, 2);
        const float* dts = dec_arr(par, 3);
        const int nt = min(kQ, S - t0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = tid + 256 * u;
            const int j = q >> 4, cc = q & 15;
            *reinterpret_cast<uint4*>(lds + kOffB + bc_off(j, cc)) = rb[u];
            *reinterpret_cast<uint4*>(lds + kOffC + bc_off(j, cc)) = rc[u];
        }
        if (tid < 2 * kQ) {
            const int j = tid >> 1, pc = 8 * (tid & 1);
            *reinterpret_cast<uint4*>(lds + kOffX + j * 32 + 2 * pc) = j < nt ? rx : uint4{0u, 0u, 0u, 0u};
        }
        if (t0 + kQ < S) gload(t0 + kQ);
        if (w == 1 && t0 + 2 * kQ < S) rnext = load_dt(t0 + 2 * kQ);
        __syncthreads();

        // wave 1: the next chunk's decay into the other set (its last readers finished before the
        // previous chunk's closing barrier)
        if (w == 1 && t0 + kQ < S) scan(rcur, min(kQ, S - t0 - kQ), par ^ 1);

        const int i = 16 * w + l16;                              // this lane's token row of G and y
        // C rows i as the B operand (k = n): used by C B^T and by S0 C^T
        bf16x8 cf[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) cf[ks] = *reinterpret_cast<const bf16x8*>(lds + kOffC + bc_off(i, 4 * ks + g4));
        // (C_i . B_j) for the token blocks jb <= w: lane (column i, g4) holds j = 16 jb + 4 g4 + r
        f32x4 cb[w + 1];
#pragma unroll
        for (int jb = 0; jb <= w; ++jb) {
            cb[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 bf = *reinterpret_cast<const bf16x8*>(lds + kOffB + bc_off(16 * jb + l16, 4 * ks + g4));
                cb[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, cf[ks], cb[jb], 0, 0, 0);
            }
        }
        // y^T (rows p = 4 g4 + r, column i) = exp(c_i) (S0 C^T) + x^T G^T + D x
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        {
            const uint8_t* s0 = lds + kOffS + par * kSBuf;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const bf16x8 sh = *reinterpret_cast<const bf16x8*>(s0 + s_off(l16, 4 * ks + g4));
                const bf16x8 sl = *reinterpret_cast<const bf16x8*>(s0 + 4096 + s_off(l16, 4 * ks + g4));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sh, cf[ks], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sl, cf[ks], acc, 0, 0, 0);
            }
        }
        const float ei = ecum[i];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= ei;
        // G_ij = (C_i . B_j) exp2(min(c_i - c_j, 0)) dt_j on and below the diagonal (one exp2 per
        // element: no factorisation, so no range test and no branch), in two bf16 parts, as the
        // B operand of pairs of token blocks (k = 8 g4 + 4 q + r <-> j = 16 (2 m + q) + 4 g4 + r), times
        // the matching x^T (two transposing reads)
        {
            const float ci = cum[i];
#pragma unroll
            for (int m = 0; 2 * m <= w; ++m) {
                {
                    float gv[8];
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const int jb = 2 * m + q;
                        const int j0 = 16 * jb + 4 * g4;
                        if (jb <= w) {
                            const f32x4 cj = *reinterpret_cast<const f32x4*>(cum + j0);
                            const f32x4 dj = *reinterpret_cast<const f32x4*>(dts + j0);
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                gv[4 * q + r] = j0 + r <= i ? cb[jb][r] * fexp2(fminf(ci - cj[r], 0.f)) * dj[r] : 0.f;
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r) gv[4 * q + r] = 0.f;
                        }
                    }
                    bf16x8 gh, gl;
                    split(gv, gh, gl);
                    const v4i16 x0 = xt4(32 * m + 4 * g4), x1 = xt4(32 * m + 16 + 4 * g4);
                    const bf16x8 xf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf, gh, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf, gl, acc, 0, 0, 0);
                }
            }
        }
        {
            // + D x: x[i][4 g4 .. + 3]; y[i][p0 + 4 g4 + r]
            const uint2 xv = *reinterpret_cast<const uint2*>(lds + kOffX + i * 32 + 8 * g4);
            const float xf[4] = {bf16lo_to_f32(xv.x), bf16hi_to_f32(xv.x), bf16lo_to_f32(xv.y), bf16hi_to_f32(xv.y)};
            float yv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) yv[r] = __builtin_fmaf(Dh, xf[r], acc[r]);
            if (i < nt) {
                uint16_t* yp = a.y + (xrow0 + t0 + i) * a.y_ld + h * a.P + p0 + 4 * g4;
                if (a.y_vec && 4 * g4 + 4 <= pw) {
                    *reinterpret_cast<uint2*>(yp) = uint2{pack_bf16(yv[0], yv[1]), pack_bf16(yv[2], yv[3])};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (4 * g4 + r < pw) yp[r] = (uint16_t)pack_bf16(yv[r], 0.f);
                }
            }
        }
        // S^T = exp(c_63) S0^T + B^T (w x): rows n = 16 (2 wave + nb) + 4 g4 + r, columns p = l16; A =
        // B^T (transposing reads of B), B = (w x) in two parts (k = 8 g4 + 4 q + e <-> token
        // 32 ks + 8 g4 + 4 q + e, x^T by transposing reads)
        {
            const float dec = ecum[kQ - 1];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r) st[nb][r] *= dec;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                float wv[8];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int j0 = 32 * ks + 8 * g4 + 4 * q;
                    const v4i16 xq = xt4(j0);
                    const f32x4 w4 = *reinterpret_cast<const f32x4*>(wj + j0);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        wv[4 * q + e] = bf16_to_f32((uint16_t)xq[e]) * w4[e];
                }
                bf16x8 wh, wl;
                split(wv, wh, wl);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    const bf16x8 ab = bt_frag(16 * (2 * w + nb), ks);
                    st[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, wh, st[nb], 0, 0, 0);
                    st[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, wl, st[nb], 0, 0, 0);
                }
            }
            // the new state's two bf16 parts into the other S0 buffer (its readers, the previous
            // chunk, finished before that chunk's closing barrier): four consecutive n of row p =
            // l16 per block
            uint8_t* s1 = lds + kOffS + (par ^ 1) * kSBuf;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int n0 = 16 * (2 * w + nb) + 4 * g4;
                const f32x4 v = st[nb];
                const uint32_t h01 = pack_bf16(v[0], v[1]), h23 = pack_bf16(v[2], v[3]);
                const uint32_t l01 = pack_bf16(v[0] - __uint_as_float(h01 << 16), v[1] - __uint_as_float(h01 & 0xffff0000u));
                const uint32_t l23 = pack_bf16(v[2] - __uint_as_float(h23 << 16), v[3] - __uint_as_float(h23 & 0xffff0000u));
                const int off = s_off(l16, n0 >> 3) + 2 * (n0 & 7);
                *reinterpret_cast<uint2*>(s1 + off) = uint2{h01, h23};
                *reinterpret_cast<uint2*>(s1 + 4096 + off) = uint2{l01, l23};
            }
        }
        __syncthreads();
    };
    // each wave runs a loop specialised to its index (the same barriers in every instantiation)
    auto run = [&](auto W) __attribute__((always_inline)) {
        for (int t0 = 0; t0 < S; t0 += 2 * kQ) {
            chunk(W, t0, rdt1, rdt2);
            if (t0 + kQ < S) chunk(W, t0 + kQ, rdt2, rdt1);
        }
    };
    switch (wave) {
        case 0: run(std::integral_constant<int, 0>{}); break;
        case 1: run(std::integral_constant<int, 1>{}); break;
        case 2: run(std::integral_constant<int, 2>{}); break;
        default: run(std::integral_constant<int, 3>{}); break;
    }
    if (a.ssm_state && l16 < pw) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int n0 = 16 * (2 * wave + nb) + 4 * g4;
            *reinterpret_cast<float4*>(a.ssm_state + (((size_t)b * a.H + h) * a.P + p0 + l16) * kN + n0) =
                float4{st[nb][0], st[nb][1], st[nb][2], st[nb][3]};
        }
    }
}

}  // namespace

hipError_t launch_mamba_prefill_mixer(const MambaPrefillArgs& a, int batch, hipStream_t stream) {
    const bool vec = a.conv_dim % 8 == 0 && a.inter % 8 == 0 && a.proj_ld % 8 == 0 && a.xc_ld % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(a.proj) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.xc) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.conv_w) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL(mamba_conv_prefill_vec_kernel,
                           dim3((a.conv_dim / 8 + 255) / 256, (a.S + kConvT - 1) / kConvT, batch), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(mamba_conv_prefill_kernel, dim3((a.conv_dim + 255) / 256, (a.S + kConvT - 1) / kConvT, batch),
                           dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (tuning().mamba_scan == 1) {
        const int splits = (a.P + kRowsPerWg - 1) / kRowsPerWg;
        hipLaunchKernelGGL(mamba_scan_kernel, dim3(a.H * splits, batch), dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&mamba_ssd_kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kSsdLds);
    if (attr != hipSuccess) return attr;
    const int slices = (a.P + kPW - 1) / kPW;
    hipLaunchKernelGGL(mamba_ssd_kernel, dim3(a.H * slices, batch), dim3(256), kSsdLds, stream, a);
    return hipGetLastError();
}

}  // namespace nmi
