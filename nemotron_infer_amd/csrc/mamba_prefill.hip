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
// The scan here is the recurrence itself, in float32 throughout: one workgroup per (sequence,
// head, 8 rows of P), a 32-lane half-wave per row holding the row's N = 128 states (4 per lane),
// tokens in chunks of 64 staged in LDS (B and C of the head's group, x, dt and the decay), the
// next chunk's loads issued before the current chunk is scanned.  Per token and row: 4 state
// FMAs, 4 output FMAs and a 32-lane sum; parallel over B x H x P rows (7680 at the model's size).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <cfloat>

namespace nmi {

namespace {

constexpr int kN = kMambaDState;       // 128
constexpr int kConvK = kMambaConvK;    // 4
constexpr int kRowsPerWg = 8;          // SSM rows (p) per workgroup: 4 waves x 2 half-waves
constexpr int kTC = 32;                // tokens per staged chunk
constexpr int kConvT = 64;             // tokens per conv thread

__device__ __forceinline__ float silu(float v) { return v / (1.f + expf(-v)); }

// One thread per (channel, 64-token run): the conv with a 3-value window, SiLU, bf16.
__global__ __launch_bounds__(256) void mamba_conv_prefill_kernel(const MambaPrefillArgs a) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int t0 = blockIdx.y * kConvT;
    const int b = blockIdx.z;
    if (c >= a.conv_dim || t0 >= a.S) return;
    const int t1 = min(t0 + kConvT, a.S);
    const uint16_t* xin = a.proj + (size_t)b * a.S * a.proj_ld + a.inter + c;   // column c of xBC
    uint16_t* out = a.xc + (size_t)b * a.S * a.xc_ld + c;
    const float4 w = *reinterpret_cast<const float4*>(a.conv_w + (size_t)c * kConvK);
    const float bias = a.conv_b[c];
    float s0 = t0 >= 3 ? bf16_to_f32(xin[(size_t)(t0 - 3) * a.proj_ld]) : 0.f;
    float s1 = t0 >= 2 ? bf16_to_f32(xin[(size_t)(t0 - 2) * a.proj_ld]) : 0.f;
    float s2 = t0 >= 1 ? bf16_to_f32(xin[(size_t)(t0 - 1) * a.proj_ld]) : 0.f;
    for (int t = t0; t < t1; ++t) {
        const float xt = bf16_to_f32(xin[(size_t)t * a.proj_ld]);
        float acc = bias;
        acc = __builtin_fmaf(w.x, s0, acc);
        acc = __builtin_fmaf(w.y, s1, acc);
        acc = __builtin_fmaf(w.z, s2, acc);
        acc = __builtin_fmaf(w.w, xt, acc);
        out[(size_t)t * a.xc_ld] = f32_to_bf16_rne(silu(acc));
        s0 = s1;
        s1 = s2;
        s2 = xt;
    }
    if (t1 == a.S && a.conv_state) {
        float* st = a.conv_state + ((size_t)b * a.conv_dim + c) * (kConvK - 1);
        st[0] = s0;
        st[1] = s1;
        st[2] = s2;
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

}  // namespace

hipError_t launch_mamba_prefill_mixer(const MambaPrefillArgs& a, int batch, hipStream_t stream) {
    hipLaunchKernelGGL(mamba_conv_prefill_kernel, dim3((a.conv_dim + 255) / 256, (a.S + kConvT - 1) / kConvT, batch),
                       dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int splits = (a.P + kRowsPerWg - 1) / kRowsPerWg;
    hipLaunchKernelGGL(mamba_scan_kernel, dim3(a.H * splits, batch), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace nmi
