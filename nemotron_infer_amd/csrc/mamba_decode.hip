// mamba_decode.hip -- the non-linear middle of the Mamba-2 mixer at decode (one token per
// sequence), for gfx950: causal conv1d step + SiLU, the SSM state update and its output, and the
// gated RMSNorm.  The block around it (mamba.cpp) runs in_proj before and out_proj after on
// the GEMV kernels.
//
// Contract of the reference's decode path (nemotron_infer/csrc/include/model/
// mamba_block.cuh:436-515): with proj = [z | xBC | dt] the in_proj output (bf16),
//   conv:  c = bf16(silu(b[c] + w[c,0] s0 + w[c,1] s1 + w[c,2] s2 + w[c,3] xBC[c])), the state
//          [s0, s1, s2] -> [s1, s2, xBC[c]]            (ops/mamba2/causal_conv1d.cuh:391-430)
//   ssm:   dt_h = softplus(dt[h] + dt_bias[h]) (20 / -20 cut-offs), dA = exp(-exp(A_log[h]) dt_h),
//          S[h,p,n] = S[h,p,n] dA + dt_h B[g,n] x[h,p];  y[h,p] = bf16(sum_n S[h,p,n] C[g,n]
//          + D[h] x[h,p]), g = h / (H / G)           (ops/mamba2/ssm.cuh:46-101)
//   norm:  u = y silu(z); per group of INTER / G: r = 1 / sqrt(mean(u^2) + eps);
//          out = bf16(u r w)                          (ops/reduce.cuh:383-480)
// with x, B, C the conv outputs (bf16) of channels [0, INTER), [INTER, INTER + G N),
// [INTER + G N, CONV_DIM).  States float32: conv [B, CONV_DIM, 3], ssm [B, H, P, N].
//
// Kernel 1 (one workgroup per (sequence, head, half of the head's P rows)): the conv of the
// head's B and C channels (every workgroup of a group recomputes the 256 channels from the old
// state -- cheaper than a launch), the conv of its own x channels (whose state it updates: each
// x channel belongs to one workgroup), then the SSM rows: a 32-lane half-wave per row of N = 128
// float32 state (16 bytes per lane, all rows of the workgroup loaded before any is computed).
// Kernel 2 (one workgroup per (group, sequence)): the gated RMSNorm in one pass, and the state
// update of the group's B and C channels, which kernel 1's workgroups all read (so it waits for
// the kernel boundary).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <cfloat>

namespace nmi {

namespace {

constexpr int kN = kMambaDState;       // 128
constexpr int kConvK = kMambaConvK;    // 4
constexpr int kSsmSplit = 2;           // workgroups per head
constexpr int kMaxRowsPerWave = 8;     // rows per half-wave at most (8 half-waves: 64 rows per workgroup)

__device__ __forceinline__ float silu(float v) { return v / (1.f + expf(-v)); }

// conv step of channel c of sequence b: the bf16-rounded SiLU output (as float); the caller
// may update the state.  xt is the channel's new input.
__device__ __forceinline__ float conv_step(const MambaDecodeArgs& a, int b, int c, float xt, float (&s)[kConvK - 1]) {
    const float* st = a.conv_state + ((size_t)b * a.conv_dim + c) * (kConvK - 1);
    const float4 w = *reinterpret_cast<const float4*>(a.conv_w + (size_t)c * kConvK);
    s[0] = st[0];
    s[1] = st[1];
    s[2] = st[2];
    float acc = a.conv_b[c];
    acc = __builtin_fmaf(w.x, s[0], acc);
    acc = __builtin_fmaf(w.y, s[1], acc);
    acc = __builtin_fmaf(w.z, s[2], acc);
    acc = __builtin_fmaf(w.w, xt, acc);
    return bf16_to_f32(f32_to_bf16_rne(silu(acc)));
}

__global__ __launch_bounds__(256) void mamba_conv_ssm_kernel(const MambaDecodeArgs a) {
    __shared__ float sBC[2 * kN];
    __shared__ float sx[8 * kMaxRowsPerWave];

    const int b = blockIdx.y;
    const int h = blockIdx.x / kSsmSplit, half = blockIdx.x % kSsmSplit;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = h / (a.H / a.G);
    const int rows = (a.P + kSsmSplit - 1) / kSsmSplit;
    const int p0 = half * rows;
    const int nrows = min(rows, a.P - p0);
    const uint16_t* xbc = a.proj + (size_t)b * a.proj_ld + a.inter;   // conv inputs [CONV_DIM]

    // B and C channels of the group (256 threads = 2 * 128 channels)
    {
        const int c = tid < kN ? a.inter + grp * kN + tid : a.inter + a.G * kN + grp * kN + (tid - kN);
        float s[kConvK - 1];
        sBC[tid] = conv_step(a, b, c, bf16_to_f32(xbc[c]), s);
    }
    // this workgroup's x channels, with their state update
    if (tid < nrows) {
        const int c = h * a.P + p0 + tid;
        const float xt = bf16_to_f32(xbc[c]);
        float s[kConvK - 1];
        sx[tid] = conv_step(a, b, c, xt, s);
        float* st = a.conv_state + ((size_t)b * a.conv_dim + c) * (kConvK - 1);
        st[0] = s[1];
        st[1] = s[2];
        st[2] = xt;
    }
    // dt, decay (every thread computes the same scalars)
    float dt = bf16_to_f32(a.proj[(size_t)b * a.proj_ld + a.inter + a.conv_dim + h]) + a.dt_bias[h];
    dt = dt > 20.f ? dt : (dt < -20.f ? 0.f : logf(1.f + expf(dt)));
    dt = fminf(FLT_MAX, fmaxf(0.f, dt));
    const float dA = expf(-expf(a.A_log[h]) * dt);
    const float Dh = a.D[h];
    __syncthreads();

    // SSM rows: half-wave hw of wave w takes rows r = 2 w + hw + 8 i; lane l of the half-wave
    // state elements 4 l .. 4 l + 3 of the row.
    const int hw = lane >> 5, l = lane & 31;
    float* S0 = a.ssm_state + (((size_t)b * a.H + h) * a.P + p0) * kN + 4 * l;
    const float4 Bv = *reinterpret_cast<const float4*>(&sBC[4 * l]);
    const float4 Cv = *reinterpret_cast<const float4*>(&sBC[kN + 4 * l]);
    float4 st[kMaxRowsPerWave];
#pragma unroll
    for (int i = 0; i < kMaxRowsPerWave; ++i) {
        const int r = 2 * wave + hw + 8 * i;
        if (r < nrows) st[i] = *reinterpret_cast<const float4*>(S0 + (size_t)r * kN);
    }
#pragma unroll
    for (int i = 0; i < kMaxRowsPerWave; ++i) {
        const int r0 = 2 * wave + 8 * i;               // wave-uniform: the wave's first row of step i
        if (r0 >= nrows) break;
        const int r = r0 + hw;
        const bool ok = r < nrows;
        const float x = ok ? sx[r] : 0.f;
        float4 s = st[i];
        s.x = __builtin_fmaf(s.x, dA, (dt * Bv.x) * x);
        s.y = __builtin_fmaf(s.y, dA, (dt * Bv.y) * x);
        s.z = __builtin_fmaf(s.z, dA, (dt * Bv.z) * x);
        s.w = __builtin_fmaf(s.w, dA, (dt * Bv.w) * x);
        float yp = s.x * Cv.x;
        yp = __builtin_fmaf(s.y, Cv.y, yp);
        yp = __builtin_fmaf(s.z, Cv.z, yp);
        yp = __builtin_fmaf(s.w, Cv.w, yp);
        yp = dpp_row_sum16(yp);
        yp += __shfl_xor(yp, 16);
        if (ok) {
            *reinterpret_cast<float4*>(S0 + (size_t)r * kN) = s;
            if (l == 0) a.y[(size_t)b * a.inter + h * a.P + p0 + r] = f32_to_bf16_rne(__builtin_fmaf(Dh, x, yp));
        }
    }
}

// Gated RMSNorm, one workgroup of 128 threads per (group, sequence): each thread holds up to
// kGnVec vectors of 8 values of the group in registers (one pass over y and z), the group's sum
// of squares goes through the two waves' sums; then the state update of the group's B and C conv
// channels, which every workgroup of kernel 1 read (so it waits for the kernel boundary).
constexpr int kGnThreads = 128;
constexpr int kGnVec = 2;              // group size <= 8 * kGnThreads * kGnVec

__global__ __launch_bounds__(kGnThreads) void mamba_gated_norm_kernel(const MambaDecodeArgs a) {
    __shared__ float red[2];
    const int grp = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int gs = a.inter / a.G;                       // group size, a multiple of 8
    const int nv = gs / 8;
    const size_t y0 = (size_t)b * a.inter + (size_t)grp * gs;
    const uint16_t* zrow = a.proj + (size_t)b * a.proj_ld + (size_t)grp * gs;
    float u[kGnVec][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kGnVec; ++i) {
        const int v = tid + kGnThreads * i;
        if (v < nv) {
            const uint4 yv = load16(a.y + y0 + (size_t)v * 8);
            const uint4 zv = load16(zrow + (size_t)v * 8);
            const uint32_t yd[4] = {yv.x, yv.y, yv.z, yv.w}, zd[4] = {zv.x, zv.y, zv.z, zv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                u[i][2 * j] = bf16lo_to_f32(yd[j]) * silu(bf16lo_to_f32(zd[j]));
                u[i][2 * j + 1] = bf16hi_to_f32(yd[j]) * silu(bf16hi_to_f32(zd[j]));
                ss = __builtin_fmaf(u[i][2 * j], u[i][2 * j], ss);
                ss = __builtin_fmaf(u[i][2 * j + 1], u[i][2 * j + 1], ss);
            }
        }
    }
    ss = wave_sum(ss);
    if (lane == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float r = 1.0f / sqrtf((red[0] + red[1]) / (float)gs + a.eps);
#pragma unroll
    for (int i = 0; i < kGnVec; ++i) {
        const int v = tid + kGnThreads * i;
        if (v < nv) {
            const size_t off = (size_t)grp * gs + (size_t)v * 8;
            const float4 w0 = *reinterpret_cast<const float4*>(a.gnorm_w + off);
            const float4 w1 = *reinterpret_cast<const float4*>(a.gnorm_w + off + 4);
            const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = pack_bf16(u[i][2 * j] * r * w[2 * j], u[i][2 * j + 1] * r * w[2 * j + 1]);
            *reinterpret_cast<uint4*>(a.g + y0 + (size_t)v * 8) = uint4{o[0], o[1], o[2], o[3]};
        }
    }
    // conv state of the group's B and C channels: [s0, s1, s2] -> [s1, s2, xBC]
    if (!a.bc_state) return;
    const uint16_t* xbc = a.proj + (size_t)b * a.proj_ld + a.inter;
    for (int i = tid; i < 2 * kN; i += kGnThreads) {
        const int c = i < kN ? a.inter + grp * kN + i : a.inter + a.G * kN + grp * kN + (i - kN);
        float* st = a.conv_state + ((size_t)b * a.conv_dim + c) * (kConvK - 1);
        const float s1 = st[1], s2 = st[2];
        st[0] = s1;
        st[1] = s2;
        st[2] = bf16_to_f32(xbc[c]);
    }
}

}  // namespace

bool mamba_decode_supported(int H, int P, int G, int d_state, int conv_k) {
    return d_state == kN && conv_k == kConvK && G >= 1 && H >= 1 && H % G == 0 && P >= 1 &&
           (P + kSsmSplit - 1) / kSsmSplit <= 8 * kMaxRowsPerWave && (H * P) % (8 * G) == 0 &&
           (H * P) / G <= 8 * kGnThreads * kGnVec;
}

hipError_t launch_mamba_decode_mixer(const MambaDecodeArgs& a, int batch, hipStream_t stream) {
    hipLaunchKernelGGL(mamba_conv_ssm_kernel, dim3(a.H * kSsmSplit, batch), dim3(256), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(mamba_gated_norm_kernel, dim3(a.G, batch), dim3(kGnThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_mamba_gated_norm(const MambaDecodeArgs& a, int rows, hipStream_t stream) {
    hipLaunchKernelGGL(mamba_gated_norm_kernel, dim3(a.G, rows), dim3(kGnThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace nmi
