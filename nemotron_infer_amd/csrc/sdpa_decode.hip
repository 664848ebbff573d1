// sdpa_decode.hip -- attention decode for gfx950: one query token per head against the
// KV cache, then the new token's K and V appended to the cache.
//
//   O[h] = softmax(q[h] . K[kv(h), 0:S]^T / sqrt(128)) . V[kv(h), 0:S],  kv(h) = h / (H / H_KV)
//   K[kv, S] = K_new[kv], V[kv, S] = V_new[kv]
//
// The contract of the reference's sdpa_decode_bf16 (nemotron_infer/csrc/include/ops/attention/
// sdpa_decode.cuh:57-166, host entry :267-285): the query attends the S cached positions only
// (the new token's K/V are appended after, at position S), float32 arithmetic on bf16 inputs,
// S == 0 gives O = 0, caches [H_KV, cap, 128] bf16, head dim 128.  The schedule is this build's:
//
// * One workgroup per (KV head, split of the positions): it serves every query head of the GQA
//   group, so K and V are read once per KV head instead of once per query head (the reference
//   reads them H / H_KV times).
// * 4 waves x 4 rows of 16 lanes: a 16-lane row takes one position, each lane 8 of the 128 dims
//   (one 16-byte load of K and of V), so a wave reads 4 consecutive positions = 1 KiB contiguous
//   per load instruction.  Scores: v_dot2_f32_bf16 over the lane's 8 dims and a 16-lane DPP
//   sum; each row keeps its own running (max, sum, o[8 dims]) per query head (online softmax in
//   base 2: scores are pre-multiplied by log2(e) / sqrt(128)).  Positions go in batches of 4
//   per row (64 per workgroup, 32 KiB of K and V); the next batch is loaded before the current
//   one is computed, so a workgroup of one batch pays one memory latency.
// * The 16 rows of a workgroup are merged through LDS; with one split the workgroup writes O,
//   otherwise fp32 partials (m, l, o[128]) per (query head, split) that a second small kernel
//   merges.  Split 0 also appends K_new / V_new (position S is read by nobody in this call).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <algorithm>
#include <cfloat>

namespace nmi {

namespace {

constexpr int kHead = 128;
constexpr int kWaves = 4;
constexpr int kRows = kWaves * 4;      // 16-lane rows per workgroup
constexpr int kPartStride = 2 + kHead; // floats per (query head, split) partial: m, l, o[128]

struct SdpaArgs {
    const uint16_t* q;       // [H, 128]
    uint16_t* k_cache;       // [H_KV, cap, 128]
    uint16_t* v_cache;
    const uint16_t* k_new;   // [H_KV, 128]
    const uint16_t* v_new;
    uint16_t* o;             // [H, 128]
    float* part;             // [H, nsplit, kPartStride] when nsplit > 1
    int S;                   // cached positions attended
    int cap;                 // cache capacity (positions per KV head)
    int nsplit;
    int chunk;               // positions per split
    float scale2;            // log2(e) / sqrt(128)
};

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr int kU = 4;                  // positions per row per batch
constexpr int kBatch = kU * kRows;     // positions per workgroup per batch

__device__ __forceinline__ void load_batch(const uint16_t* Kh, const uint16_t* Vh, int pos, int e, uint4 (&k)[kU],
                                           uint4 (&v)[kU]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int s = min(pos + u * kRows, e - 1);
        k[u] = load16(Kh + (size_t)s * kHead);
        v[u] = load16(Vh + (size_t)s * kHead);
    }
}

// One batch of a row (kU positions): the kU x R scores (16-lane dot products, independent
// chains), then per query head one online-softmax step for the whole batch -- the running max
// and the rescale of o move once per batch, not once per position.  `p` is the wave's first
// position of the batch; positions at or past e score -inf (weight 0).
template <int R>
__device__ __forceinline__ void compute_batch(const uint4 (&k)[kU], const uint4 (&v)[kU], int p, int g, int e,
                                              const uint4 (&q)[R], float scale2, float (&m)[R], float (&l)[R],
                                              float (&o)[R][8]) {
    float sc[kU][R];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        if (p + u * kRows < e) {                        // wave-uniform: some row of step u is valid
            const bool valid = p + u * kRows + g < e;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float d = dot2_bf16(k[u].x, q[r].x, 0.f);
                d = dot2_bf16(k[u].y, q[r].y, d);
                d = dot2_bf16(k[u].z, q[r].z, d);
                d = dot2_bf16(k[u].w, q[r].w, d);
                d = dpp_row_sum16(d);
                sc[u][r] = valid ? d * scale2 : -INFINITY;
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) sc[u][r] = -INFINITY;
        }
    }
    float vf[kU][8];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const uint4 vv = v[u];
        vf[u][0] = bf16lo_to_f32(vv.x), vf[u][1] = bf16hi_to_f32(vv.x);
        vf[u][2] = bf16lo_to_f32(vv.y), vf[u][3] = bf16hi_to_f32(vv.y);
        vf[u][4] = bf16lo_to_f32(vv.z), vf[u][5] = bf16hi_to_f32(vv.z);
        vf[u][6] = bf16lo_to_f32(vv.w), vf[u][7] = bf16hi_to_f32(vv.w);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float bm = sc[0][r];
#pragma unroll
        for (int u = 1; u < kU; ++u) bm = fmaxf(bm, sc[u][r]);
        const float mn = fmaxf(m[r], bm);
        const float corr = fexp2(m[r] - mn);
        float pr[kU];
        float ps = 0.f;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            pr[u] = fexp2(sc[u][r] - mn);
            ps += pr[u];
        }
        l[r] = __builtin_fmaf(l[r], corr, ps);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float acc = o[r][i] * corr;
#pragma unroll
            for (int u = 0; u < kU; ++u) acc = __builtin_fmaf(pr[u], vf[u][i], acc);
            o[r][i] = acc;
        }
        m[r] = mn;
    }
}

template <int R>
__global__ __launch_bounds__(256) void sdpa_decode_split_kernel(const SdpaArgs a) {
    __shared__ float sm_ml[kRows][R][2];
    __shared__ float sm_o[kRows][R][kHead];

    const int split = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, sub = lane & 15;
    const int row = wave * 4 + g;
    const int b = split * a.chunk;
    const int e = min(a.S, b + a.chunk);

    uint4 q[R];
#pragma unroll
    for (int r = 0; r < R; ++r) q[r] = load16(a.q + (size_t)(kvh * R + r) * kHead + sub * 8);

    float m[R], l[R], o[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = -FLT_MAX;
        l[r] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[r][i] = 0.f;
    }

    const uint16_t* Kh = a.k_cache + (size_t)kvh * a.cap * kHead + sub * 8;
    const uint16_t* Vh = a.v_cache + (size_t)kvh * a.cap * kHead + sub * 8;
    // Row (wave, g) takes positions b + wave * 4 + g + 16 j.  A batch is kU such positions per
    // row (64 per workgroup); the next batch is loaded before the current one is computed.
    // Positions past e are loaded clamped to e - 1 (a cached line) and score -inf; the loop
    // bounds are wave-uniform.
    int p = b + wave * 4;
    if (p < e) {
        // A counted loop with no exit between a batch's loads and their use: the compiler then
        // keeps the loads where they are issued (with an exit in between it sinks them to the use).
        const int nb = (e - p + kBatch - 1) / kBatch;
        uint4 ka[kU], va[kU], kz[kU], vz[kU];
        load_batch(Kh, Vh, p + g, e, ka, va);
        int i = 0;
        for (; i + 2 <= nb; i += 2) {
            load_batch(Kh, Vh, p + kBatch + g, e, kz, vz);
            __builtin_amdgcn_sched_barrier(0);
            compute_batch<R>(ka, va, p, g, e, q, a.scale2, m, l, o);
            load_batch(Kh, Vh, p + 2 * kBatch + g, e, ka, va);
            __builtin_amdgcn_sched_barrier(0);
            compute_batch<R>(kz, vz, p + kBatch, g, e, q, a.scale2, m, l, o);
            p += 2 * kBatch;
        }
        if (i < nb) compute_batch<R>(ka, va, p, g, e, q, a.scale2, m, l, o);
    }

    // merge the 16 rows
    if (sub == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            sm_ml[row][r][0] = m[r];
            sm_ml[row][r][1] = l[r];
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        *reinterpret_cast<float4*>(&sm_o[row][r][sub * 8]) = float4{o[r][0], o[r][1], o[r][2], o[r][3]};
        *reinterpret_cast<float4*>(&sm_o[row][r][sub * 8 + 4]) = float4{o[r][4], o[r][5], o[r][6], o[r][7]};
    }
    __syncthreads();
    for (int it = tid; it < R * kHead; it += 256) {
        const int r = it / kHead, d = it % kHead;
        float M = -FLT_MAX;
#pragma unroll
        for (int j = 0; j < kRows; ++j) M = fmaxf(M, sm_ml[j][r][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int j = 0; j < kRows; ++j) {
            const float w = fexp2(sm_ml[j][r][0] - M);
            L = __builtin_fmaf(w, sm_ml[j][r][1], L);
            O = __builtin_fmaf(w, sm_o[j][r][d], O);
        }
        const int h = kvh * R + r;
        if (a.nsplit == 1) {
            const float inv = L > 0.f ? 1.f / L : 0.f;
            a.o[(size_t)h * kHead + d] = f32_to_bf16_rne(O * inv);
        } else {
            float* p = a.part + ((size_t)h * a.nsplit + split) * kPartStride;
            if (d == 0) {
                p[0] = M;
                p[1] = L;
            }
            p[2 + d] = O;
        }
    }
    // append the new token's K and V at position S (16 lanes x 16 bytes each)
    if (split == 0 && tid < 32) {
        const int c = tid & 15;
        const bool is_v = tid >= 16;
        const uint16_t* src = (is_v ? a.v_new : a.k_new) + (size_t)kvh * kHead + c * 8;
        uint16_t* dst = (is_v ? a.v_cache : a.k_cache) + ((size_t)kvh * a.cap + a.S) * kHead + c * 8;
        *reinterpret_cast<uint4*>(dst) = load16(src);
    }
}

// One workgroup of 256 threads per query head merges the splits' partials:
// O[h, d] = sum_i w_i o_i[d] / sum_i w_i l_i with w_i = 2^(m_i - max_i m_i).  Wave w takes splits
// w, w + 4, ... with its own running maximum (one pass over the partials); lane j dims 2j, 2j + 1;
// the four waves' sums meet in LDS, rescaled to the common maximum.
__global__ __launch_bounds__(256) void sdpa_decode_combine_kernel(const SdpaArgs a) {
    __shared__ float sm_m[kWaves];
    __shared__ float sm_l[kWaves];
    __shared__ float2 sm_o[kWaves][kHead / 2];
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float* p = a.part + (size_t)h * a.nsplit * kPartStride;
    float M = -FLT_MAX, L = 0.f, O0 = 0.f, O1 = 0.f;
#pragma unroll 4
    for (int i = wave; i < a.nsplit; i += kWaves) {
        const float* pi = p + (size_t)i * kPartStride;
        const float mi = pi[0], li = pi[1];
        const float2 oi = *reinterpret_cast<const float2*>(pi + 2 + 2 * lane);
        const float mn = fmaxf(M, mi);
        const float c = fexp2(M - mn), w = fexp2(mi - mn);
        L = __builtin_fmaf(w, li, L * c);
        O0 = __builtin_fmaf(w, oi.x, O0 * c);
        O1 = __builtin_fmaf(w, oi.y, O1 * c);
        M = mn;
    }
    if (lane == 0) {
        sm_m[wave] = M;
        sm_l[wave] = L;
    }
    sm_o[wave][lane] = float2{O0, O1};
    __syncthreads();
    if (tid < kHead / 2) {
        const float Mt = fmaxf(fmaxf(sm_m[0], sm_m[1]), fmaxf(sm_m[2], sm_m[3]));
        float c[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) c[w] = fexp2(sm_m[w] - Mt);
        const float Lt = (sm_l[0] * c[0] + sm_l[1] * c[1]) + (sm_l[2] * c[2] + sm_l[3] * c[3]);
        float o0 = 0.f, o1 = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            o0 = __builtin_fmaf(sm_o[w][tid].x, c[w], o0);
            o1 = __builtin_fmaf(sm_o[w][tid].y, c[w], o1);
        }
        const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
        *reinterpret_cast<uint32_t*>(a.o + (size_t)h * kHead + 2 * tid) = pack_bf16(o0 * inv, o1 * inv);
    }
}

template <int R>
hipError_t launch_split(const SdpaArgs& a, int n_kv, hipStream_t stream) {
    hipLaunchKernelGGL(sdpa_decode_split_kernel<R>, dim3(a.nsplit, n_kv), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

void sdpa_decode_plan(int S, int n_kv, int* nsplit, int* chunk) {
    const Tuning& t = tuning();
    // Splits of kSdpaMinChunk positions (the "sdpa.chunk" knob overrides), at most one
    // workgroup per CU in all (measured best from 1k to 32k positions) and at most
    // kSdpaMaxSplits per KV head.
    int target = t.sdpa_chunk > 0 ? t.sdpa_chunk : kSdpaMinChunk;
    int n = S <= 0 ? 1 : (S + target - 1) / target;
    const int cap = std::max(1, device_info().num_cu / std::max(1, n_kv));
    if (t.sdpa_chunk <= 0 && n > cap) n = cap;
    if (n > kSdpaMaxSplits) n = kSdpaMaxSplits;
    if (n < 1) n = 1;
    int c = S <= 0 ? 0 : (S + n - 1) / n;
    if (c > 0) n = (S + c - 1) / c;
    *nsplit = n;
    *chunk = c;
}

size_t sdpa_decode_workspace_bytes(int n_heads, int S, int n_kv) {
    int nsplit = 1, chunk = 0;
    sdpa_decode_plan(S, n_kv, &nsplit, &chunk);
    if (nsplit <= 1) return 0;
    return (size_t)n_heads * nsplit * kPartStride * sizeof(float);
}

hipError_t launch_sdpa_decode(const uint16_t* q, uint16_t* k_cache, uint16_t* v_cache, const uint16_t* k_new,
                              const uint16_t* v_new, uint16_t* o, int S, int cap, int n_heads, int n_kv,
                              void* workspace, hipStream_t stream) {
    SdpaArgs a{};
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.k_new = k_new;
    a.v_new = v_new;
    a.o = o;
    a.part = static_cast<float*>(workspace);
    a.S = S;
    a.cap = cap;
    sdpa_decode_plan(S, n_kv, &a.nsplit, &a.chunk);
    a.scale2 = 1.4426950408889634f / sqrtf((float)kHead);
    const int R = n_heads / n_kv;
    hipError_t e;
    switch (R) {
        case 1: e = launch_split<1>(a, n_kv, stream); break;
        case 2: e = launch_split<2>(a, n_kv, stream); break;
        case 3: e = launch_split<3>(a, n_kv, stream); break;
        case 4: e = launch_split<4>(a, n_kv, stream); break;
        case 5: e = launch_split<5>(a, n_kv, stream); break;
        case 6: e = launch_split<6>(a, n_kv, stream); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || a.nsplit == 1) return e;
    hipLaunchKernelGGL(sdpa_decode_combine_kernel, dim3(n_heads), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace nmi
