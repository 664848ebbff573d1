// sdpa_prefill.hip -- causal attention over a whole prompt (prefill) for gfx950, on bf16 MFMA.
//
//   O[s, h] = softmax_{t <= s}(q[s, h] . k[t, kv(h)] / sqrt(128)) . v[t, kv(h)],  kv(h) = h / (H / H_KV)
//
// The contract of the reference's sdpa_prefill_bf16 (nemotron_infer/csrc/include/ops/attention/
// sdpa_prefill.cuh:224-320, host entry :364-395): causal, GQA, head dim 128, float32 softmax and
// accumulation on bf16 inputs, bf16 output.  The layouts are this build's: q, k, v and O stay
// token-major ([S, heads * 128], as the projections write them) -- the reference transposes
// them to head-major around its kernel (model/attention_block.cuh:339-345) -- and V is read
// through a head-major transposed copy V^T [H_KV, 128, ldvt] that the layout kernel below writes
// (together with the KV cache).
//
// Kernel: one workgroup per (query head, tile of 128 query rows), 4 waves of 32 rows; key/value
// tiles of 64 positions staged in LDS (K as [64][128], V^T as [128][64] with the positions of each
// 16-key group in the P operand's order, both swizzled so that the MFMA operand reads hit distinct
// banks), the next tile prefetched into registers while the current one is multiplied.  Per wave
// and key tile (v_mfma_f32_32x32x16_bf16):
// * S^T = K . Q^T (64 keys x 32 queries): the wave's query rows are the B operand, held in
//   registers for the whole kernel; the scores of one query then sit in one lane (16 registers
//   per 32-key block, the two lane halves holding alternate 4-key groups), so the row max and
//   sum are in-lane plus one exchange between the halves.
// * online softmax in base 2 (weights exp2((s - m) log2(e) / sqrt(128)) with one fma per score),
//   the running max m raised lazily (only when a score exceeds it by 2^8 in weight, so the
//   accumulators are rescaled rarely); keys after the query masked on the diagonal tiles only.
// * O^T += V^T . P^T: P is the B operand straight from the score registers -- a 16-key step's
//   lane-half h holds keys {4h..4h+3, 8+4h..8+4h+3}, and the V^T operand is read in the same
//   key order -- in two bf16 parts (hi = bf16(p), lo = bf16(p - hi)), so the weights carry about
//   16 significant bits and the float32 row sums stay consistent with them.
// Query tiles are scheduled longest first over all heads (the last tiles see the most keys).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <cfloat>

namespace nmi {

namespace {

constexpr int kD = 128;           // head dim
constexpr int kBQ = 128;          // query rows per workgroup
constexpr int kBK = 64;           // key positions per tile
constexpr int kKBytes = kBK * kD * 2;        // K tile, 16 KiB
constexpr int kVBytes = kD * kBK * 2;        // V^T tile, 16 KiB
constexpr int kStage = kKBytes + kVBytes;
constexpr float kLazy = 8.f;       // log2 of the largest unnormalised softmax weight (lazy max)

struct PrefillArgs {
    const uint16_t* q;      // [S, ldq], head h at column 128 h
    const uint16_t* k;      // [S, ldk], KV head j at column 128 j
    const uint16_t* vt;     // [H_KV, 128, ldvt]: V^T, zero past S
    uint16_t* o;            // [S, ldo], head h at column 128 h
    int64_t ldq, ldk, ldvt, ldo;
    int S, H, H_KV, qtiles;
    float scale2;           // log2(e) / sqrt(128)
};

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS K tile: row r (key) of 16 chunks of 16 B, chunk c at c ^ (r & 15)
__device__ __forceinline__ int k_off(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 4); }
// LDS V^T tile: row d of 8 chunks of 16 B (64 keys), chunk c at c ^ ((d >> 1) & 7)
__device__ __forceinline__ int v_off(int d, int c) { return d * 128 + ((c ^ ((d >> 1) & 7)) << 4); }

__global__ __launch_bounds__(256, 2) void sdpa_prefill_kernel(const PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, l32 = lane & 31;
    // longest tiles first over all heads: workgroup g takes query tile qtiles - 1 - g / H of head g % H
    const int qt = a.qtiles - 1 - (int)blockIdx.x / a.H;
    const int head = (int)blockIdx.x - (int)blockIdx.x / a.H * a.H;
    const int kvh = head / (a.H / a.H_KV);
    const int q0 = qt * kBQ;
    const int qw = q0 + 32 * wave;                              // the wave's first query row
    const int qrow = qw + l32;                                  // this lane's query (B operand column)
    const int S = a.S;
    const int kv_end = min(S, q0 + kBQ);                        // keys this workgroup needs
    const int ntiles = (kv_end + kBK - 1) / kBK;

    // the wave's query rows as B fragments: k step s holds dims 16 s + 8 h .. + 7 of row qrow
    bf16x8 qf[8];
    {
        const uint16_t* qp = a.q + (int64_t)min(qrow, S - 1) * a.ldq + head * kD + 8 * h;
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = __builtin_bit_cast(bf16x8, load16(qp + 16 * s));
    }

    // staging: thread t moves chunks t + 256 u (u = 0..3) of the K tile (row i / 16, chunk i % 16)
    // and of the V^T tile (row i / 8, chunk i % 8)
    const uint16_t* kbase = a.k + kvh * kD;
    const uint16_t* vbase = a.vt + (int64_t)kvh * kD * a.ldvt;
    uint4 rk[4], rv[4];
    auto gload = [&](int kv0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = tid + 256 * u;
            const int kr = i >> 4, kc = i & 15;
            rk[u] = load16(kbase + (int64_t)min(kv0 + kr, S - 1) * a.ldk + 8 * kc);
            const int vd = i >> 3, vc = i & 7;
            rv[u] = load16(vbase + (int64_t)vd * a.ldvt + kv0 + 8 * vc);
        }
    };
    auto sstore = [&](int buf) {
        uint8_t* st = lds + buf * kStage;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = tid + 256 * u;
            *reinterpret_cast<uint4*>(st + k_off(i >> 4, i & 15)) = rk[u];
            *reinterpret_cast<uint4*>(st + kKBytes + v_off(i >> 3, i & 7)) = rv[u];
        }
    };

    f32x16 oacc[4];                                             // O^T: 4 blocks of 32 dims x 32 queries
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[b][r] = 0.f;
    float m = -INFINITY, l = 0.f;                               // raw score units

    gload(0);
    // complete the query loads before the loop (with the first tile's, in flight together):
    // otherwise the compiler's wait analysis, merging the loop paths with and without the next
    // tile's prefetch, waits for that prefetch before the score MFMAs of every tile (loads retire
    // in order), which puts a memory round trip on each tile's critical path
#pragma unroll
    for (int s = 0; s < 8; ++s) asm volatile("" ::"v"(qf[s]));
    sstore(0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int kv0 = t * kBK;
        if (t + 1 < ntiles) gload(kv0 + kBK);
        const uint8_t* st = lds + buf * kStage;
        if (kv0 <= qw + 31) {                                   // wave-uniform: some key <= some query of the wave
            // S^T = K . Q^T, two blocks of 32 keys
            f32x16 sacc[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[b][r] = 0.f;
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const bf16x8 kf = *reinterpret_cast<const bf16x8*>(st + k_off(32 * b + l32, 2 * s + h));
                    sacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], sacc[b], 0, 0, 0);
                }
            }
            // causal mask, only where the tile reaches past the wave's first query: register r of
            // block b is key kv0 + 32 b + 8 (r / 4) + 4 h + r % 4, kept where it is <= qrow (then also
            // < S for every stored query; rows past S are not stored)
            if (kv0 + kBK - 1 > qw) {
                // a branch the compiler keeps: the tiles below the diagonal skip the mask entirely
                asm volatile("" ::: "memory");
                const int dq = qrow - kv0 - 4 * h;
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (32 * b + 8 * (r >> 2) + (r & 3) > dq) sacc[b][r] = -INFINITY;
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sacc[b][r]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            // running max m in raw score units, raised lazily: only when a score exceeds it by more
            // than 8 / scale2 (then the weights exp2((s - m) scale2) stay below 2^8); the rescale of
            // the accumulators runs when any lane of the wave raises its max.  O / l does not depend
            // on m.
            const bool raise = tmax > m + kLazy / a.scale2;
            if (__builtin_amdgcn_ballot_w64(raise)) {
                const float mn = raise ? tmax : m;
                const float corr = raise ? fexp2((m - mn) * a.scale2) : 1.f;
                l *= corr;
#pragma unroll
                for (int b = 0; b < 4; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[b][r] *= corr;
                m = mn;
            }
            const float mc = m * a.scale2;
            float psum = 0.f;
            // P^T as B fragments: key step j (16 keys) = block j / 2, registers 8 (j % 2) .. + 7, each
            // weight in two bf16 parts: hi = bf16(p), lo = bf16(p - hi)
            bf16x8 phi[4], plo[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const float p0 = fexp2(__builtin_fmaf(sacc[j >> 1][8 * (j & 1) + e], a.scale2, -mc));
                    const float p1 = fexp2(__builtin_fmaf(sacc[j >> 1][8 * (j & 1) + e + 1], a.scale2, -mc));
                    psum += p0;
                    psum += p1;
                    const uint32_t w = pack_bf16(p0, p1);
                    hw[e >> 1] = w;
                    lw[e >> 1] = pack_bf16(p0 - __uint_as_float(w << 16), p1 - __uint_as_float(w & 0xffff0000u));
                }
                phi[j] = __builtin_bit_cast(bf16x8, uint4{hw[0], hw[1], hw[2], hw[3]});
                plo[j] = __builtin_bit_cast(bf16x8, uint4{lw[0], lw[1], lw[2], lw[3]});
            }
            psum += __shfl_xor(psum, 32);
            l += psum;
            // O^T += V^T . P^T: the V^T operand of key step j, lane half h: keys 16 j + 4 h + {0..3}
            // and 16 j + 8 + 4 h + {0..3}, which the layout kernel stores as chunk 2 j + h of the row
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int d = 32 * b + l32;
                    const bf16x8 vf = *reinterpret_cast<const bf16x8*>(st + kKBytes + v_off(d, 2 * j + h));
                    oacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, phi[j], oacc[b], 0, 0, 0);
                    oacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, plo[j], oacc[b], 0, 0, 0);
                }
            }
        }
        if (t + 1 < ntiles) {
            // the other stage was last read in iteration t - 1, which every wave left through the
            // barrier below; this barrier publishes it for iteration t + 1
            sstore(buf ^ 1);
            __syncthreads();
        }
    }

    // O = O^T / l: register r of block b is dim 32 b + 8 (r / 4) + 4 h + r % 4 of query qrow
    if (qrow < S) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        uint16_t* op = a.o + (int64_t)qrow * a.ldo + head * kD;
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * b + 8 * g + 4 * h;
                *reinterpret_cast<uint2*>(op + d) = uint2{pack_bf16(oacc[b][4 * g] * inv, oacc[b][4 * g + 1] * inv),
                                                          pack_bf16(oacc[b][4 * g + 2] * inv, oacc[b][4 * g + 3] * inv)};
            }
    }
}

// Layout kernel: one workgroup per (64 positions, KV head).  V^T [H_KV, 128, ldvt] from v
// [S, ldv] (positions S .. ldvt zero), and, when caches are given, k_cache / v_cache
// [H_KV, cap, 128] positions [0, S) from k and v (the reference's cudaMemcpy2DAsync of its
// head-major K/V, attention_block.cuh:355-364).
__global__ __launch_bounds__(256) void kv_layout_kernel(const uint16_t* __restrict__ k, int64_t ldk,
                                                        const uint16_t* __restrict__ v, int64_t ldv,
                                                        uint16_t* __restrict__ vt, int64_t ldvt,
                                                        uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int cap,
                                                        int S) {
    __shared__ uint16_t tile[64][kD + 8];                    // 64 positions x 128 dims (+ pad)
    const int p0 = blockIdx.x * 64, kvh = blockIdx.y, tid = threadIdx.x;
    // rows of v (and k): 64 positions x 16 chunks; thread t chunks t + 256 u
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = tid + 256 * u;
        const int r = i >> 4, c = i & 15;
        const int p = p0 + r;
        uint4 vv = uint4{0, 0, 0, 0};
        if (p < S) {
            vv = load16(v + (int64_t)p * ldv + kvh * kD + 8 * c);
            if (kc) {
                const uint4 kk = load16(k + (int64_t)p * ldk + kvh * kD + 8 * c);
                *reinterpret_cast<uint4*>(kc + ((int64_t)kvh * cap + p) * kD + 8 * c) = kk;
                *reinterpret_cast<uint4*>(vc + ((int64_t)kvh * cap + p) * kD + 8 * c) = vv;
            }
        }
        const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tile[r][8 * c + 2 * e] = (uint16_t)w[e];
            tile[r][8 * c + 2 * e + 1] = (uint16_t)(w[e] >> 16);
        }
    }
    __syncthreads();
    // V^T rows: 128 dims x 8 chunks of 8 slots.  Within each group of 16 positions the slots hold
    // the positions in the order 0-3, 8-11, 4-7, 12-15 (slot 4 b + c holds position 4 perm(b) + c,
    // perm = 0, 2, 1, 3), the key order of the attention kernel's P operand: chunk 2 j + h is then
    // exactly the 8 keys lane half h multiplies in key step j.
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = tid + 256 * u;
        const int d = i >> 3, c = i & 7;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int slot = 8 * c + 2 * e;                     // even: slots slot, slot + 1 share b
            const int bq = (slot >> 2) & 3;
            const int key = (slot & ~15) + 4 * ((bq == 1 || bq == 2) ? 3 - bq : bq) + (slot & 3);
            w[e] = (uint32_t)tile[key][d] | ((uint32_t)tile[key + 1][d] << 16);
        }
        *reinterpret_cast<uint4*>(vt + ((int64_t)kvh * kD + d) * ldvt + p0 + 8 * c) = uint4{w[0], w[1], w[2], w[3]};
    }
}

}  // namespace

int64_t sdpa_prefill_vt_ld(int S) { return ((int64_t)S + 63) / 64 * 64; }

hipError_t launch_kv_layout(const uint16_t* k, int64_t ldk, const uint16_t* v, int64_t ldv, uint16_t* vt, int S,
                            int H_KV, uint16_t* k_cache, uint16_t* v_cache, int cap, hipStream_t stream) {
    const int64_t ldvt = sdpa_prefill_vt_ld(S);
    hipLaunchKernelGGL(kv_layout_kernel, dim3((unsigned)(ldvt / 64), H_KV), dim3(256), 0, stream, k, ldk, v, ldv, vt,
                       ldvt, k_cache, v_cache, cap, S);
    return hipGetLastError();
}

hipError_t launch_sdpa_prefill(const uint16_t* q, int64_t ldq, const uint16_t* k, int64_t ldk, const uint16_t* vt,
                               uint16_t* o, int64_t ldo, int S, int H, int H_KV, hipStream_t stream) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&sdpa_prefill_kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 2 * kStage);
    if (attr != hipSuccess) return attr;
    PrefillArgs a{};
    a.q = q;
    a.k = k;
    a.vt = vt;
    a.o = o;
    a.ldq = ldq;
    a.ldk = ldk;
    a.ldvt = sdpa_prefill_vt_ld(S);
    a.ldo = ldo;
    a.S = S;
    a.H = H;
    a.H_KV = H_KV;
    a.qtiles = (S + kBQ - 1) / kBQ;
    a.scale2 = 1.4426950408889634f / sqrtf((float)kD);
    hipLaunchKernelGGL(sdpa_prefill_kernel, dim3(a.qtiles * H), dim3(256), 2 * kStage, stream, a);
    return hipGetLastError();
}

}  // namespace nmi
