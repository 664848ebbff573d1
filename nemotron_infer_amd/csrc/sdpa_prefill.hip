// sdpa_prefill.hip -- causal attention over a whole prompt (prefill) for gfx950, on bf16 MFMA.
//
//   O[s, h] = softmax_{t <= s}(q[s, h] . k[t, kv(h)] / sqrt(128)) . v[t, kv(h)],  kv(h) = h / (H / H_KV)
//
// The contract of the reference's sdpa_prefill_bf16 (nemotron_infer/csrc/include/ops/attention/
// sdpa_prefill.cuh:224-320, host entry :364-395): causal, GQA, head dim 128, float32 softmax and
// accumulation on bf16 inputs, bf16 output.  The layouts are this build's: q, k, v and O stay
// token-major ([S, heads * 128], as the projections write them) -- the reference transposes
// them to head-major around its kernel (model/attention_block.cuh:339-345); V is read token-major
// too, its MFMA operand built by transposing LDS reads.
//
// Kernel: one workgroup per (query head, tile of 128 query rows), 4 waves of 32 rows.  K and V
// reach LDS by DMA (global_load_lds_dwordx4, no register staging), token-major and swizzled so
// that the operand reads hit distinct banks: K in blocks of 32 keys (four 8 KiB slots), V in tiles
// of 64 keys (two 16 KiB stages); one barrier per 64 keys.  Per wave and 32-key block
// (v_mfma_f32_32x32x16_bf16):
// * S^T = K . Q^T (32 keys x 32 queries): the wave's query rows are the B operand, held in
//   registers for the whole kernel; the scores of one query then sit in one lane (16 registers,
//   the two lane halves holding alternate 4-key groups), so the row max and sum are in-lane plus
//   one exchange between the halves.  The next block's scores are computed while this block's
//   softmax runs, their MFMAs interleaved with its vector work.
// * online softmax in base 2 (weights exp2((s - m) log2(e) / sqrt(128)) with one fma per score),
//   the running max m raised lazily (only when a score exceeds it by 2^8 in weight, so the
//   accumulators are rescaled rarely); keys after the query masked on the diagonal blocks only.
// * O^T += V^T . P^T: P is the B operand straight from the score registers -- a 16-key step's
//   lane-half h holds keys {4h..4h+3, 8+4h..8+4h+3} -- in two bf16 parts (hi = bf16(p), lo =
//   bf16(p - hi)), so the weights carry about 16 significant bits and the float32 row sums stay
//   consistent with them.  The V^T operand, in the same key order, comes from two transposing
//   LDS reads (ds_read_b64_tr_b16) of the token-major V tile.
// Query tiles are scheduled longest first over all heads (the last tiles see the most keys).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <cfloat>
#include <type_traits>

namespace nmi {

namespace {

constexpr int kD = 128;           // head dim
constexpr int kBQ = 128;          // query rows per workgroup
constexpr int kBK = 64;           // key positions per tile
constexpr int kKBlk = 32 * kD * 2;           // K block of 32 keys, 8 KiB (four slots)
constexpr int kVBytes = kBK * kD * 2;        // V tile of 64 keys, 16 KiB (two stages)
constexpr int kLds = 4 * kKBlk + 2 * kVBytes;
constexpr float kLazy = 8.f;       // log2 of the largest unnormalised softmax weight (lazy max)

struct PrefillArgs {
    const uint16_t* q;      // [S, ldq], head h at column 128 h
    const uint16_t* k;      // [S, ldk], KV head j at column 128 j
    const uint16_t* v;      // [S, ldv], KV head j at column 128 j
    uint16_t* o;            // [S, ldo], head h at column 128 h
    int64_t ldq, ldk, ldv, ldo;
    int S, H, H_KV, qtiles;
    int nslot;              // workgroups per pass of the dispatcher (one per CU)
    float scale2;           // log2(e) / sqrt(128)
};

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS K tile: row r (key) of 16 chunks of 16 B, chunk c at c ^ (r & 15)
__device__ __forceinline__ int k_off(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 4); }
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__global__ __launch_bounds__(256, 2) void sdpa_prefill_kernel(const PrefillArgs a) {
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)lds;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, l32 = lane & 31;
    // Tiles by rank, longest first over all heads: rank r is query tile qtiles - 1 - r / H of head
    // r % H.  The dispatcher gives each CU one workgroup per pass (workgroups g and g + nslot
    // share a CU), so the second pass takes its ranks in reverse: a CU then holds a long and a
    // short tile of about the same sum; the rest follow longest first.
    const int total = a.qtiles * a.H, g = (int)blockIdx.x;
    const int n2 = min(2 * a.nslot, total);
    const int rank = (g >= a.nslot && g < n2) ? a.nslot + (n2 - 1 - g) : g;
    const int qt = a.qtiles - 1 - rank / a.H;
    const int head = rank - rank / a.H * a.H;
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

    // LDS: K blocks of 32 keys, block g in slot g % 4 at g % 4 * 8 KiB; V tiles of 64 keys, tile t in
    // stage t & 1 at 32 KiB + (t & 1) * 16 KiB; both token-major, 256 B per key.
    // LDS DMA sources.  Instruction i of the wave fills rows r = 16 i + 4 wave + lane / 16 of a K slot
    // (i = 0, 1) or V stage (i = 0 .. 3) (1 KiB: 4 rows of 256 B); lane position p = lane % 16 of row r
    // takes chunk p ^ (r & 15) (K) or p ^ (4 (r & 3)) (V).  The swizzles do not depend on i, so one
    // lane offset serves every instruction (i moves the scalar base).
    const int64_t ldk2 = a.ldk * 2, ldv2 = a.ldv * 2;
    const int kr0 = 4 * wave + (lane >> 4);
    const uint32_t kchunk = 16u * (uint32_t)((lane & 15) ^ (kr0 & 15));
    const uint32_t koff = (uint32_t)(kr0 * ldk2) + kchunk;
    const uint32_t vchunk = 16u * (uint32_t)((lane & 15) ^ (4 * (kr0 & 3)));
    const uint32_t voff = (uint32_t)(kr0 * ldv2) + vchunk;
    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.k + kvh * kD);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.v + kvh * kD);
    const int nblk = 2 * ntiles;
    // K block g into slot g % 4; rows past S - 1 (of a last, partial block, or of a block wholly
    // past S) read row S - 1
    auto issue_k = [&](int g) {
        const int kv0 = 32 * g;
        const uint32_t sb = lds0 + (uint32_t)((g & 3) * kKBlk) + wave * 1024;
        if (kv0 + 32 <= S) {
            const uint8_t* base = kbase + (int64_t)kv0 * ldk2;
#pragma unroll
            for (int i = 0; i < 2; ++i) dma16_lds(base + 16 * i * ldk2, koff, sb + i * 4096);
        } else {
            const int r0 = min(kv0, S - 1);
            const uint8_t* base = kbase + (int64_t)r0 * ldk2;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                dma16_lds(base, (uint32_t)((min(kv0 + 16 * i + kr0, S - 1) - r0) * ldk2) + kchunk, sb + i * 4096);
        }
    };
    // V tile t (64 keys, token-major) into stage t & 1, row r's chunk c at c ^ (4 (r & 3)); rows past
    // S - 1 read row S - 1 (finite values; their weights are 0)
    auto issue_v = [&](int t) {
        const int kv0 = t * kBK;
        const uint32_t sb = lds0 + (uint32_t)(4 * kKBlk + (t & 1) * kVBytes) + wave * 1024;
        if (kv0 + kBK <= S) {
            const uint8_t* base = vbase + (int64_t)kv0 * ldv2;
#pragma unroll
            for (int i = 0; i < 4; ++i) dma16_lds(base + 16 * i * ldv2, voff, sb + i * 4096);
        } else {
            const int r0 = min(kv0, S - 1);
            const uint8_t* base = vbase + (int64_t)r0 * ldv2;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dma16_lds(base, (uint32_t)((min(kv0 + 16 * i + kr0, S - 1) - r0) * ldv2) + vchunk, sb + i * 4096);
        }
    };
    // V^T operand reads (ds_read_b64_tr_b16: in each 16-lane group, output lane 4 a + b, element e
    // is element b of source lane 4 e + a's 8 bytes).  For key step j, dim block b and part q,
    // source lane s of group G reads key row 16 j + 8 q + 4 (G / 2) + s / 4, dims 32 b + 16 (G % 2)
    // + 4 (s % 4) .. + 3; lane (l32, h) then holds keys 16 j + 8 q + 4 h + {0..3} of dim 32 b + l32
    // -- the P operand's key order.  Per lane: the byte offset within a stage of part 0 of key step
    // 0 for each b (key step and part add 4096 j + 2048 q).
    uint32_t vtr[4];
    {
        const int G = lane >> 4, s16 = lane & 15;
        const int rb = 4 * (G >> 1) + (s16 >> 2);
        const int cb = 2 * (G & 1) + ((s16 & 3) >> 1);
#pragma unroll
        for (int b = 0; b < 4; ++b)
            vtr[b] = (uint32_t)(rb * 256 + 64 * (b ^ (rb & 3)) + 16 * cb + 8 * (s16 & 1));
    }

    f32x16 oacc[4];                                             // O^T: 4 blocks of 32 dims x 32 queries
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[b][r] = 0.f;
    float m = -INFINITY, l = 0.f;                               // raw score units

    // causal mask of a block of 32 keys at kvb (only where it reaches past the wave's first query:
    // register r is key kvb + 8 (r / 4) + 4 h + r % 4, kept where it is <= qrow, then also < S for
    // every stored query), the block's row max, and the lazy raise of the running max m: only when a
    // score exceeds it by more than 8 / scale2 (then the weights exp2((s - m) scale2) stay below 2^8);
    // the rescale of the accumulators runs when any lane of the wave raises its max.  O / l does not
    // depend on m.  The first block holds key 0, so every query's max is finite from there on.
    auto front = [&](f32x16& sc, int kvb) {
        if (kvb + 31 > qw) {
            // a branch the compiler keeps: the blocks below the diagonal skip the mask entirely
            asm volatile("" ::: "memory");
            const int dq = qrow - kvb - 4 * h;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (8 * (r >> 2) + (r & 3) > dq) sc[r] = -INFINITY;
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, sc[r]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
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
    };
    // One block of 32 keys = key steps j0, j0 + 1 of the V tile at vst.  Key step j (16 keys): the
    // weights as the P^T B fragment (registers 8 (j - j0) .. + 7 of sc), each in two bf16 parts
    // (hi = bf16(p), lo = bf16(p - hi)), then O^T += V^T . P^T (the V^T operand of lane half h: keys
    // 16 j + 4 h + {0..3} and 16 j + 8 + 4 h + {0..3}, two transposing reads of the V tile).  With NEXT, the next block's scores S^T = K . Q^T (the K slot at kst, four MFMAs
    // per key step) go between them: independent work for the matrix cores under the softmax.
    auto block = [&](auto next, const f32x16& sc, int j0, const uint8_t* vst, f32x16& nxt, const uint8_t* kst) {
        constexpr bool NEXT = decltype(next)::value;
        const float mc = m * a.scale2;
        float psum = 0.f;
        if constexpr (NEXT) {
#pragma unroll
            for (int r = 0; r < 16; ++r) nxt[r] = 0.f;
        }
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float p0 = fexp2(__builtin_fmaf(sc[8 * jj + e], a.scale2, -mc));
                const float p1 = fexp2(__builtin_fmaf(sc[8 * jj + e + 1], a.scale2, -mc));
                psum += p0;
                psum += p1;
                const uint32_t w = pack_bf16(p0, p1);
                hw[e >> 1] = w;
                lw[e >> 1] = pack_bf16(p0 - __uint_as_float(w << 16), p1 - __uint_as_float(w & 0xffff0000u));
            }
            const bf16x8 phi = __builtin_bit_cast(bf16x8, uint4{hw[0], hw[1], hw[2], hw[3]});
            const bf16x8 plo = __builtin_bit_cast(bf16x8, uint4{lw[0], lw[1], lw[2], lw[3]});
            if constexpr (NEXT) {
#pragma unroll
                for (int s = 4 * jj; s < 4 * jj + 4; ++s) {
                    const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kst + k_off(l32, 2 * s + h));
                    nxt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], nxt, 0, 0, 0);
                }
            }
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = j0 + jj;
                const v4i16 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vst + vtr[b] + 4096 * j));
                const v4i16 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vst + vtr[b] + 4096 * j + 2048));
                const bf16x8 vf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
                oacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, phi, oacc[b], 0, 0, 0);
                oacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, plo, oacc[b], 0, 0, 0);
            }
        }
        psum += __shfl_xor(psum, 32);
        l += psum;
    };
    auto kslot = [&](int g) { return lds + (g & 3) * kKBlk; };
    auto vstage = [&](int t) { return lds + 4 * kKBlk + (t & 1) * kVBytes; };
    // Tile t (blocks 2 t, 2 t + 1) with a tile after it: every wave has keys <= its queries in all
    // tiles but the last.  On entry sa holds block 2 t's scores, K slots hold blocks 2 t + 1 and
    // 2 t + 2, V stage t & 1 tile t.  The DMAs refill the slots and the stage read in step t - 1
    // (published by its closing barrier).  P, the parity of t, makes the LDS offsets constants.
    f32x16 sa, sb;
    auto step = [&](auto P, int t) {
        constexpr int par = decltype(P)::value;
        issue_v(t + 1);
        issue_k(2 * t + 3);
        if (2 * t + 4 < nblk) issue_k(2 * t + 4);
        front(sa, t * kBK);
        block(std::true_type{}, sa, 0, vstage(par), sb, kslot(2 * par + 1));
        front(sb, t * kBK + 32);
        block(std::true_type{}, sb, 2, vstage(par), sa, kslot(2 * par + 2));
        // this wave's DMAs done and its LDS reads returned (the compiler may place the MFMAs that
        // consume the last reads after this statement; the stages they read are refilled right
        // after the barrier), then the barrier
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    // the last tile: only the waves with a key <= some query of theirs (a second block past the
    // wave's queries is all masked: weights 0)
    auto last = [&](auto P, int t) {
        constexpr int par = decltype(P)::value;
        if (t * kBK <= qw + 31) {
            front(sa, t * kBK);
            block(std::true_type{}, sa, 0, vstage(par), sb, kslot(2 * par + 1));
            front(sb, t * kBK + 32);
            block(std::false_type{}, sb, 2, vstage(par), sb, lds);
        }
    };

    issue_k(0);
    issue_v(0);
    issue_k(1);
    if (nblk > 2) issue_k(2);
    // every load complete (the query's too, so the compiler has no load of its own outstanding in
    // the loop and places no wait there), then the barrier that publishes the first blocks
#pragma unroll
    for (int s = 0; s < 8; ++s) asm volatile("" ::"v"(qf[s]));
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int r = 0; r < 16; ++r) sa[r] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(lds + k_off(l32, 2 * s + h));
        sa = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], sa, 0, 0, 0);
    }
    // slot 0 is refilled in step 0: every wave's block-0 reads first
    __syncthreads();
    using even = std::integral_constant<int, 0>;
    using odd = std::integral_constant<int, 1>;
    // pairs of tiles, then the tail (one exit: the register allocation of the loop stays simple)
    int t = 0;
    for (; t + 2 < ntiles; t += 2) {
        step(even{}, t);
        step(odd{}, t + 1);
    }
    if (t + 1 < ntiles) {
        step(even{}, t);
        last(odd{}, t + 1);
    } else {
        last(even{}, t);
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

// KV cache fill: k_cache / v_cache [H_KV, cap, 128] positions [0, S) from k and v (the
// reference's cudaMemcpy2DAsync of its head-major K/V, attention_block.cuh:355-364).  One workgroup
// per (64 positions, KV head); thread t copies chunk t % 16 of rows t / 16 + 16 u.
__global__ __launch_bounds__(256) void kv_cache_kernel(const uint16_t* __restrict__ k, int64_t ldk,
                                                       const uint16_t* __restrict__ v, int64_t ldv,
                                                       uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int cap,
                                                       int S) {
    const int p0 = blockIdx.x * 64, kvh = blockIdx.y, tid = threadIdx.x;
    const int c = tid & 15;
    uint4 kr[4], vr[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int p = min(p0 + (tid >> 4) + 16 * u, S - 1);
        kr[u] = load16(k + (int64_t)p * ldk + kvh * kD + 8 * c);
        vr[u] = load16(v + (int64_t)p * ldv + kvh * kD + 8 * c);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int p = p0 + (tid >> 4) + 16 * u;
        if (p < S) {
            *reinterpret_cast<uint4*>(kc + ((int64_t)kvh * cap + p) * kD + 8 * c) = kr[u];
            *reinterpret_cast<uint4*>(vc + ((int64_t)kvh * cap + p) * kD + 8 * c) = vr[u];
        }
    }
}

}  // namespace

hipError_t launch_kv_cache(const uint16_t* k, int64_t ldk, const uint16_t* v, int64_t ldv, int S, int H_KV,
                           uint16_t* k_cache, uint16_t* v_cache, int cap, hipStream_t stream) {
    hipLaunchKernelGGL(kv_cache_kernel, dim3((unsigned)((S + 63) / 64), H_KV), dim3(256), 0, stream, k, ldk, v, ldv,
                       k_cache, v_cache, cap, S);
    return hipGetLastError();
}

hipError_t launch_sdpa_prefill(const uint16_t* q, int64_t ldq, const uint16_t* k, int64_t ldk, const uint16_t* v,
                               int64_t ldv, uint16_t* o, int64_t ldo, int S, int H, int H_KV, hipStream_t stream) {
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&sdpa_prefill_kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
    if (attr != hipSuccess) return attr;
    PrefillArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.ldq = ldq;
    a.ldk = ldk;
    a.ldv = ldv;
    a.ldo = ldo;
    a.S = S;
    a.H = H;
    a.H_KV = H_KV;
    a.qtiles = (S + kBQ - 1) / kBQ;
    a.nslot = device_info().num_cu;
    a.scale2 = 1.4426950408889634f / sqrtf((float)kD);
    hipLaunchKernelGGL(sdpa_prefill_kernel, dim3(a.qtiles * H), dim3(256), kLds, stream, a);
    return hipGetLastError();
}

}  // namespace nmi
