// skinny16_fp8.hip -- fp8 (OCP e4m3) W8A16 linear for small M (up to 16 activation rows) on
// 16x16x32 bf16 MFMA (gfx950): one row tile per workgroup, K split between its waves.
//
//   y[m,n] = bf16_rne( (sum_k float(W[n,k]) * float(x[m,k])) * s[n] )
//
// The crossover between the reference's M == 1 GEMV (ops/gemv.cuh:48-104) and its prefill GEMM
// (ops/gemm.cuh:325-403, reached for every M > 1 at model/mlp_block.cuh:149-171).  Up to M = 16
// the work is bound by streaming W from HBM (<= 31.5 flop/B), and at the decode shapes a launch
// moves only 3-40 MB, so what sets its time is how many memory round trips lie on its critical
// path and how many bytes each CU keeps in flight.
//
// * A workgroup owns one row tile (16 R weight rows) over all of K; its NW waves split K into
//   contiguous runs of 256-k groups (four 64-k slabs).  Per slab, lane (r, p) = (lane % 16,
//   lane / 16) holds 16 codes of row 16 j + r (j < R) at k = 16 p and the 32 bytes
//   x[r][16 p .. 16 p + 15] (the activations are a few hundred KiB, read by every workgroup: L2
//   hits).  Codes 0-7 and 8-15 feed two v_mfma_f32_16x16x32_bf16 (A = weights: row r, k 8 p + e;
//   B = activations: column m = r); D[n][m] lands as rows 4 p + i, column r of lane (r, p).
//   Columns m >= M read row M - 1 and are not stored.
// * DMA form (the default, skinny16_dma_kernel): both operands go global -> LDS by
//   global_load_lds_dwordx4, the weights 4 rows x 256 contiguous bytes and the activations
//   2 rows x 512 bytes per instruction, into a few wave-private slots; each wave takes a
//   contiguous run of 256-k groups and reads the operands back in the MFMA layout.  Against the
//   row-run form (skinny16_rows_kernel, tuning knob s16.t = 1: weights staged through registers
//   into LDS, activations loaded in the MFMA layout, which touches 16 rows per instruction) it
//   measured 4-16% faster per launch on the config-2 shapes, the most at M = 16.  The row runs
//   remain for operands beyond the DMA form's 32-bit offsets.  (A direct form that loaded the
//   MFMA layout itself, 16 rows x 64 bytes per weight instruction, was 10-20% slower than the
//   row runs: DRAM efficiency.)
// * In the row-run form, loads go in batches, the next in flight while this one is
//   multiplied; every batch is issued (slabs past the wave's run read one word every lane
//   shares), so the compiler's wait counts are exact on every path.
// * The waves' sums meet in LDS and are added in wave order (a fixed order: results do not depend
//   on timing), then the per-row scale, one bf16 rounding and the epilogue.  No workspace, no
//   inter-workgroup communication.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

#include <algorithm>

namespace nmi {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Matrices of one launch: up to kS16MaxGroups, each with its own activations (x, ldx, K): the
// groups of a grouped call share them, a batch of independent linears does not.
constexpr int kS16MaxGroups = 8;

struct S16Group {
    const uint16_t* x;
    int64_t ldx;
    int K;
    const uint8_t* W;
    int64_t ldw;
    const float* s;
    uint16_t* y;
    int64_t ldy;
    const uint16_t* res;
    int64_t ldres;
    int N;
    int tile_begin;      // first row tile of this matrix in the launch's tile numbering
    int epi;
    int vec;             // s 16-byte aligned, y (and res) 8-byte aligned with row strides % 4 == 0
};

struct S16Args {
    int M;
    int ngroups;
    S16Group g[kS16MaxGroups];
};

// Stores four outputs n0 .. n0 + 3 of activation row m (lane layout of the MFMA result).
__device__ __forceinline__ void s16_store(const S16Group& G, int m, int n0, const f32x4 v) {
    if (n0 >= G.N) return;
    if (G.vec && n0 + 3 < G.N) {
        const float4 sc = *reinterpret_cast<const float4*>(G.s + n0);
        uint2 rr{0u, 0u};
        if (G.epi == kEpiResidual) rr = *reinterpret_cast<const uint2*>(G.res + (int64_t)m * G.ldres + n0);
        const uint16_t o0 = epilogue(v[0], sc.x, G.epi, (uint16_t)(rr.x & 0xFFFFu));
        const uint16_t o1 = epilogue(v[1], sc.y, G.epi, (uint16_t)(rr.x >> 16));
        const uint16_t o2 = epilogue(v[2], sc.z, G.epi, (uint16_t)(rr.y & 0xFFFFu));
        const uint16_t o3 = epilogue(v[3], sc.w, G.epi, (uint16_t)(rr.y >> 16));
        *reinterpret_cast<uint2*>(G.y + (int64_t)m * G.ldy + n0) =
            uint2{(uint32_t)o0 | ((uint32_t)o1 << 16), (uint32_t)o2 | ((uint32_t)o3 << 16)};
        return;
    }
    uint16_t rr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        rr[i] = (G.epi == kEpiResidual && n0 + i < G.N) ? G.res[(int64_t)m * G.ldres + n0 + i] : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (n0 + i < G.N) G.y[(int64_t)m * G.ldy + n0 + i] = epilogue(v[i], G.s[n0 + i], G.epi, rr[i]);
}

// Row-run form: the same products and sums, with the weights loaded as 4 rows x 256 contiguous
// bytes per instruction (lane 16 i + b: row 4 q + i of the load, 16-byte chunk b of a 256-k
// group of four slabs) and turned into the MFMA layout through a wave-private LDS region (rows
// 272 bytes apart: reads of 16 rows at one column hit distinct banks).  Longer contiguous runs
// per row than the 16 x 64 bytes of the direct form.  Each wave takes a contiguous run of
// groups; slabs past K are skipped.
template <int R, int NW, int D>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(R == 1 && D == 2 ? 4 : 1))) void
skinny16_rows_kernel(const S16Args a) {
    constexpr int kPitch = 272;                        // bytes per staged row
    __shared__ f32x4 red[NW][R][64];
    __shared__ __attribute__((aligned(16))) uint8_t stage[NW][16 * R * kPitch];

    const int tile = blockIdx.x;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kS16MaxGroups; ++i)
        if (i < a.ngroups && tile >= a.g[i].tile_begin) gi = i;
    const S16Group& G = a.g[gi];
    const int row0 = (tile - G.tile_begin) * 16 * R;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int r = lane & 15, p = lane >> 4;           // MFMA layout
    const int li = lane >> 4, lb = lane & 15;         // load layout: row 4 q + li, chunk lb
    const int M = a.M;
    const int S = G.K >> 6;
    const int G4 = (S + 3) >> 2;
    const int g_beg = wave * G4 / NW, g_end = (wave + 1) * G4 / NW;
    const int n = g_end - g_beg;
    const int nb = n;
    const int C = G.K >> 4;                            // 16-byte chunks per row

    const uint8_t* wrow[R][4];
#pragma unroll
    for (int j = 0; j < R; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) wrow[j][q] = G.W + (int64_t)min(row0 + 16 * j + 4 * q + li, G.N - 1) * G.ldw;
    const uint16_t* xrow = G.x + (int64_t)min(r, M - 1) * G.ldx + 16 * p;
    const uint8_t* wdummy = G.W;
    const uint16_t* xdummy = G.x;
    uint8_t* st = stage[wave];

    struct Batch {
        u32x4 w[R][4];
        u32x4 x[4][2];
    };
    auto load = [&](Batch& bt, int b) {
        const bool ok = b < n;
        const int g4 = g_beg + b;
        const int chunk = min(g4 * 16 + lb, C - 1);
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                bt.w[j][q] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(ok ? wrow[j][q] + (int64_t)chunk * 16 : wdummy));
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
            const int s = g4 * 4 + sl;
            const bool sok = ok && s < S;
            const uint16_t* xp = sok ? xrow + s * 64 : xdummy;
            bt.x[sl][0] = *reinterpret_cast<const u32x4*>(xp);
            bt.x[sl][1] = *reinterpret_cast<const u32x4*>(sok ? xp + 8 : xdummy);
        }
    };

    f32x4 acc[R];
#pragma unroll
    for (int j = 0; j < R; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](const Batch& bt, int b) {
        if (b >= n) return;
        const int g4 = g_beg + b;
        // the group's rows into the wave's region, then read back in the MFMA layout (one wave
        // writes and reads it: LDS keeps a wave's operations in order)
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<u32x4*>(st + (16 * j + 4 * q + li) * kPitch + 16 * lb) = bt.w[j][q];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
            if (g4 * 4 + sl >= S) break;
            const bf16x8 B0 = __builtin_bit_cast(bf16x8, bt.x[sl][0]);
            const bf16x8 B1 = __builtin_bit_cast(bf16x8, bt.x[sl][1]);
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(st + (16 * j + r) * kPitch + sl * 64 + 16 * p);
                const uint2 c0 = e4m3x4_to_bf16(w[0]), c1 = e4m3x4_to_bf16(w[1]);
                const uint2 c2 = e4m3x4_to_bf16(w[2]), c3 = e4m3x4_to_bf16(w[3]);
                const bf16x8 A0 = __builtin_bit_cast(bf16x8, uint4{c0.x, c0.y, c1.x, c1.y});
                const bf16x8 A1 = __builtin_bit_cast(bf16x8, uint4{c2.x, c2.y, c3.x, c3.y});
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, B0, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, B1, acc[j], 0, 0, 0);
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    // D groups in flight: buffer d holds groups d, d + D, d + 2 D, ...
    Batch bt[D];
#pragma unroll
    for (int d = 0; d < D; ++d) load(bt[d], d);
    for (int b = 0; b < nb; b += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            consume(bt[d], b + d);
            load(bt[d], b + d + D);
        }
    }

#pragma unroll
    for (int j = 0; j < R; ++j) red[wave][j][lane] = acc[j];
    __syncthreads();
    if (wave < R) {
        f32x4 v = red[0][wave][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const f32x4 u = red[w][wave][lane];
            v = f32x4{v[0] + u[0], v[1] + u[1], v[2] + u[2], v[3] + u[3]};
        }
        if (r < M) s16_store(G, r, row0 + 16 * wave + 4 * p, v);
    }
}

// DMA form: the same products and sums, with both operands brought global -> LDS by
// global_load_lds_dwordx4 (no register staging, no LDS store instructions) into D slots per
// wave.  A slot holds one 256-k group: the weights, 16 R rows x 256 bytes (4 rows per
// instruction), and the activations, 16 rows x 512 bytes (2 rows per instruction: 1 KiB of
// consecutive bytes, where the MFMA layout touches 16 rows per instruction).  A DMA instruction
// writes 1 KiB of consecutive LDS (lane l at 16 l), so the layout is set by which global chunk
// each lane fetches: chunk c of local row r (r < 16) sits at chunk position c ^ r of its row,
// and a fragment read (16 rows, one logical chunk) hits 16 distinct bank groups.  Waits are
// explicit vmcnt counts (every group issues the same instructions, and only groups of the wave's
// run are issued: a wait counts the groups issued after the one it waits for).
// XR activation rows are staged: 16, 8 where M <= 8, 4 where M <= 4 (lanes of MFMA columns
// XR .. 15 then read row XR - 1, and their products are dropped).  Fewer staged rows measured
// faster: M = 8 on 8 rows 40.4 against 42.7 us per config-2 step on 16, M = 2 on 4 rows 33.4-34.1
// against 34.3 on 8.
constexpr int kS16DmaW = 4096;                         // bytes per slot and row tile

template <int R, int NW, int D, int XR>
constexpr int s16_dma_lds() {
    return NW * D * (R * kS16DmaW + XR * 512) + NW * R * 64 * 16;
}

template <int R, int NW, int D, int XR>
__global__ __launch_bounds__(64 * NW) void skinny16_dma_kernel(const S16Args a) {
    constexpr int kW = R * kS16DmaW, kSlot = kW + XR * 512;
    constexpr int kPer = 4 * R + XR / 2;               // DMA instructions per group
    static_assert(D >= 1 && D <= 3 && (D - 1) * kPer <= 63, "vmcnt range");
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ __attribute__((aligned(16))) uint8_t s16_lds[];

    const int tile = blockIdx.x;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kS16MaxGroups; ++i)
        if (i < a.ngroups && tile >= a.g[i].tile_begin) gi = i;
    const S16Group& G = a.g[gi];
    const int row0 = (tile - G.tile_begin) * 16 * R;

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int r = lane & 15, p = lane >> 4;           // MFMA layout
    const int M = a.M;
    const int S = G.K >> 6;
    const int G4 = (S + 3) >> 2;
    const int g_beg = wave * G4 / NW, g_end = (wave + 1) * G4 / NW;
    const int n = g_end - g_beg;
    const int CW = G.K >> 4;                           // 16-byte chunks per weight row
    const int CX = G.K >> 3;                           // 16-byte chunks per activation row

    uint8_t* const slots = s16_lds + wave * D * kSlot;
    const uint32_t lds_slots = (uint32_t)(uintptr_t)(lds_void*)slots;
    f32x4* const red = reinterpret_cast<f32x4*>(s16_lds + NW * D * kSlot);

    // per-lane row offsets and chunk swizzles: weights, instruction (j, q) -> local row 4 q + lane / 16,
    // position lane % 16; activations, instruction i -> row 2 i + lane / 32, position lane % 32
    uint32_t wbase[R][4];
    int wsw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int rl = 4 * q + (lane >> 4);
        wsw[q] = (lane & 15) ^ rl;
#pragma unroll
        for (int j = 0; j < R; ++j)
            wbase[j][q] = (uint32_t)((int64_t)min(row0 + 16 * j + rl, G.N - 1) * G.ldw);
    }
    const int xl = lane & 31, xh = lane >> 5;

    auto issue = [&](int b, int d) {
        if (b >= n) return;
        const int g4 = g_beg + b;
        const uint32_t sw = lds_slots + (uint32_t)(d * kSlot);
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                dma16_lds_nt(G.W, wbase[j][q] + 16u * (uint32_t)min(g4 * 16 + wsw[q], CW - 1),
                        sw + (uint32_t)((4 * j + q) * 1024));
#pragma unroll
        for (int i = 0; i < XR / 2; ++i) {
            const int rho = 2 * i + xh;
            const uint32_t xoff = (uint32_t)((int64_t)min(rho, M - 1) * G.ldx * 2);
            dma16_lds(G.x, xoff + 16u * (uint32_t)min(g4 * 32 + (xl ^ rho), CX - 1), sw + (uint32_t)(kW + i * 1024));
        }
    };

    f32x4 acc[R];
#pragma unroll
    for (int j = 0; j < R; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](int b, int d) {
        if (b >= n) return;
        const int g4 = g_beg + b;
        const uint8_t* sw = slots + d * kSlot;
        const int xr = min(r, XR - 1);
        const uint8_t* sx = sw + kW + xr * 512;
        struct Slab {
            u32x4 x0, x1, w[R];
        };
        auto read = [&](Slab& o, int sl) {
            o.x0 = *reinterpret_cast<const u32x4*>(sx + 16 * ((8 * sl + 2 * p) ^ xr));
            o.x1 = *reinterpret_cast<const u32x4*>(sx + 16 * ((8 * sl + 2 * p + 1) ^ xr));
#pragma unroll
            for (int j = 0; j < R; ++j)
                o.w[j] = *reinterpret_cast<const u32x4*>(sw + j * 4096 + r * 256 + 16 * ((4 * sl + p) ^ r));
        };
        auto mma = [&](const Slab& o) {
            const bf16x8 B0 = __builtin_bit_cast(bf16x8, o.x0);
            const bf16x8 B1 = __builtin_bit_cast(bf16x8, o.x1);
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const u32x4 w = o.w[j];
                const uint2 c0 = e4m3x4_to_bf16(w[0]), c1 = e4m3x4_to_bf16(w[1]);
                const uint2 c2 = e4m3x4_to_bf16(w[2]), c3 = e4m3x4_to_bf16(w[3]);
                const bf16x8 A0 = __builtin_bit_cast(bf16x8, uint4{c0.x, c0.y, c1.x, c1.y});
                const bf16x8 A1 = __builtin_bit_cast(bf16x8, uint4{c2.x, c2.y, c3.x, c3.y});
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, B0, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, B1, acc[j], 0, 0, 0);
            }
        };
        if (g4 * 4 + 4 <= S) {                         // a whole group: every LDS read first
            Slab o[4];
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) read(o[sl], sl);
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) mma(o[sl]);
        } else {
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) {
                if (g4 * 4 + sl >= S) break;
                Slab o;
                read(o, sl);
                mma(o);
            }
        }
    };

    // slot d holds groups d, d + D, ...; when group b is consumed, groups b + 1 .. min(n, b + D) - 1
    // have been issued after it; before a slot is refilled its LDS reads have completed
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
    for (int b = 0; b < n; b += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int after = min(n - 1 - (b + d), D - 1);
            if (after >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kPer) : "memory");
            else if (after == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kPer) : "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            consume(b + d, d);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(b + d + D, d);
        }
    }

#pragma unroll
    for (int j = 0; j < R; ++j) red[(wave * R + j) * 64 + lane] = acc[j];
    __syncthreads();
    if (wave < R) {
        f32x4 v = red[wave * 64 + lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const f32x4 u = red[(w * R + wave) * 64 + lane];
            v = f32x4{v[0] + u[0], v[1] + u[1], v[2] + u[2], v[3] + u[3]};
        }
        if (r < M) s16_store(G, r, row0 + 16 * wave + 4 * p, v);
    }
}

// One matrix of a launch and its activations.
struct S16Input {
    const uint16_t* x;
    int64_t ldx;
    int K;
};

// Fills the launch's group table (the row tiles of each matrix in turn); returns the tile count.
// The matrices go in order of decreasing K (a stable order): a tile's time grows with K, and the
// dispatcher hands out workgroups in tile order, so the longest tiles start in the first round
// and the short ones fill the gaps behind them instead of forming the launch's tail (config 2's
// batch: down_proj's K = 12544 tiles, four times an up_proj tile, were dispatched last).  Which
// workgroup computes a tile does not change its result.
template <int R>
int s16_tables(S16Args& a, const GemvGroup* groups, const S16Input* in, int ng) {
    int order[kS16MaxGroups];
    for (int i = 0; i < ng; ++i) {
        int j = i;
        for (; j > 0 && in[order[j - 1]].K < in[i].K; --j) order[j] = order[j - 1];
        order[j] = i;
    }
    int tb = 0;
    for (int t = 0; t < ng; ++t) {
        const int i = order[t];
        const GemvGroup& G = groups[i];
        const Epi& e = G.epi;
        const bool res = e.kind == kEpiResidual;
        const bool vec = (reinterpret_cast<uintptr_t>(G.s) & 15) == 0 && (reinterpret_cast<uintptr_t>(G.y) & 7) == 0 &&
                         (G.ldy & 3) == 0 &&
                         (!res || ((reinterpret_cast<uintptr_t>(e.res) & 7) == 0 && (e.ldres & 3) == 0));
        a.g[t] = S16Group{in[i].x, in[i].ldx, in[i].K, G.W, G.ldw, G.s, G.y, G.ldy, res ? e.res : nullptr, e.ldres, G.N,
                          tb, e.kind, vec ? 1 : 0};
        tb += (G.N + 16 * R - 1) / (16 * R);
    }
    return tb;
}

template <int R, int NW, int D, int XR>
hipError_t s16_dma_launch(S16Args& a, const GemvGroup* groups, const S16Input* in, int ng, hipStream_t stream) {
    constexpr int lds = s16_dma_lds<R, NW, D, XR>();
    static_assert(lds <= 152 * 1024, "LDS");
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&skinny16_dma_kernel<R, NW, D, XR>), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    const int tb = s16_tables<R>(a, groups, in, ng);
    if (tb < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL((skinny16_dma_kernel<R, NW, D, XR>), dim3(tb), dim3(64 * NW), lds, stream, a);
    return hipGetLastError();
}

template <int R, int NW>
hipError_t s16_rows_launch(S16Args& a, const GemvGroup* groups, const S16Input* in, int ng, hipStream_t stream) {
    const int tb = s16_tables<R>(a, groups, in, ng);
    if (tb < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL((skinny16_rows_kernel<R, NW, 2>), dim3(tb), dim3(64 * NW), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

// Where this kernel is taken (tuning knob s16 = 2: never): 2 <= M <= 16; M = 2 only when the
// GEMV kernel would not fuse an RMSNorm (the caller decides).  Measured on MI355X (bench, config
// 2, four launches per step, DMA form with non-temporal weight loads): M = 2 34.4 against 38.5 us
// on the stream GEMV, M = 4 35.6 against 43.3 on the 4x4x4 kernel, M = 8 38.3 against 53, M = 16
// 44.2 against 74.
bool skinny16_wanted(int M, int K) {
    const int knob = tuning().s16;
    (void)K;
    return knob != 2 && M >= 2 && M <= 16;
}

namespace {

// The launch behind both entries below: matrices `groups` with their activations `in` (M rows
// each), one row tile per workgroup.
bool s16_launch(const GemvGroup* groups, const S16Input* in, int ngroups, int M, bool batch, hipStream_t stream,
                hipError_t* err) {
    if (ngroups < 1 || ngroups > kS16MaxGroups) return false;
    int64_t rows = 0;
    for (int i = 0; i < ngroups; ++i) {
        if (!skinny16_wanted(M, in[i].K) || in[i].K < 64 || in[i].K % 64 != 0) return false;
        if ((reinterpret_cast<uintptr_t>(in[i].x) & 15) != 0 || (in[i].ldx & 7) != 0) return false;
        if ((reinterpret_cast<uintptr_t>(groups[i].W) & 15) != 0 || (groups[i].ldw & 15) != 0) return false;
        rows += groups[i].N;
    }
    S16Args a{};
    a.M = M;
    a.ngroups = ngroups;
    // Row tiles of 32 from 4096 rows (half the activation reads per weight byte), else 16 (more
    // workgroups); four waves per workgroup, two where the row tiles outnumber the CUs (more,
    // shorter-lived workgroups resident per CU: all of a launch's tiles in one round); two groups
    // in flight per wave.  Measured on MI355X for the row-run form, kernel time at M = 8 / 16: four
    // waves against eight q 8.7 / 9.6 vs 9.2 / 10.2 us, k 6.8 / 7.9 vs 7.3 / 8.2, o 8.6 / 10.4 vs
    // 9.5 / 11.0, down 13.7 / 17.6 vs 14.4 / 18.5; up (392 tiles) with two waves 13.6 / 15.2
    // against 14.3 / 16.1 (four) and 16.2 / 18.4 (eight).  The DMA form (default; it needs 32-bit
    // offsets within x and each W) keeps the same choices: eager per-launch time at M = 8 / 16
    // against the row runs q 9.7 / 9.9 vs 10.5 / 10.9 us, o 9.5 / 9.8 vs 9.7 / 10.9, up 12.9 /
    // 14.0 vs 13.5 / 15.3, down 12.9 / 14.6 vs 13.6 / 17.3; three groups in flight measured 1-2 us
    // slower per launch (the LDS holds fewer waves), eight waves with 8 staged rows equal within
    // the noise.  Tuning knobs: s16.r (1, 2) forces the row tile, s16.w (2, 4) the waves, s16.t = 1
    // the row-run form.
    const Tuning& tn = tuning();
    // A batch of independent linears (one launch over a whole decode set, thousands of row
    // tiles, the longest-K matrices first) takes its own choices, measured on MI355X for config
    // 2's six linears (one box, the other forms in brackets): row tiles of 16 up to M = 8 (M = 8
    // 26.8 us [28.3 with 32]), of 32 above (M = 16 29.5 [41.4 with 16]); two waves per workgroup
    // above M = 4 (M = 16 29.5 [32.1 with four]), four at M <= 4 (M = 2 22.9 [23.3 with two]).
    const int R = tn.s16_r == 1 || tn.s16_r == 2 ? tn.s16_r : batch ? (M <= 8 ? 1 : 2) : (rows >= 4096 ? 2 : 1);
    int tiles = 0;
    for (int i = 0; i < ngroups; ++i) tiles += (groups[i].N + 16 * R - 1) / (16 * R);
    const bool four = tn.s16_w == 2 || tn.s16_w == 4 ? tn.s16_w == 4 : batch ? M <= 4 : tiles <= device_info().num_cu;
    bool dma_ok = true;
    for (int i = 0; i < ngroups; ++i)
        dma_ok = dma_ok && (in[i].ldx * 2) * (int64_t)(M - 1) + 2 * (int64_t)in[i].K < ((int64_t)1 << 31) &&
                 groups[i].ldw * (int64_t)(groups[i].N - 1) + in[i].K < ((int64_t)1 << 31);
    if (tn.s16_t != 1 && dma_ok) {
        if (M <= 4) {                                  // 4 staged activation rows
            const int f4 = (R == 2 ? 2 : 0) + (four ? 1 : 0);
            switch (f4) {
                case 0: *err = s16_dma_launch<1, 2, 2, 4>(a, groups, in, ngroups, stream); break;
                case 1: *err = s16_dma_launch<1, 4, 2, 4>(a, groups, in, ngroups, stream); break;
                case 2: *err = s16_dma_launch<2, 2, 2, 4>(a, groups, in, ngroups, stream); break;
                default: *err = s16_dma_launch<2, 4, 2, 4>(a, groups, in, ngroups, stream); break;
            }
            return true;
        }
        const int form = (M <= 8 ? 4 : 0) + (R == 2 ? 2 : 0) + (four ? 1 : 0);
        switch (form) {
            case 0: *err = s16_dma_launch<1, 2, 2, 16>(a, groups, in, ngroups, stream); break;
            case 1: *err = s16_dma_launch<1, 4, 2, 16>(a, groups, in, ngroups, stream); break;
            case 2: *err = s16_dma_launch<2, 2, 2, 16>(a, groups, in, ngroups, stream); break;
            case 3: *err = s16_dma_launch<2, 4, 2, 16>(a, groups, in, ngroups, stream); break;
            case 4: *err = s16_dma_launch<1, 2, 2, 8>(a, groups, in, ngroups, stream); break;
            case 5: *err = s16_dma_launch<1, 4, 2, 8>(a, groups, in, ngroups, stream); break;
            case 6: *err = s16_dma_launch<2, 2, 2, 8>(a, groups, in, ngroups, stream); break;
            default: *err = s16_dma_launch<2, 4, 2, 8>(a, groups, in, ngroups, stream); break;
        }
        return true;
    }
    const int form = (R == 2 ? 2 : 0) + (four ? 1 : 0);
    switch (form) {
        case 0: *err = s16_rows_launch<1, 2>(a, groups, in, ngroups, stream); break;
        case 1: *err = s16_rows_launch<1, 4>(a, groups, in, ngroups, stream); break;
        case 2: *err = s16_rows_launch<2, 2>(a, groups, in, ngroups, stream); break;
        default: *err = s16_rows_launch<2, 4>(a, groups, in, ngroups, stream); break;
    }
    return true;
}

}  // namespace

bool launch_skinny16_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups, int ngroups,
                             hipStream_t stream, hipError_t* err) {
    if (ngroups < 1 || ngroups > kMaxGroups) return false;
    S16Input in[kMaxGroups];
    for (int i = 0; i < ngroups; ++i) in[i] = S16Input{x, ldx, K};
    return s16_launch(groups, in, ngroups, M, false, stream, err);
}

bool launch_skinny16_batch(const uint16_t* const* xs, const int64_t* ldxs, const int* Ks, const GemvGroup* groups,
                           int n, int M, hipStream_t stream, hipError_t* err) {
    if (n < 1 || n > kS16MaxGroups) return false;
    S16Input in[kS16MaxGroups];
    for (int i = 0; i < n; ++i) in[i] = S16Input{xs[i], ldxs[i], Ks[i]};
    return s16_launch(groups, in, n, M, true, stream, err);
}

}  // namespace nmi
