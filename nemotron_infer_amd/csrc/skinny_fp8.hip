// skinny_fp8.hip -- fp8 (OCP e4m3) W8A16 linear for 1 <= M <= 16 on bf16 MFMA (gfx950).
//
//   y[m,n] = bf16_rne( (sum_k float(W[n,k]) * float(x[m,k])) * s[n] )
//
// The weight-streaming kernel behind the reference's GEMV/GEMM crossover: the reference
// sends M == 1 to its GEMV (nemotron_infer/csrc/include/ops/gemv.cuh:48-104) and every
// M > 1 to activation quantization plus cuBLASLt (ops/gemm.cuh:257-403,
// model/mlp_block.cuh:142-171).  For M <= 16 the work is HBM-bound on W (<= 31.5 flop/B),
// so this kernel streams W once and keeps x in bf16:
//
// * One wave computes a 16-row tile of W against all M activation rows with
//   v_mfma_f32_16x16x32_bf16: A = 16 weight rows x 32 k (converted from e4m3 in registers
//   with v_cvt_scalef32_pk_bf16_fp8 -- exact), B = 32 k x 16 activation rows (rows >= M read
//   a zero word), so the reduction over k happens inside the matrix core.
// * Lane l loads 16 bytes of weight row (l % 16): chunk (l / 16) + 4 i of the wave's K slice,
//   i.e. each load instruction fetches 64 contiguous bytes of each of 16 rows.  The 16 codes
//   feed two MFMAs (codes 0-7 and 8-15); B holds x at the same k.
// * x [M, K-range] is staged per workgroup in LDS as bf16 (low and high 8 elements of each
//   16-element chunk apart, rows padded to an odd number of 16-byte words so that the 16
//   activation rows of one read land in different banks).
// * K is split between the KSW waves of a workgroup (partials summed through LDS in a fixed
//   order) and, when the caller provides a workspace, between KG workgroups: each writes its
//   float32 partial tile to the workspace, and the last workgroup of a row block (arrival
//   counter) adds the KG partials in order 0..KG-1, so results do not depend on timing.
// * Epilogue: per-row scale in float32, one bf16 RNE rounding.
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kWaves = 4;
constexpr int kTileRows = 16;
constexpr int kXPieces = 8;                       // 16-byte x pieces staged per thread
constexpr int kMaxStagePieces = 256 * kXPieces;   // per window: 2 * M * window <= 2048
// Workspace layout: a fixed block of arrival counters (so that calls of different shapes can
// share one workspace: a counter slot is only ever a counter), then the float32 partials.
constexpr int kCounterSlots = 16384;
constexpr size_t kCounterBytes = kCounterSlots * sizeof(uint32_t);

struct SkinnyArgs {
    const uint16_t* x;
    int64_t ldx;              // elements between activation rows
    int M, K;
    int kgroups;              // workgroups that split K (1: no workspace)
    int cpg;                  // 16-byte chunks per K group
    int window;               // chunks per LDS window
    int ngroups;
    GemvGroup g[kMaxGroups];  // wg_begin counts row blocks
    float* ws;                // [kgroups][M][ws_ld] partials (kgroups > 1)
    uint32_t* counters;       // one per row block; zero between launches
    int ws_ld;                // sum of N over the groups
};

// bf16x8 view of four dwords.
__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(bf16x8, u32x4_t{a, b, c, d});
}

// Residual bits of output (m, n), n clamped into the row (read only for kEpiResidual).
__device__ __forceinline__ uint16_t residual(const GemvGroup& grp, int m, int n) {
    return grp.epi.kind == kEpiResidual ? grp.epi.res[(int64_t)m * grp.epi.ldres + min(n, grp.N - 1)] : 0;
}

template <int U, int KSW>
__global__ __launch_bounds__(256) void skinny_fp8_kernel(const SkinnyArgs a) {
    extern __shared__ uint4 xs[];                 // [M][rs] words, then one zero word
    constexpr int kTiles = kWaves / KSW;
    constexpr int kRowsPerWG = kTiles * kTileRows;
    __shared__ f32x4 red[KSW][kTiles][64];
    __shared__ uint32_t last_flag;

    const int blk = (int)blockIdx.x;
    const int rb_all = blk / a.kgroups;
    const int kg = blk - rb_all * a.kgroups;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < a.ngroups && rb_all >= a.g[i].wg_begin) gi = i;
    const GemvGroup grp = a.g[gi];
    const int rb = rb_all - grp.wg_begin;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int t = wave / KSW;                  // row tile of this wave
    const int q = wave % KSW;                  // K slice of this wave
    const int m = lane & 15;                   // B column (activation row) / A row (weight row)
    const int a4 = lane >> 4;                  // k slot of this lane
    const int row0 = rb * kRowsPerWG + t * kTileRows;
    // Weight rows past N read row N-1 (in bounds); their outputs are never stored.
    const uint8_t* __restrict__ wrow = grp.W + (int64_t)min(row0 + m, grp.N - 1) * grp.ldw;
    const int M = a.M;
    const int C = a.K >> 4;
    const int kb = kg * a.cpg;
    const int ke = min(C, kb + a.cpg);
    const int window = a.window;
    const int rs = 2 * window + 1;             // odd row stride in 16-byte words
    const int zero_word = M * rs;
    if (tid == 0) xs[zero_word] = uint4{0, 0, 0, 0};

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int w0 = kb; w0 < ke; w0 += window) {
        const int wc = min(window, ke - w0);
        const int npieces = 2 * M * wc;
        // 1. activation pieces of this window (issued before the weights)
        uint4 xr[kXPieces];
#pragma unroll
        for (int p = 0; p < kXPieces; ++p) {
            const int e = min(tid + 256 * p, npieces - 1);
            const int mm = e / (2 * wc);
            const int rem = e - mm * 2 * wc;
            xr[p] = load16(a.x + (int64_t)mm * a.ldx + (int64_t)(w0 + (rem >> 1)) * 16 + (rem & 1) * 8);
        }
        // 2. first batch of weights of this wave's slice [cb, ce)
        const int cb = w0 + (q * wc) / KSW;
        const int ce = w0 + ((q + 1) * wc) / KSW;
        const int clast = min(max(ce - 1, cb), C - 1);
        int c0 = cb + a4;
        uint4 wv[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            wv[u] = load_stream16(wrow + (int64_t)min(c0 + 4 * u, clast) * 16);
        // 3. stage x once the previous window has been consumed
        if (w0 != kb) __syncthreads();
#pragma unroll
        for (int p = 0; p < kXPieces; ++p) {
            const int e = tid + 256 * p;
            if (e < npieces) {
                const int mm = e / (2 * wc);
                const int rem = e - mm * 2 * wc;
                xs[mm * rs + (rem & 1) * window + (rem >> 1)] = xr[p];
            }
        }
        __syncthreads();
        // 4. consume.  Slots past the slice (or activation rows >= M) take B from the zero
        //    word: their A values are codes of the same weight row, so a product with them
        //    is +-0 unless the row holds a NaN code, in which case the row's result is NaN
        //    anyway.
        const bool mvalid = m < M;
        const int xrow = m * rs - w0;
        for (;;) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + 4 * u;
                const bool valid = mvalid && (c < ce);
                const int lo = valid ? xrow + c : zero_word;
                const int hi = valid ? xrow + window + c : zero_word;
                const uint4 xl = xs[lo], xh = xs[hi];
                const uint2 p0 = e4m3x4_to_bf16(wv[u].x), p1 = e4m3x4_to_bf16(wv[u].y);
                const uint2 p2 = e4m3x4_to_bf16(wv[u].z), p3 = e4m3x4_to_bf16(wv[u].w);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(p0.x, p0.y, p1.x, p1.y), as_bf16x8(xl.x, xl.y, xl.z, xl.w), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(p2.x, p2.y, p3.x, p3.y), as_bf16x8(xh.x, xh.y, xh.z, xh.w), acc, 0, 0, 0);
            }
            c0 += 4 * U;
            if (c0 - a4 >= ce) break;           // uniform: every lane's next slot is past ce
#pragma unroll
            for (int u = 0; u < U; ++u)
                wv[u] = load_stream16(wrow + (int64_t)min(c0 + 4 * u, clast) * 16);
        }
    }

    // Lane l holds D[row 4 (l / 16) + i][column l % 16] = partial y[m][row0 + 4 (l / 16) + i].
    red[q][t][lane] = acc;
    __syncthreads();
    if (q == 0) {
        f32x4 sum = red[0][t][lane];
#pragma unroll
        for (int qq = 1; qq < KSW; ++qq) {
            const f32x4 v = red[qq][t][lane];
            sum = f32x4{sum.x + v.x, sum.y + v.y, sum.z + v.z, sum.w + v.w};
        }
        red[0][t][lane] = sum;
    }
    const int ncol = grp.ws_col;                // column of this group in the workspace
    if (a.kgroups > 1) {
        // Write this workgroup's partial tile with agent-scope stores (written through to
        // the level every XCD sees), wait until they have completed, and count the row
        // block's arrivals; the last arrival reads the partials back with agent-scope loads
        // and sums them in K-group order.  No cache-wide fence is needed: every word that
        // crosses workgroups is accessed only with agent-scope operations.
        if (q == 0 && m < M) {
            const f32x4 v = red[0][t][lane];
            float* dst = a.ws + ((int64_t)kg * M + m) * a.ws_ld + ncol + row0 + 4 * a4;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (row0 + 4 * a4 + i < grp.N)
                    __hip_atomic_store(dst + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);          // this wave's partial stores have completed
        __syncthreads();
        if (tid == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(a.counters + rb_all, 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            last_flag = (prev == (uint32_t)(a.kgroups - 1)) ? 1u : 0u;
        }
        __syncthreads();
        if (!last_flag) return;
        if (q == 0 && m < M) {
            uint16_t rres[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) rres[i] = residual(grp, m, row0 + 4 * a4 + i);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = row0 + 4 * a4 + i;
                if (n < grp.N) {
                    const float* src = a.ws + (int64_t)m * a.ws_ld + ncol + n;
                    float tsum = 0.f;
                    for (int g2 = 0; g2 < a.kgroups; ++g2)
                        tsum += __hip_atomic_load(src + (int64_t)g2 * M * a.ws_ld, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                    grp.y[(int64_t)m * grp.ldy + n] = epilogue(tsum, grp.s[n], grp.epi.kind, rres[i]);
                }
            }
        }
        if (tid == 0) __hip_atomic_store(a.counters + rb_all, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (q == 0 && m < M) {
        const f32x4 v = red[0][t][lane];
        uint16_t rres[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) rres[i] = residual(grp, m, row0 + 4 * a4 + i);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = row0 + 4 * a4 + i;
            if (n < grp.N) grp.y[(int64_t)m * grp.ldy + n] = epilogue(v[i], grp.s[n], grp.epi.kind, rres[i]);
        }
    }
}

template <int U, int KSW>
hipError_t launch_cfg(SkinnyArgs& a, hipStream_t stream) {
    constexpr int rows_per_wg = (kWaves / KSW) * kTileRows;
    int blocks = 0, col = 0;
    for (int i = 0; i < a.ngroups; ++i) {
        a.g[i].wg_begin = blocks;
        a.g[i].ws_col = col;
        blocks += (a.g[i].N + rows_per_wg - 1) / rows_per_wg;
        col += a.g[i].N;
    }
    a.ws_ld = col;
    const size_t lds = ((size_t)a.M * (2 * a.window + 1) + 1) * sizeof(uint4);
    hipLaunchKernelGGL((skinny_fp8_kernel<U, KSW>), dim3(blocks * a.kgroups), dim3(256), lds, stream, a);
    return hipGetLastError();
}

template <int U>
hipError_t launch_ksw(int ksw, SkinnyArgs& a, hipStream_t stream) {
    switch (ksw) {
        case 1: return launch_cfg<U, 1>(a, stream);
        case 2: return launch_cfg<U, 2>(a, stream);
        default: return launch_cfg<U, 4>(a, stream);
    }
}

struct Plan {
    int ksw, kgroups, cpg, window, u;
};

// Chunks per LDS window for M activation rows (2 * M * window pieces of 16 B per window).
int max_window(int M) { return kMaxStagePieces / (2 * M); }

Plan plan(int M, int K, int64_t rows, int num_cu, bool have_ws) {
    const int C = K >> 4;
    Plan p{};
    const int wmax = max_window(M);
    const Tuning& tn = tuning();
    // K groups: enough that one window covers a group's K range, and (with a workspace)
    // enough workgroups to give every CU about three.
    p.kgroups = 1;
    if (have_ws) {
        p.kgroups = (C + wmax - 1) / wmax;
        const int64_t blocks64 = (rows + 63) / 64;
        while (p.kgroups < 64 && blocks64 * p.kgroups < 3 * (int64_t)num_cu && C / (p.kgroups + 1) >= 16)
            ++p.kgroups;
        if (tn.skinny_kg > 0) p.kgroups = tn.skinny_kg;
    }
    p.cpg = (C + p.kgroups - 1) / p.kgroups;
    p.kgroups = (C + p.cpg - 1) / p.cpg;
    p.window = p.cpg < wmax ? p.cpg : wmax;
    // Waves per row tile splitting K: more when there are few row blocks.
    p.ksw = 1;
    const int64_t wgs1 = (rows + 63) / 64 * p.kgroups;
    if (wgs1 < 2 * (int64_t)num_cu) p.ksw = (wgs1 * 2 < 2 * (int64_t)num_cu) ? 4 : 2;
    if (tn.skinny_ks == 1 || tn.skinny_ks == 2 || tn.skinny_ks == 4) p.ksw = tn.skinny_ks;
    p.u = (p.window / (4 * p.ksw) > 8) ? 16 : 8;
    if (tn.skinny_u == 8 || tn.skinny_u == 16) p.u = tn.skinny_u;
    return p;
}

}  // namespace

size_t skinny_workspace_bytes(int M, int K, int64_t total_rows, int num_cu) {
    const Plan p = plan(M, K, total_rows, num_cu, true);
    if (p.kgroups <= 1) return 0;
    // row blocks of any KSW (>= 16 rows each) plus one partial block per group
    if ((total_rows + kTileRows - 1) / kTileRows + kMaxGroups > kCounterSlots) return 0;
    return kCounterBytes + (size_t)p.kgroups * M * total_rows * sizeof(float);
}

hipError_t launch_skinny_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                                 int ngroups, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const DeviceInfo& dev = device_info();
    int64_t rows = 0;
    for (int i = 0; i < ngroups; ++i) rows += groups[i].N;
    const bool have_ws = workspace != nullptr &&
                         workspace_bytes >= skinny_workspace_bytes(M, K, rows, dev.num_cu) &&
                         skinny_workspace_bytes(M, K, rows, dev.num_cu) > 0;
    const Plan p = plan(M, K, rows, dev.num_cu, have_ws);
    SkinnyArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.M = M;
    a.K = K;
    a.kgroups = p.kgroups;
    a.cpg = p.cpg;
    a.window = p.window;
    a.ngroups = ngroups;
    for (int i = 0; i < ngroups; ++i) a.g[i] = groups[i];
    if (p.kgroups > 1) {
        a.counters = static_cast<uint32_t*>(workspace);
        a.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    }
    if (p.u == 16) return launch_ksw<16>(p.ksw, a, stream);
    return launch_ksw<8>(p.ksw, a, stream);
}

}  // namespace nmi
