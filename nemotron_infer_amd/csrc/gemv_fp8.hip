// gemv_fp8.hip -- M = 1 fp8 (OCP e4m3) W8A16 GEMV for gfx950.
//
//   y[n] = bf16_rne( (sum_k float(W[n,k]) * float(x[k])) * s[n] )
//
// Same result contract as the reference's gemv_fp8_kernel
// (nemotron_infer/csrc/include/ops/gemv.cuh:48-89, formula :19-20, epilogue :87-88); the
// schedule is designed for CDNA4 and for HBM3E instead of a warp-per-row port:
//
// * A whole wave64 reads one weight row at a time: lane l takes the 16-byte chunks
//   l, l + 64, l + 128, ... of its K slice, so every load instruction fetches 1 KiB of
//   contiguous bytes (measured on MI355X: the fastest of the row-major access patterns).
//   A wave covers T rows (the same chunk columns of each), and KS waves of a workgroup
//   split K, so a workgroup of 4 waves covers (4 / KS) * T rows.
// * All of a lane's weight loads (T * P of them, P = chunks per row per lane) are issued
//   before any is consumed; the activation loads are issued first so that waiting for them
//   leaves the weight loads in flight.  The schedules are chosen so that P is 2-4: many
//   short-lived waves, every byte of W requested at kernel start.
// * x either staged per workgroup in LDS as raw bf16 (half-major: the low 8 elements of every
//   16-element chunk, then the high 8, so 64 lanes read 64 consecutive 16-byte words) or read
//   by each lane straight from global memory (its own chunks, reused for its T rows).
// * e4m3 -> bf16 pairs with v_cvt_scalef32_pk_bf16_fp8 (exact), v_dot2_f32_bf16 with float32
//   accumulation (bf16 x bf16 products are exact in float32), a wave reduction (DPP within
//   16-lane rows, then the four row sums in a fixed order), the KS K-slice partials summed in
//   a fixed order through LDS, the per-row scale and a single bf16 RNE rounding.
// * One launch may cover several matrices that share x and K (a group table in the kernel
//   arguments): q/k/v of an attention block, or the row slices of a Mamba in_proj.
// * Fused block ops: the RMSNorm that precedes every block's first linear can be applied while
//   x is staged (NORM: each workgroup reduces the row's sum of squares in the same fixed order
//   as the standalone kernel in rmsnorm.hip, so both give identical bf16 activations), and the
//   store can apply relu^2 or a residual add (epilogue() in nmi_device.hpp).
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kWaves = 4;
constexpr int kMaxWindowChunks = 1024;                  // bf16 x window: 1024 chunks * 32 B = 32 KiB
constexpr int kMaxXPieces = 2 * kMaxWindowChunks / 256; // 16-byte x pieces per thread per window

struct GemvArgs {
    const uint16_t* x;
    int64_t ldx;          // elements between activation rows (MR > 1)
    int M;                // activation rows (<= MR)
    int K;
    int window;           // chunks per LDS window
    int ngroups;
    const float* norm_w;  // NORM: RMSNorm weight [K]
    float eps;            // NORM: RMSNorm epsilon
    GemvGroup g[kMaxGroups];
};

// 16 e4m3 codes times 16 bf16 activations (low and high 8 of the chunk), two accumulators.
__device__ __forceinline__ void dot16(const uint4 w, const uint4 xl, const uint4 xh, float& a0,
                                      float& a1) {
    const uint2 p0 = e4m3x4_to_bf16(w.x), p1 = e4m3x4_to_bf16(w.y);
    const uint2 p2 = e4m3x4_to_bf16(w.z), p3 = e4m3x4_to_bf16(w.w);
    a0 = dot2_bf16(p0.x, xl.x, a0);
    a1 = dot2_bf16(p0.y, xl.y, a1);
    a0 = dot2_bf16(p1.x, xl.z, a0);
    a1 = dot2_bf16(p1.y, xl.w, a1);
    a0 = dot2_bf16(p2.x, xh.x, a0);
    a1 = dot2_bf16(p2.y, xh.y, a1);
    a0 = dot2_bf16(p3.x, xh.z, a0);
    a1 = dot2_bf16(p3.y, xh.w, a1);
}

// dot16 for MR activation rows: the codes are converted once.
template <int MR>
__device__ __forceinline__ void dot16_rows(const uint4 w, const uint4 (&xl)[MR], const uint4 (&xh)[MR],
                                           float (&a0)[MR], float (&a1)[MR]) {
    const uint2 p0 = e4m3x4_to_bf16(w.x), p1 = e4m3x4_to_bf16(w.y);
    const uint2 p2 = e4m3x4_to_bf16(w.z), p3 = e4m3x4_to_bf16(w.w);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        a0[m] = dot2_bf16(p0.x, xl[m].x, a0[m]);
        a1[m] = dot2_bf16(p0.y, xl[m].y, a1[m]);
        a0[m] = dot2_bf16(p1.x, xl[m].z, a0[m]);
        a1[m] = dot2_bf16(p1.y, xl[m].w, a1[m]);
        a0[m] = dot2_bf16(p2.x, xh[m].x, a0[m]);
        a1[m] = dot2_bf16(p2.y, xh[m].y, a1[m]);
        a0[m] = dot2_bf16(p3.x, xh[m].z, a0[m]);
        a1[m] = dot2_bf16(p3.y, xh[m].w, a1[m]);
    }
}

// KS: waves splitting K; T: rows per wave; P: 16-byte chunks per lane per row per batch;
// XG: x read from global memory instead of LDS; MR: activation rows computed together
// (M <= MR; rows >= M are zero and never stored -- the weight codes are converted once and
// reused for every activation row); XP: 16-byte x pieces per thread per window (LDS mode;
// 256 * XP >= 2 * window * MR); NORM: x is RMSNorm-ed while staged (one window covers K; the
// pieces are then [MR][XP / MR], piece (m, p) being the 8 activations at 8 * (tid + 256 p) of
// row m).
template <int KS, int T, int P, bool XG, int MR, int XP, bool NORM>
__global__ __launch_bounds__(256) void gemv_fp8_m1_kernel(const GemvArgs args) {
    static_assert(!NORM || (!XG && XP % MR == 0), "NORM stages x in LDS, XP / MR pieces per row");
    extern __shared__ uint4 xs[];                  // [m][half][window] (LDS mode)
    constexpr int kRowGroups = kWaves / KS;        // waves with distinct rows
    constexpr int kRowsPerWG = kRowGroups * T;
    constexpr int XPR = XP / MR;                   // NORM: pieces per thread per activation row
    __shared__ float partial[KS > 1 ? KS : 1][kRowsPerWG][MR];
    __shared__ float red[NORM ? kWaves : 1][MR];

    // Group of this workgroup (uniform scalar scan over <= kMaxGroups entries).
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < args.ngroups && (int)blockIdx.x >= args.g[i].wg_begin) gi = i;
    const GemvGroup grp = args.g[gi];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = wave / KS;                // row group (T rows) of this wave
    const int q = wave % KS;                // K slice of this wave
    const int row_base = ((int)blockIdx.x - grp.wg_begin) * kRowsPerWG + g * T;
    const uint16_t* __restrict__ x = args.x;
    const int C = args.K >> 4;              // 16-byte weight chunks per row
    const int window = XG ? C : args.window;

    // The epilogue operands of this lane (lane t * MR + m stores row row_base + t of activation
    // row m), loaded before everything else: they arrive with the weights instead of after them,
    // and the residual is read before any store (y may be the residual).
    const int st_t = lane / MR, st_m = lane % MR, st_row = row_base + st_t;
    const bool st_lane = lane < T * MR && st_row < grp.N && st_m < args.M && (KS == 1 || q == 0);
    float st_s = 0.f;
    uint16_t st_res = 0;
    if (st_lane) {
        st_s = grp.s[st_row];
        if (grp.epi.kind == kEpiResidual) st_res = grp.epi.res[(int64_t)st_m * grp.epi.ldres + st_row];
    }

    // Row t of this wave; rows past N read row N-1 (in bounds) and never store.
    const uint8_t* __restrict__ wrow[T];
#pragma unroll
    for (int t = 0; t < T; ++t)
        wrow[t] = grp.W + (int64_t)min(row_base + t, grp.N - 1) * grp.ldw;

    // Loads are unconditional, from addresses clamped into the valid range, so that no
    // branch separates them (a branch around a load makes the compiler wait for it); the
    // values of clamped slots are never consumed.
    float a0[T][MR], a1[T][MR];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) a0[t][m] = a1[t][m] = 0.f;
    for (int w0 = 0; w0 < C; w0 += window) {
        const int wc = min(window, C - w0);
        // 1. activations of this window (LDS mode; issued first), and the RMSNorm weights
        uint4 xr[XG ? 1 : XP];
        [[maybe_unused]] float4 gr[NORM ? 2 * XPR : 1];
        if constexpr (NORM) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int p = 0; p < XPR; ++p) {
                    const int ee = min(tid + 256 * p, 2 * wc - 1);
                    const int mm = m < args.M ? m : 0;      // rows >= M: never stored
                    xr[m * XPR + p] = load16(x + (int64_t)mm * args.ldx + (int64_t)ee * 8);
                }
#pragma unroll
            for (int p = 0; p < XPR; ++p) {
                const int ee = min(tid + 256 * p, 2 * wc - 1);
                gr[2 * p] = *reinterpret_cast<const float4*>(args.norm_w + ee * 8);
                gr[2 * p + 1] = *reinterpret_cast<const float4*>(args.norm_w + ee * 8 + 4);
            }
        } else if constexpr (!XG) {
#pragma unroll
            for (int p = 0; p < XP; ++p) {
                const int e = min(tid + 256 * p, 2 * wc * args.M - 1);
                const int mm = MR == 1 ? 0 : e / (2 * wc);
                const int ee = e - mm * 2 * wc;
                xr[p] = load16(x + (int64_t)mm * args.ldx + (int64_t)(w0 * 16 + ee * 8));
            }
        }
        // 2. this wave's K slice [cb, ce) of the window
        const int cb = w0 + (q * wc) / KS;
        const int ce = w0 + ((q + 1) * wc) / KS;
        const int clast = max(ce - 1, cb);
        int c0 = cb + lane;
        uint4 xl[XG ? P : 1], xh[XG ? P : 1];
        static_assert(!XG || MR == 1, "x from global memory is for one activation row");
        uint4 wv[T][P];
        if constexpr (XG) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int c = min(c0 + 64 * i, clast);
                xl[i] = load16(x + (int64_t)c * 16);
                xh[i] = load16(x + (int64_t)c * 16 + 8);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int i = 0; i < P; ++i)
                wv[t][i] = load_stream16(wrow[t] + (int64_t)min(c0 + 64 * i, clast) * 16);
        // 3. stage x (LDS mode) once the previous window has been consumed
        if constexpr (NORM) {
            // Sum of squares of each activation row: per thread over its pieces in order, then
            // the wave sum, then the four waves (0 + 1) + (2 + 3).
            float ss[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                ss[m] = 0.f;
#pragma unroll
                for (int p = 0; p < XPR; ++p)
                    if (tid + 256 * p < 2 * wc) ss[m] = sumsq8(xr[m * XPR + p], ss[m]);
                ss[m] = wave_sum(ss[m]);
            }
            if (lane == 0) {
#pragma unroll
                for (int m = 0; m < MR; ++m) red[wave][m] = ss[m];
            }
            __syncthreads();
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float r = rms_factor((red[0][m] + red[1][m]) + (red[2][m] + red[3][m]), args.K, args.eps);
#pragma unroll
                for (int p = 0; p < XPR; ++p) {
                    const int ee = tid + 256 * p;
                    if (ee < 2 * wc && m < args.M)
                        xs[(m * 2 + (ee & 1)) * window + (ee >> 1)] =
                            rms_scale8(xr[m * XPR + p], gr[2 * p], gr[2 * p + 1], r);
                }
            }
            __syncthreads();
        } else if constexpr (!XG) {
            if (w0 != 0) __syncthreads();
#pragma unroll
            for (int p = 0; p < XP; ++p) {
                const int e = tid + 256 * p;
                if (e < 2 * wc * args.M) {
                    const int mm = MR == 1 ? 0 : e / (2 * wc);
                    const int ee = e - mm * 2 * wc;
                    xs[(mm * 2 + (ee & 1)) * window + (ee >> 1)] = xr[p];
                }
            }
            __syncthreads();
        }
        // 4. consume; further batches only when a lane's slice exceeds P chunks per row
        for (;;) {
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int c = c0 + 64 * i;
                if (c < ce) {
                    if constexpr (XG) {
#pragma unroll
                        for (int t = 0; t < T; ++t) dot16(wv[t][i], xl[i], xh[i], a0[t][0], a1[t][0]);
                    } else if constexpr (MR == 1) {
                        const uint4 lo = xs[c - w0], hi = xs[window + c - w0];
#pragma unroll
                        for (int t = 0; t < T; ++t) dot16(wv[t][i], lo, hi, a0[t][0], a1[t][0]);
                    } else {
                        uint4 lo[MR], hi[MR];
#pragma unroll
                        for (int m = 0; m < MR; ++m) {
                            const int mm = m < args.M ? m : 0;       // rows >= M: never stored
                            lo[m] = xs[(2 * mm) * window + c - w0];
                            hi[m] = xs[(2 * mm + 1) * window + c - w0];
                        }
#pragma unroll
                        for (int t = 0; t < T; ++t) dot16_rows<MR>(wv[t][i], lo, hi, a0[t], a1[t]);
                    }
                }
            }
            c0 += 64 * P;
            if (c0 - lane >= ce) break;         // uniform across the wave
            if constexpr (XG) {
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    const int c = min(c0 + 64 * i, clast);
                    xl[i] = load16(x + (int64_t)c * 16);
                    xh[i] = load16(x + (int64_t)c * 16 + 8);
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int i = 0; i < P; ++i)
                    wv[t][i] = load_stream16(wrow[t] + (int64_t)min(c0 + 64 * i, clast) * 16);
        }
    }

    // Wave sums in a fixed order: 16-lane DPP rows, then rows 0 + 1 + 2 + 3.
    float sums[T][MR];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) sums[t][m] = wave_sum(a0[t][m] + a1[t][m]);
    if constexpr (KS > 1) {
        if (lane == 0) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int m = 0; m < MR; ++m) partial[q][g * T + t][m] = sums[t][m];
        }
        __syncthreads();
        if (q != 0) return;
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float v = partial[0][g * T + t][m];
#pragma unroll
                for (int qq = 1; qq < KS; ++qq) v += partial[qq][g * T + t][m];
                sums[t][m] = v;
            }
    }
    // Lane t * MR + m stores row row_base + t of activation row m.
    if (lane < T * MR) {
        float v = 0.f;
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (lane == t * MR + m) v = sums[t][m];
        if (st_lane) grp.y[(int64_t)st_m * grp.ldy + st_row] = epilogue(v, st_s, grp.epi.kind, st_res);
    }
}

template <int KS, int T, int P, bool XG, int MR, int XP, bool NORM>
hipError_t launch_cfg(GemvArgs& a, hipStream_t stream) {
    constexpr int rows_per_wg = (kWaves / KS) * T;
    int wgs = 0;
    for (int i = 0; i < a.ngroups; ++i) {
        a.g[i].wg_begin = wgs;
        wgs += (a.g[i].N + rows_per_wg - 1) / rows_per_wg;
    }
    const size_t lds = XG ? 0 : (size_t)a.window * 2 * MR * sizeof(uint4);
    hipLaunchKernelGGL((gemv_fp8_m1_kernel<KS, T, P, XG, MR, XP, NORM>), dim3(wgs), dim3(256), lds, stream, a);
    return hipGetLastError();
}

// x staging mode: from global memory (M = 1), LDS with XP pieces per thread, or LDS with the
// RMSNorm applied (M <= 2).
struct Mode {
    bool xg;
    bool norm;
    int mr;
    int xp;
};

template <int KS, int T, int P>
hipError_t launch_mode(const Mode& md, GemvArgs& a, hipStream_t stream) {
    if (md.xg) return launch_cfg<KS, T, P, true, 1, 1, false>(a, stream);
    if (md.norm) {
        if (md.mr == 1) {
            switch (md.xp) {
                case 2: return launch_cfg<KS, T, P, false, 1, 2, true>(a, stream);
                case 4: return launch_cfg<KS, T, P, false, 1, 4, true>(a, stream);
                default: return launch_cfg<KS, T, P, false, 1, 8, true>(a, stream);
            }
        }
        return md.xp <= 4 ? launch_cfg<KS, T, P, false, 2, 4, true>(a, stream)
                          : launch_cfg<KS, T, P, false, 2, 8, true>(a, stream);
    }
    if (md.mr == 1) {
        switch (md.xp) {
            case 2: return launch_cfg<KS, T, P, false, 1, 2, false>(a, stream);
            case 4: return launch_cfg<KS, T, P, false, 1, 4, false>(a, stream);
            default: return launch_cfg<KS, T, P, false, 1, 8, false>(a, stream);
        }
    }
    if (md.mr == 2) {
        return md.xp <= 4 ? launch_cfg<KS, T, P, false, 2, 4, false>(a, stream)
                          : launch_cfg<KS, T, P, false, 2, 8, false>(a, stream);
    }
    return launch_cfg<KS, T, P, false, 4, 8, false>(a, stream);
}

template <int KS, int T>
hipError_t launch_p(int p, const Mode& md, GemvArgs& a, hipStream_t stream) {
    switch (p) {
        case 2: return launch_mode<KS, T, 2>(md, a, stream);
        case 3: return launch_mode<KS, T, 3>(md, a, stream);
        default: return launch_mode<KS, T, 4>(md, a, stream);
    }
}

template <int KS>
hipError_t launch_t(int t, int p, const Mode& md, GemvArgs& a, hipStream_t stream) {
    switch (t) {
        case 1: return launch_p<KS, 1>(p, md, a, stream);
        case 2: return launch_p<KS, 2>(p, md, a, stream);
        default: return launch_p<KS, 4>(p, md, a, stream);
    }
}

int pow2_pieces(int need) { return need <= 2 ? 2 : (need <= 4 ? 4 : 8); }

// ---------------------------------------------------------------------------------------
// GEMV chain: the GEMVs of a decode step (phases, each a grouped GEMV sharing one x) in one
// launch.  Work items (T * 4 / ks rows of one group each) are numbered in phase order; the grid
// is at most the number of workgroups that fit on the device at once, and workgroup b takes
// items b, b + G, b + 2G, ... in order.  An item of a waiting phase issues its first weight
// loads, then waits until the previous phase has completed (its x may be that phase's output),
// then stages x and finishes its rows.  The weight stream of the next phase therefore starts
// while the current one drains, and the step pays one launch.  Deadlock-free when all G
// workgroups are resident together (G is sized so): the lowest unfinished item belongs to a
// running workgroup whose earlier items are done, and it waits only on lower items.
//
// Completion is counted only for phases that a later phase waits on, and without one contended
// address (device-scope atomics on one cache line serialize at a few ns each): such an item,
// once its stores have completed (s_waitcnt), adds 1 to stripe (local index % kChainStripes) of
// its phase, each stripe on its own 128-byte line; the item completing a stripe adds 1 to the
// phase's done line, which the waiters poll.  Other items store and go on.  Every workgroup
// leaving the loop adds 1 to its exit stripe (blockIdx % kChainStripes), the one completing a
// stripe to the exit-done line, and the one completing that re-arms every line: the counters
// are zero again when the launch ends.  A wait that has not ended after 0.2 s (tuning knob
// chain.wait_us) gives up (wrong outputs, never a hang) and sets the error word, which is left
// set.  Outputs of a signalling
// phase are stored, and x of a waiting phase is loaded, at device scope (coherent across the
// XCDs' L2 caches).
__device__ __forceinline__ uint32_t* chain_line(uint32_t* ctr, int p, int line) {
    return ctr + ((int64_t)p * (kChainStripes + 1) + line) * kChainLineWords;
}

// Pointers read from the phase table carry no address space; the chain kernel converts them to
// global-memory pointers so that its loads and stores are global (not FLAT) instructions.
#define NMI_GLOBAL __attribute__((address_space(1)))
template <class E>
__device__ __forceinline__ NMI_GLOBAL E* global_ptr(E* p) {
    return (NMI_GLOBAL E*)p;
}

__device__ __forceinline__ uint4 load_stream16_g(const NMI_GLOBAL uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const NMI_GLOBAL u32x4*>(p));
    return uint4{v.x, v.y, v.z, v.w};
}

// The phase table is written before the launch and never by a kernel: read through the constant
// address space, its uniform fields are scalar loads (as generic memory, next to the kernel's
// own stores, the compiler would read it with vector loads and wait for them together with the
// weight loads in flight).
#define NMI_CONST __attribute__((address_space(4)))

__device__ __forceinline__ int chain_stripes(int nitems) { return nitems < kChainStripes ? nitems : kChainStripes; }

template <int T, int P>
__global__ __launch_bounds__(256) void gemv_chain_kernel(const ChainItem* __restrict__ items, int nphases,
                                                          int total_items, uint32_t* __restrict__ ctr,
                                                          uint64_t wait_ticks) {
    typedef __attribute__((address_space(3))) void lds_void;
    extern __shared__ uint4 xs[];                  // [half][window rounded up to 64 chunks]
    __shared__ float partial[kWaves][kWaves * T];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const uint32_t xs_addr = (uint32_t)(uintptr_t)(lds_void*)xs;
    uint32_t* err = ctr + (int64_t)(gemv_chain_counter_lines(nphases) - 1) * kChainLineWords;
    const NMI_CONST ChainItem* tab = (const NMI_CONST ChainItem*)items;
    for (int item = blockIdx.x; item < total_items; item += gridDim.x) {
        const NMI_CONST ChainItem& it = tab[item];
        const int ks = it.ks;                      // waves splitting K: 1, 2 or 4
        const int g = wave / ks, q = wave % ks;
        const int row0 = g * T;                    // this wave's first row within the item
        const int rows = it.rows;
        const int64_t ldw = it.ldw;
        const int C = it.K >> 4, window = it.window;
        const int wpad = (window + 63) & ~63;      // LDS chunks per half
        const bool wait = it.flags & kChainWait, signal = it.flags & kChainSignal;
        const NMI_GLOBAL uint8_t* gW = global_ptr(it.w);

        // this lane's row scale (lane t < T of a K-slice-0 wave), issued before the weights so that
        // it has arrived with them
        float sc = 0.f;
        if (q == 0 && lane < T && row0 + lane < rows) sc = global_ptr(it.s)[row0 + lane];
        const NMI_GLOBAL uint8_t* wrow[T];
#pragma unroll
        for (int t = 0; t < T; ++t) wrow[t] = gW + (int64_t)min(row0 + t, rows - 1) * ldw;
        float a0[T], a1[T];
#pragma unroll
        for (int t = 0; t < T; ++t) a0[t] = a1[t] = 0.f;
        for (int w0 = 0; w0 < C; w0 += window) {
            const int wc = min(window, C - w0);
            const int cb = w0 + (q * wc) / ks;
            const int ce = w0 + ((q + 1) * wc) / ks;
            const int clast = max(ce - 1, cb);
            int c0 = cb + lane;
            // 1. this window's first batch of weights (independent of earlier phases)
            uint4 wv[T][P];
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int i = 0; i < P; ++i)
                    wv[t][i] = load_stream16_g(wrow[t] + (int64_t)min(c0 + 64 * i, clast) * 16);
            // 2. x may be the previous phase's output: wait for that phase (first window only)
            if (w0 == 0 && wait) {
                if (tid == 0) {
                    const uint32_t need = (uint32_t)it.wait_need;
                    const uint32_t* done = chain_line(ctr, it.phase - 1, kChainStripes);
                    const uint64_t t_end = wall_clock64() + wait_ticks;   // wall clock: 100 MHz
                    while (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
                        if ((uint64_t)wall_clock64() > t_end) {
                            __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(2);
                    }
                }
                __syncthreads();
            } else if (w0 != 0) {
                __syncthreads();                   // the previous window has been consumed
            }
            // 3. stage x by LDS DMA (two 16-byte halves per chunk, as the one-launch kernel): job
            //    (half h, 64-chunk block b) has lane l load piece 2 (64 b + l) + h; lanes past the
            //    window load a valid piece into an unread pad slot of the block
            const uint8_t* xw = reinterpret_cast<const uint8_t*>(it.x) + (int64_t)w0 * 32;
            const int jobs = 2 * ((wc + 63) >> 6);
            for (int j = wave; j < jobs; j += kWaves) {
                const int h = j & 1, s0 = (j >> 1) << 6;
                const uint32_t off = (uint32_t)min(2 * (s0 + lane) + h, 2 * wc - 1) * 16;
                const uint32_t dst = xs_addr + (uint32_t)(h * wpad + s0) * 16;
                if (wait) dma16_lds_device(xw, off, dst);
                else dma16_lds(xw, off, dst);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            // 4. consume; further batches when a lane's slice exceeds P chunks per row
            for (;;) {
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    const int c = c0 + 64 * i;
                    if (c < ce) {
                        const uint4 lo4 = xs[c - w0], hi4 = xs[wpad + c - w0];
#pragma unroll
                        for (int t = 0; t < T; ++t) dot16(wv[t][i], lo4, hi4, a0[t], a1[t]);
                    }
                }
                c0 += 64 * P;
                if (c0 - lane >= ce) break;         // uniform across the wave
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int i = 0; i < P; ++i)
                        wv[t][i] = load_stream16_g(wrow[t] + (int64_t)min(c0 + 64 * i, clast) * 16);
            }
        }
        // wave sums (16-lane DPP rows, then 0 + 1 + 2 + 3), then the K slices in order q = 0..ks-1
        float sums[T];
#pragma unroll
        for (int t = 0; t < T; ++t) sums[t] = wave_sum(a0[t] + a1[t]);
        if (lane == 0) {
#pragma unroll
            for (int t = 0; t < T; ++t) partial[q][g * T + t] = sums[t];
        }
        __syncthreads();                           // also: every wave is done reading xs
        if (q == 0 && lane < T) {
            const int t = lane;
            float v = partial[0][g * T + t];
            for (int qq = 1; qq < ks; ++qq) v += partial[qq][g * T + t];
            const int row = row0 + t;
            if (row < rows) {
                // plain epilogue: a chain group has no fused relu^2 or residual
                const uint16_t out = epilogue(v, sc, kEpiNone, 0);
                NMI_GLOBAL uint16_t* yp = global_ptr(it.y) + row;
                if (signal) __hip_atomic_store(yp, out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else *yp = out;
            }
        }
        // completion (counted when a later phase waits on this one): the stores have completed,
        // then the count
        if (signal) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0) {
                const uint32_t v = __hip_atomic_fetch_add(chain_line(ctr, it.phase, it.stripe), 1u, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT);
                if (v + 1 == (uint32_t)it.stripe_items)
                    __hip_atomic_fetch_add(chain_line(ctr, it.phase, kChainStripes), 1u, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    // exit count, after this workgroup's own counts have landed; the last workgroup out re-arms
    // the counters (nothing reads them any more)
    if (wave == 0) {
        __builtin_amdgcn_s_waitcnt(0);
        int rearm = 0;
        if (lane == 0) {
            const int G = (int)gridDim.x;
            const int stripe = (int)blockIdx.x % kChainStripes;
            const uint32_t v = __hip_atomic_fetch_add(chain_line(ctr, nphases, stripe), 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
            if (v + 1 == (uint32_t)((G - stripe + kChainStripes - 1) / kChainStripes)) {
                const uint32_t d = __hip_atomic_fetch_add(chain_line(ctr, nphases, kChainStripes), 1u,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                rearm = d + 1 == (uint32_t)chain_stripes(G);
            }
        }
        if (__builtin_amdgcn_readfirstlane(rearm)) {
            const int lines = (nphases + 1) * (kChainStripes + 1);
            for (int l = lane; l < lines; l += 64)
                __hip_atomic_store(ctr + (int64_t)l * kChainLineWords, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace

bool gemv_norm_supported(int M, int K) {
    const int C = K >> 4;
    return (M == 1 || M == 2) && 2 * C <= 256 * (8 / M);
}

hipError_t launch_gemv_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                               int ngroups, hipStream_t stream, const Norm& norm) {
    const DeviceInfo& dev = device_info();
    if (norm.w && !gemv_norm_supported(M, K)) return hipErrorInvalidValue;
    GemvArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.M = M;
    a.K = K;
    a.norm_w = norm.w;
    a.eps = norm.eps;
    const int C = K >> 4;
    const int mr = M == 1 ? 1 : (M == 2 ? 2 : 4);
    const int wmax = kMaxWindowChunks / mr;        // 2 * mr * window pieces <= 8 per thread
    a.window = C < wmax ? C : wmax;
    a.ngroups = ngroups;
    static_assert(2 * kMaxWindowChunks <= 256 * kMaxXPieces, "window larger than the staging pieces");
    int64_t rows = 0;
    for (int i = 0; i < ngroups; ++i) {
        a.g[i] = groups[i];
        rows += groups[i].N;
    }
    const Tuning& tn = tuning();
    // K split: about 3-4 chunks per lane per row (KS waves of 64 lanes cover a row).
    int ks = C <= 64 * 4 ? 1 : (C <= 2 * 64 * 4 ? 2 : 4);
    if (tn.gemv_ks == 1 || tn.gemv_ks == 2 || tn.gemv_ks == 4) ks = tn.gemv_ks;
    const int slice = (C + ks - 1) / ks;
    int p = (slice + 63) / 64;
    p = p <= 2 ? 2 : (p <= 3 ? 3 : 4);
    if (tn.gemv_p >= 2 && tn.gemv_p <= 4) p = tn.gemv_p;
    // Rows per wave: as many as keep about three workgroups per CU.
    int t = 1;
    for (int cand : {4, 2}) {
        const int64_t wgs = (rows + (int64_t)(kWaves / ks) * cand - 1) / ((int64_t)(kWaves / ks) * cand);
        if (wgs >= 3 * (int64_t)dev.num_cu) { t = cand; break; }
    }
    if (tn.gemv_t == 1 || tn.gemv_t == 2 || tn.gemv_t == 4) t = tn.gemv_t;
    Mode md{};
    md.norm = norm.w != nullptr;
    md.xg = !md.norm && tn.gemv_xg == 1 && M == 1;
    md.mr = mr;
    md.xp = md.norm ? mr * pow2_pieces((2 * C + 255) / 256) : pow2_pieces((2 * a.window * mr + 255) / 256);
    switch (ks) {
        case 1: return launch_t<1>(t, p, md, a, stream);
        case 2: return launch_t<2>(t, p, md, a, stream);
        default: return launch_t<4>(t, p, md, a, stream);
    }
}

namespace {
constexpr int kChainT = 4;       // rows per wave in the chain kernel
constexpr int kChainP = 4;       // 16-byte chunks per lane per row per batch
}  // namespace

int gemv_chain_plan(ChainPhase* phases, int nphases, size_t* lds_bytes) {
    int items = 0;
    int wmax = 1;
    for (int p = 0; p < nphases; ++p) {
        ChainPhase& ph = phases[p];
        const int C = ph.K >> 4;
        ph.ks = C <= 64 * 4 ? 1 : (C <= 2 * 64 * 4 ? 2 : 4);   // about 3-4 chunks per lane per row
        ph.window = C < kMaxWindowChunks ? C : kMaxWindowChunks;
        wmax = ph.window > wmax ? ph.window : wmax;
        const int rows_per_wg = (kWaves / ph.ks) * kChainT;
        ph.item_begin = items;
        int n = 0;
        for (int i = 0; i < ph.ngroups; ++i) {
            ph.g[i].wg_begin = n;
            n += (ph.g[i].N + rows_per_wg - 1) / rows_per_wg;
        }
        ph.nitems = n;
        items += n;
    }
    for (int p = 0; p < nphases; ++p) phases[p].signal = p + 1 < nphases && phases[p + 1].wait;
    *lds_bytes = (size_t)((wmax + 63) & ~63) * 2 * sizeof(uint4);
    return items;
}

void gemv_chain_items(const ChainPhase* planned, int nphases, ChainItem* out) {
    int k = 0;
    for (int p = 0; p < nphases; ++p) {
        const ChainPhase& ph = planned[p];
        const int rows_per_item = (kWaves / ph.ks) * kChainT;
        int local = 0;
        for (int gi = 0; gi < ph.ngroups; ++gi) {
            const GemvGroup& grp = ph.g[gi];
            for (int r0 = 0; r0 < grp.N; r0 += rows_per_item, ++local, ++k) {
                ChainItem& it = out[k];
                it.w = grp.W + (int64_t)r0 * grp.ldw;
                it.x = ph.x;
                it.y = grp.y + r0;
                it.s = grp.s + r0;
                it.ldw = grp.ldw;
                it.rows = grp.N - r0 < rows_per_item ? grp.N - r0 : rows_per_item;
                it.K = ph.K;
                it.ks = ph.ks;
                it.window = ph.window;
                it.phase = p;
                it.flags = (p > 0 && ph.wait ? kChainWait : 0) | (ph.signal ? kChainSignal : 0);
                it.wait_need = p > 0 ? (planned[p - 1].nitems < kChainStripes ? planned[p - 1].nitems : kChainStripes) : 0;
                it.stripe = local % kChainStripes;
                it.stripe_items = (ph.nitems - it.stripe + kChainStripes - 1) / kChainStripes;
            }
        }
    }
}

hipError_t gemv_chain_grid(size_t lds_bytes, int total_items, int* grid) {
    const DeviceInfo& dev = device_info();
    int per_cu = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, gemv_chain_kernel<kChainT, kChainP>, 256, lds_bytes);
    if (e != hipSuccess) return e;
    // Measured on the config-1 set: 4 workgroups per CU stream faster than the 5 that fit.
    const int cap = tuning().chain_wgs >= 1 ? tuning().chain_wgs : 4;
    if (cap < per_cu) per_cu = cap;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    const int64_t resident = (int64_t)per_cu * dev.num_cu;
    *grid = (int)(total_items < resident ? total_items : resident);
    return hipSuccess;
}

hipError_t launch_gemv_chain(const ChainItem* items, int nphases, int total_items, int grid, size_t lds_bytes,
                             uint32_t* ctr, hipStream_t stream) {
    // the bound of a wait: 0.2 s, or tuning knob chain.wait_us (microseconds) when set
    const uint64_t wait_ticks = tuning().chain_wait_us > 0 ? (uint64_t)tuning().chain_wait_us * 100u : 20000000ull;
    hipLaunchKernelGGL((gemv_chain_kernel<kChainT, kChainP>), dim3(grid), dim3(256), lds_bytes, stream,
                       items, nphases, total_items, ctr, wait_ticks);
    return hipGetLastError();
}

hipError_t launch_gemv_m1_grouped(const uint16_t* x, int K, const GemvGroup* groups, int ngroups,
                                  hipStream_t stream) {
    return launch_gemv_grouped(x, K, 1, K, groups, ngroups, stream, Norm{});
}

hipError_t launch_gemv_m1(const uint16_t* x, const uint8_t* W, int64_t ldw, const float* s,
                          uint16_t* y, int N, int K, hipStream_t stream) {
    GemvGroup g{W, ldw, s, y, N, N, 0, 0, Epi{}};
    return launch_gemv_m1_grouped(x, K, &g, 1, stream);
}

}  // namespace nmi
