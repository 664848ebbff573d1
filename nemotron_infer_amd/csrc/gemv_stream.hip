// gemv_stream.hip -- M = 1 fp8 (OCP e4m3) W8A16 GEMV for gfx950 as a per-wave weight stream.
//
//   y[n] = bf16_rne( (sum_k float(W[n,k]) * float(x[k])) * s[n] )
//
// Same result contract as the reference's gemv_fp8_kernel (nemotron_infer/csrc/include/
// ops/gemv.cuh:48-89, formula :19-20, epilogue :87-88).  The schedule is built for HBM3E:
//
// * Work is a list of phases (one GEMV, or the GEMVs of a decode step), each phase a grouped
//   GEMV of one x against up to four matrices.  Rows are taken T = 2 at a time ("row groups"),
//   numbered across the whole list; wave w of the grid (NW waves) takes row groups w, w + NW,
//   w + 2 NW, ...  Concurrent waves therefore read neighbouring rows: the front of in-flight
//   reads stays compact.
// * Every wave streams on its own: no workgroup barrier after the start.  A row group is
//   walked in K slices of at most 256 16-byte chunks; one "step" is T rows x one slice, i.e.
//   4 loads of 16 bytes per row and lane (lane l takes chunks l, l + 64, l + 128, l + 192 of the
//   slice, so each load instruction reads 1 KiB of a row).  Steps are double-buffered in
//   registers: the loads of step i + 1 are issued before step i is computed, so a wave always
//   has one step in flight while it computes the other (measured: the plain streaming read of
//   the same bytes is not faster).
// * x comes from LDS (single launches: the workgroup stages the whole vector once, optionally
//   applying the block's RMSNorm while doing so) or, per step, from global memory next to the
//   weights (chains: x changes with the phase, and every phase's x is an L2-resident vector).
//   The arithmetic is the same in both modes, so a chain's outputs equal the single launches'
//   bit for bit.
// * e4m3 -> bf16 pairs with v_cvt_scalef32_pk_bf16_fp8 (exact), v_dot2_f32_bf16 with float32
//   accumulation in a fixed order (per lane: slice by slice, chunk by chunk; then the wave sum,
//   16-lane DPP rows and (r0 + r1) + (r2 + r3)), the per-row scale and one bf16 RNE rounding,
//   with the optional relu^2 / residual epilogue.  Deterministic.
// * Stores are raw buffer stores whose descriptor covers exactly the step's valid output rows
//   (none for a step that is not the last slice of its rows): out-of-range lanes are dropped by
//   the hardware, so the loop body has no branch around a memory instruction and the loads of
//   the next step stay in flight across it.
// * A chain whose phase p + 1 reads the output of phase p (wait_prev) is launched as one kernel
//   per run of phases up to the next waiting phase: the stream orders the launches, so the
//   ordering needs no in-kernel synchronisation.  (Measured on MI355X: a device-scope
//   release/acquire between workgroups compiles to cache-wide L2 write-back / invalidate
//   instructions, one per workgroup, and cost about 50 us per phase boundary; a kernel boundary
//   costs about 3 us.)
#include "nmi_device.hpp"
#include "nmi_launch.hpp"

namespace nmi {

namespace {

constexpr int kWaves = 4;              // waves per workgroup
constexpr int kLoads = 4;              // 16-byte loads per row and lane in one step

#define NMI_CONST __attribute__((address_space(4)))

typedef __attribute__((address_space(3))) void lds_void;

// 16 e4m3 codes -> 16 bf16 in four packed pairs of pairs.
struct Codes16 {
    uint2 p0, p1, p2, p3;
};
__device__ __forceinline__ Codes16 conv16(const uint4 w) {
    return Codes16{e4m3x4_to_bf16(w.x), e4m3x4_to_bf16(w.y), e4m3x4_to_bf16(w.z), e4m3x4_to_bf16(w.w)};
}

// 16 converted codes times 16 bf16 activations (low and high 8 of the chunk), two accumulators.
__device__ __forceinline__ void dot16s(const Codes16& c, const uint4 xl, const uint4 xh, float& a0, float& a1) {
    const uint2 p0 = c.p0, p1 = c.p1, p2 = c.p2, p3 = c.p3;
    a0 = dot2_bf16(p0.x, xl.x, a0);
    a1 = dot2_bf16(p0.y, xl.y, a1);
    a0 = dot2_bf16(p1.x, xl.z, a0);
    a1 = dot2_bf16(p1.y, xl.w, a1);
    a0 = dot2_bf16(p2.x, xh.x, a0);
    a1 = dot2_bf16(p2.y, xh.y, a1);
    a0 = dot2_bf16(p3.x, xh.z, a0);
    a1 = dot2_bf16(p3.y, xh.w, a1);
}

// Where a wave is in the work list, with the step's operands cached (every field wave-uniform,
// held in scalar registers: the phase table is read only when the wave enters a row group).
struct Cursor {
    int valid;
    int p;                  // phase
    int g;                  // global row group
    int j;                  // slice within the row group
    int S, sw, C;           // the phase's slices, chunks per slice, chunks
    int rows;               // rows of the row group that exist (1..T)
    int epi;
    int ldy, ldres;         // output / residual row strides (activation rows)
    int M;                  // activation rows (single launches)
    const uint8_t* w0;      // first weight row of the row group
    int64_t ldw;
    const float* s0;        // its scale
    uint16_t* y0;           // its output
    const uint16_t* r0;     // its residual
    const uint16_t* x;      // the phase's activations
};

// One step's operands, loaded one step ahead.
template <int T, bool XG>
struct Buf {
    uint4 w[T][kLoads];
    uint4 x[XG ? kLoads : 1][2];
    float sc;
    uint32_t res;
};

template <bool CHAIN>
__device__ __forceinline__ const NMI_CONST StreamPhase& phase_at(const StreamArgs& a,
                                                                  const NMI_CONST StreamPhase* tab, int p) {
    if constexpr (CHAIN) return tab[p];
    else return *(const NMI_CONST StreamPhase*)&a.one;
}

// Enter row group c.g (< total_rg): find its phase (at or after c.p) and group, cache the
// operands.
template <int T, bool CHAIN>
__device__ __forceinline__ void locate(const StreamArgs& a, const NMI_CONST StreamPhase* tab, Cursor& c) {
    if constexpr (CHAIN) {
        while (c.g >= tab[c.p].g_end) ++c.p;
    }
    const NMI_CONST StreamPhase& ph = phase_at<CHAIN>(a, tab, c.p);
    const int r = c.g - ph.g_begin;
    int gi = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < ph.ngroups && r >= ph.g[i].rg_begin) gi = i;
    const NMI_CONST StreamGroup& gr = ph.g[gi];
    const int row0 = (r - gr.rg_begin) * T;
    c.j = 0;
    c.S = ph.S;
    c.sw = ph.sw;
    c.C = ph.C;
    c.rows = min(T, gr.N - row0);
    c.epi = gr.epi;
    c.ldy = gr.ldy;
    c.ldres = gr.ldres;
    c.M = CHAIN ? 1 : a.M;
    c.ldw = gr.ldw;
    c.w0 = gr.W + (int64_t)row0 * gr.ldw;
    c.s0 = gr.s + row0;
    c.y0 = gr.y + row0;
    c.r0 = gr.res + row0;
    c.x = ph.x;
}

template <int T, bool CHAIN>
__device__ __forceinline__ Cursor cursor_start(const StreamArgs& a, const NMI_CONST StreamPhase* tab, int gw) {
    Cursor c{};
    c.p = 0;
    c.g = gw < a.total_rg ? gw : a.total_rg - 1;
    locate<T, CHAIN>(a, tab, c);
    c.valid = gw < a.total_rg;
    return c;
}

// The step after c; past the wave's last step the cursor becomes invalid and keeps c's operands
// (an invalid step's loads all read one chunk of c's first row: a "null" step).
template <int T, bool CHAIN>
__device__ __forceinline__ Cursor cursor_next(const StreamArgs& a, const NMI_CONST StreamPhase* tab, Cursor c,
                                              int nw) {
    if (c.j + 1 < c.S) {
        ++c.j;
        return c;
    }
    if (c.g + nw >= a.total_rg) {
        c.valid = 0;
        c.j = 0;
        return c;
    }
    c.g += nw;
    locate<T, CHAIN>(a, tab, c);
    return c;
}

// Issue the weight, scale and residual loads of step c into b (lane t < T: row t's scale and
// residual).  Every address is clamped into the valid range (rows past the group's end read its
// last row, chunks past the slice its last chunk), so the loads are unconditional; a null step
// reads chunk 0 of its rows from every lane.
template <int T, bool RES, bool XG, int MR>
__device__ __forceinline__ void issue_w(const Cursor& c, int lane, Buf<T, XG>& b) {
    const int cb = c.valid ? c.j * c.sw : 0;                       // first chunk of the slice
    const int clast = c.valid ? min(cb + c.sw, c.C) - 1 : 0;       // last chunk of the slice
    const int l = c.valid ? lane : 0;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const uint8_t* wr = c.w0 + (int64_t)min(t, c.rows - 1) * c.ldw;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) b.w[t][i] = load_stream16(wr + (int64_t)min(cb + l + 64 * i, clast) * 16);
    }
    // lane t MR + m: output row t of activation row m
    const int lt = lane < T * MR ? lane : 0;
    const int tr = min(lt / MR, c.rows - 1);
    b.sc = c.s0[tr];
    if constexpr (RES) b.res = c.r0[(int64_t)min(lt % MR, c.M - 1) * c.ldres + tr];
    __builtin_amdgcn_sched_barrier(0);
}

// Issue the x loads of step c (XG mode): lane l's chunks of the slice, lo and hi halves.  A
// phase that waits reads its x after an agent-scope acquire, so plain loads see the previous
// phase's stores.
template <int T>
__device__ __forceinline__ void issue_x(const Cursor& c, int lane, Buf<T, true>& b) {
    const int cb = c.valid ? c.j * c.sw : 0;
    const int clast = c.valid ? min(cb + c.sw, c.C) - 1 : 0;
    const int l = c.valid ? lane : 0;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)c.x, 0, c.C * 32, 0x00020000);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int off = min(cb + l + 64 * i, clast) * 32;
        b.x[i][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        b.x[i][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, off + 16, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);
}

// Compute step c from b into the running sums; on the last slice of the row group reduce, apply
// the scale and the epilogue, and store (lane t < rows stores row t).  A null step computes
// nothing it keeps and stores nothing.
template <int T, bool XG, bool RES, int MR>
__device__ __forceinline__ void compute(const Cursor& c, int lane, const Buf<T, XG>& b, const uint4* xs, int xs_half,
                                        float (&a0)[T][MR], float (&a1)[T][MR]) {
    static_assert(!XG || MR == 1, "x from global memory is for one activation row");
    const int cb = c.j * c.sw;
    const int nvalid = min(c.sw, c.C - cb);
    const bool first = c.j == 0, last = c.valid && c.j == c.S - 1;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            a0[t][m] = first ? 0.f : a0[t][m];
            a1[t][m] = first ? 0.f : a1[t][m];
        }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int c_in = lane + 64 * i;
        const bool ok = c_in < nvalid;
        uint4 lo[MR], hi[MR];
        if constexpr (XG) {
            lo[0] = b.x[i][0];
            hi[0] = b.x[i][1];
        } else {
            const int cc = cb + min(c_in, nvalid - 1);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                lo[m] = xs[2 * m * xs_half + cc];
                hi[m] = xs[(2 * m + 1) * xs_half + cc];
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            if constexpr (MR == 1) {
                // converted inside the dot product: the form the one-row kernels were tuned with
                float b0 = a0[t][0], b1 = a1[t][0];
                dot16s(conv16(b.w[t][i]), lo[0], hi[0], b0, b1);
                a0[t][0] = ok ? b0 : a0[t][0];
                a1[t][0] = ok ? b1 : a1[t][0];
            } else {
                const Codes16 cw = conv16(b.w[t][i]);          // converted once for both rows
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float b0 = a0[t][m], b1 = a1[t][m];
                    dot16s(cw, lo[m], hi[m], b0, b1);
                    a0[t][m] = ok ? b0 : a0[t][m];
                    a1[t][m] = ok ? b1 : a1[t][m];
                }
            }
        }
    }
    float v = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float sum = wave_sum(a0[t][m] + a1[t][m]);
            v = lane == t * MR + m ? sum : v;
        }
    // epilogue() of nmi_device.hpp, on the raw 32-bit residual load: the shift drops its upper
    // half, so no zero-extension of a register of the step in flight is ever needed here
    const uint16_t lin = f32_to_bf16_rne(v * b.sc);
    uint16_t out = lin;
    if (c.epi == kEpiRelu2) {
        float f = bf16_to_f32(lin);
        f = f < 0.f ? 0.f : f;
        out = f32_to_bf16_rne(f * f);
    } else if (RES) {
        out = f32_to_bf16_rne(__uint_as_float(b.res << 16) + bf16_to_f32(lin));
    }
    // the descriptor covers the output rows of the last slice only (other steps drop every
    // store); lanes past T MR or past the valid rows store out of range
    const int st_t = lane / MR, st_m = lane % MR;
    const bool st_ok = lane < T * MR && st_t < c.rows && st_m < c.M;
    const __amdgpu_buffer_rsrc_t yr =
        __builtin_amdgcn_make_buffer_rsrc(c.y0, 0, last ? ((MR - 1) * c.ldy + c.rows) * 2 : 0, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b16(out, yr, st_ok ? (st_m * c.ldy + st_t) * 2 : 0x40000000, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
}

// Steps of wave gw of a single launch: its row groups (gw, gw + nw, ...) times the slices.
__device__ __forceinline__ int single_steps(const StreamArgs& a, int gw, int nw) {
    const int n = a.total_rg;
    return (gw < n ? (n - 1 - gw) / nw + 1 : 0) * a.one.S;
}

// CHAIN: the phases come from a.tab (device memory, read as constant memory), x per step from
// global memory.  Otherwise one phase in a.one, x staged in LDS (NORM: RMSNorm-ed on the way).
template <int T, bool CHAIN, bool XG, bool NORM, bool RES, int XPC, int MR>
__global__ __launch_bounds__(256, 2) void gemv_stream_kernel(const StreamArgs a) {
    static_assert(!(NORM && (XG || CHAIN)), "the fused RMSNorm stages x in LDS (single launches)");
    static_assert(!CHAIN || XG, "chains read x per step");
    static_assert(MR == 1 || !(XG || CHAIN), "two activation rows are staged in LDS (single launches)");
    extern __shared__ uint4 xs[];                  // [row][half][xs_half] (LDS mode)
    __shared__ float red[NORM ? kWaves * MR : 1];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const NMI_CONST StreamPhase* tab = (const NMI_CONST StreamPhase*)a.tab;
    const int nw = (int)gridDim.x * kWaves;
    const int gw = (int)blockIdx.x * kWaves + wave;
    const int xs_half = a.xs_half;
    // the wave's step count: a scalar load from the chain's table (constant address space, read
    // before any vector load so that no wait for it can hold one up), or arithmetic
    const int nsteps = CHAIN ? ((const NMI_CONST int*)a.wave_steps)[gw] : single_steps(a, gw, nw);

    Buf<T, XG> A, B;
    float a0[T][MR], a1[T][MR];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int m = 0; m < MR; ++m) a0[t][m] = a1[t][m] = 0.f;

    Cursor c0 = cursor_start<T, CHAIN>(a, tab, gw);
    if constexpr (!XG) {
        // stage x [MR][K] (single phase): per activation row, pieces of 8 activations, piece e ->
        // chunk e >> 1, half e & 1; issued before the first weights, written to LDS after them
        const NMI_CONST StreamPhase& ph = phase_at<false>(a, tab, 0);
        const int npieces = 2 * ph.C;                // XPC * 256 >= npieces
        uint4 xr[MR][XPC];
        float4 gr[NORM ? 2 * XPC : 1];
#pragma unroll
        for (int q = 0; q < XPC; ++q) {
            const int e = min(tid + 256 * q, npieces - 1);
#pragma unroll
            for (int m = 0; m < MR; ++m) xr[m][q] = load16(ph.x + (int64_t)min(m, a.M - 1) * a.ldx + (int64_t)e * 8);
            if constexpr (NORM) {
                gr[2 * q] = *reinterpret_cast<const float4*>(a.norm_w + e * 8);
                gr[2 * q + 1] = *reinterpret_cast<const float4*>(a.norm_w + e * 8 + 4);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        issue_w<T, RES, XG, MR>(c0, lane, A);
        float r[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) r[m] = 1.f;
        if constexpr (NORM) {
            // sum of squares per row: per thread over its pieces in order, the wave sum, then the
            // four waves (0 + 1) + (2 + 3) -- the order of rmsnorm.hip
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float ss = 0.f;
#pragma unroll
                for (int q = 0; q < XPC; ++q)
                    if (tid + 256 * q < npieces) ss = sumsq8(xr[m][q], ss);
                ss = wave_sum(ss);
                if (lane == 0) red[wave * MR + m] = ss;
            }
            __syncthreads();
#pragma unroll
            for (int m = 0; m < MR; ++m)
                r[m] = rms_factor((red[m] + red[MR + m]) + (red[2 * MR + m] + red[3 * MR + m]), ph.K, a.eps);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int q = 0; q < XPC; ++q) {
                const int e = tid + 256 * q;
                if (e < npieces) {
                    uint4 v = xr[m][q];
                    if constexpr (NORM) v = rms_scale8(v, gr[2 * q], gr[2 * q + 1], r[m]);
                    xs[(2 * m + (e & 1)) * xs_half + (e >> 1)] = v;
                }
            }
        __syncthreads();
    } else {
        issue_w<T, RES, XG, MR>(c0, lane, A);
        if constexpr (XG) issue_x(c0, lane, A);
    }

    // Double-buffered walk over the wave's nsteps steps, two per iteration: each half issues the
    // successor's weights into the other buffer, finds the step after the successor (scalar work
    // and descriptor loads that overlap this step's memory wait), computes the current step, then
    // issues the successor's x.  The loop exits only at its top (steps past the end are null
    // steps); an odd last step is computed after it.
    Cursor c1 = cursor_next<T, CHAIN>(a, tab, c0, nw);
    int k = 0;
    for (; k + 2 <= nsteps; k += 2) {
        issue_w<T, RES, XG, MR>(c1, lane, B);
        Cursor c2 = cursor_next<T, CHAIN>(a, tab, c1, nw);
        compute<T, XG, RES, MR>(c0, lane, A, xs, xs_half, a0, a1);
        if constexpr (XG) issue_x(c1, lane, B);
        issue_w<T, RES, XG, MR>(c2, lane, A);
        c0 = cursor_next<T, CHAIN>(a, tab, c2, nw);       // the step after c2, for the next iteration
        compute<T, XG, RES, MR>(c1, lane, B, xs, xs_half, a0, a1);
        if constexpr (XG) issue_x(c2, lane, A);
        // rotate: the current step is c2 (in A), its successor c0
        const Cursor t = c0;
        c0 = c2;
        c1 = t;
    }
    if (k < nsteps) {
        compute<T, XG, RES, MR>(c0, lane, A, xs, xs_half, a0, a1);
    }

}

// Slices of a phase: at most 256 chunks each, as equal as possible.
void plan_slices(StreamPhase& ph) {
    ph.C = ph.K >> 4;
    ph.S = (ph.C + 255) / 256;
    ph.sw = (ph.C + ph.S - 1) / ph.S;
}

// Row groups of a phase's groups (rg_begin) and of the phase; returns the phase's count.
int plan_rows(StreamPhase& ph, int T) {
    int n = 0;
    for (int i = 0; i < ph.ngroups; ++i) {
        ph.g[i].rg_begin = n;
        n += (ph.g[i].N + T - 1) / T;
    }
    return n;
}

template <int T, bool NORM, bool RES, int XPC, int MR>
hipError_t launch_single(const StreamArgs& a, int grid, size_t lds, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_stream_kernel<T, false, false, NORM, RES, XPC, MR>), dim3(grid), dim3(256), lds, stream,
                       a);
    return hipGetLastError();
}

template <int T, bool NORM, bool RES, int MR>
hipError_t launch_single_x(int xpc, const StreamArgs& a, int grid, size_t lds, hipStream_t stream) {
    switch (xpc) {
        case 2: return launch_single<T, NORM, RES, 2, MR>(a, grid, lds, stream);
        case 4: return launch_single<T, NORM, RES, 4, MR>(a, grid, lds, stream);
        case 8:
            // two activation rows with the fused RMSNorm over 8 staging pieces each would spill:
            // never launched
            if constexpr (MR == 2 && NORM) return hipErrorInvalidValue;
            else return launch_single<T, NORM, RES, 8, MR>(a, grid, lds, stream);
        default:
            // 4 weight rows, or several activation rows, with 16 staging pieces would spill: never launched
            if constexpr ((T == 4 && NORM) || MR > 1) return hipErrorInvalidValue;
            else return launch_single<T, NORM, RES, 16, MR>(a, grid, lds, stream);
    }
}

// The fused RMSNorm (up projection) and the residual (down projection) never come together.
template <int T, int MR>
hipError_t launch_single_t(bool norm, bool res, int xpc, const StreamArgs& a, int grid, size_t lds,
                           hipStream_t stream) {
    if (norm) return launch_single_x<T, true, false, MR>(xpc, a, grid, lds, stream);
    if (res) return launch_single_x<T, false, true, MR>(xpc, a, grid, lds, stream);
    return launch_single_x<T, false, false, MR>(xpc, a, grid, lds, stream);
}

// x pieces (8 activations) per thread and row: 2 C pieces over 256 threads, in powers of two
int stream_xpc(int C) {
    const int need = (2 * C + 255) / 256;
    return need <= 2 ? 2 : (need <= 4 ? 4 : (need <= 8 ? 8 : 16));
}

}  // namespace

// M = 1: K up to 16 * kStreamMaxLdsChunks; M = 2: the two rows' staging pieces fit the registers
// (8 per thread and row, 4 with the fused RMSNorm), i.e. K <= 16384 (8192).  (M = 4 as four
// rows per weight step measured slower than the 4x4x4 MFMA kernel: config 2 at M = 4 72 against
// 44 us.)
bool gemv_stream_supported(int M, int K, bool norm) {
    const int C = K >> 4;
    if (M == 1) return C <= kStreamMaxLdsChunks;
    if (M == 2) return stream_xpc(C) <= (norm ? 4 : 8);
    return false;
}

hipError_t launch_gemv_stream(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups, int ngroups,
                              hipStream_t stream, const Norm& norm) {
    if (!gemv_stream_supported(M, K, norm.w != nullptr)) return hipErrorInvalidValue;
    const DeviceInfo& dev = device_info();
    StreamArgs a{};
    StreamPhase& ph = a.one;
    ph.x = x;
    ph.K = K;
    ph.ngroups = ngroups;
    for (int i = 0; i < ngroups; ++i) {
        const GemvGroup& G = groups[i];
        ph.g[i] = StreamGroup{G.W,  G.ldw, G.s,        G.y, G.epi.kind == kEpiResidual ? G.epi.res : nullptr,
                              G.N,  0,     G.epi.kind, (int)G.ldy, (int)G.epi.ldres, 0};
    }
    a.ldx = ldx;
    a.M = M;
    // rows per step: 2 (measured on the decode shapes, 3-46 MB: more, shorter-lived waves ramp
    // a single launch faster), or 4 with tuning knob gemv.t = 4 (the chains' choice; M = 1)
    const int need_x = (2 * (K >> 4) + 255) / 256;      // x pieces per thread
    const int T = M == 1 && tuning().gemv_t == 4 && !(norm.w && need_x > 8) ? 4 : 2;
    plan_slices(ph);
    const int nrg = plan_rows(ph, T);
    ph.g_begin = 0;
    ph.g_end = nrg;
    a.nphases = 1;
    a.total_rg = nrg;
    a.norm_w = norm.w;
    a.eps = norm.eps;
    // x in LDS: per row two halves of C chunks (rounded up to 64 so that the halves start 1 KiB
    // apart)
    a.xs_half = (ph.C + 63) & ~63;
    const size_t lds = (size_t)M * a.xs_half * 2 * sizeof(uint4);
    // waves: about 3 steps each, at most one workgroup per CU (measured on 12544 x 3136: one
    // workgroup of 4 waves per CU, each wave double-buffering its rows, ramps faster than two)
    const Tuning& tn = tuning();
    const int per_cu = tn.gemv_wgs >= 1 && tn.gemv_wgs <= 2 ? tn.gemv_wgs : 1;
    const int64_t want = ((int64_t)nrg * ph.S + 3 * kWaves - 1) / (3 * kWaves);
    const int64_t cap = (int64_t)per_cu * dev.num_cu;
    int grid = (int)(want < 1 ? 1 : (want < cap ? want : cap));
    if (tn.gemv_balance != 2) {
        // as few waves as keep the most row groups per wave, so that no wave ends a round early
        // (measured: 1-6% faster on five of the six decode shapes, 1% slower on up_proj)
        const int64_t per_wave = ((int64_t)nrg + (int64_t)grid * kWaves - 1) / ((int64_t)grid * kWaves);
        const int64_t waves = ((int64_t)nrg + per_wave - 1) / per_wave;
        grid = (int)((waves + kWaves - 1) / kWaves);
    }
    if (tn.gemv_grid > 0) grid = tn.gemv_grid;
    const int xpc = stream_xpc(ph.C);
    bool res = false;
    for (int i = 0; i < ngroups; ++i) res = res || groups[i].epi.kind == kEpiResidual;
    if (norm.w && res) return hipErrorInvalidValue;
    if (M == 2) return launch_single_t<2, 2>(norm.w != nullptr, res, xpc, a, grid, lds, stream);
    return T == 4 ? launch_single_t<4, 1>(norm.w != nullptr, res, xpc, a, grid, lds, stream)
                  : launch_single_t<2, 1>(norm.w != nullptr, res, xpc, a, grid, lds, stream);
}

int stream_chain_plan(StreamPhase* phases, int nphases) {
    int g = 0;
    for (int p = 0; p < nphases; ++p) {
        StreamPhase& ph = phases[p];
        plan_slices(ph);
        const int n = plan_rows(ph, kStreamChainT);
        ph.g_begin = g;
        ph.g_end = g + n;
        g += n;
    }
    return g;
}

void stream_chain_wave_steps(const StreamPhase* phases, int nphases, int nw, int* out) {
    for (int w = 0; w < nw; ++w) out[w] = 0;
    for (int p = 0; p < nphases; ++p) {
        const StreamPhase& ph = phases[p];
        for (int g = ph.g_begin; g < ph.g_end; ++g) out[g % nw] += ph.S;
    }
}

hipError_t stream_chain_grid(int total_rg, int* grid) {
    const DeviceInfo& dev = device_info();
    int per_cu = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, gemv_stream_kernel<kStreamChainT, true, true, false, false, 1, 1>, 256, 0);
    if (e != hipSuccess) return e;
    const int cap = tuning().chain_wgs >= 1 ? tuning().chain_wgs : 2;
    if (cap < per_cu) per_cu = cap;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    const int64_t resident = (int64_t)per_cu * dev.num_cu;
    const int64_t want = ((int64_t)total_rg + kWaves - 1) / kWaves;     // at least one row group per wave
    *grid = (int)(want < resident ? (want < 1 ? 1 : want) : resident);
    return hipSuccess;
}

hipError_t launch_gemv_stream_chain(const StreamPhase* tab, const int* wave_steps, int nphases, int total_rg, int grid,
                                    hipStream_t stream) {
    StreamArgs a{};
    a.tab = tab;
    a.wave_steps = wave_steps;
    a.nphases = nphases;
    a.total_rg = total_rg;
    hipLaunchKernelGGL((gemv_stream_kernel<kStreamChainT, true, true, false, false, 1, 1>), dim3(grid), dim3(256), 0,
                       stream, a);
    return hipGetLastError();
}

}  // namespace nmi
