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

}  // namespace

bool gemv_norm_supported(int M, int K) {
    if (M <= 2 && tuning().gemv_multirow == 0 && gemv_stream_supported(M, K, true)) return true;
    const int C = K >> 4;
    return (M == 1 || M == 2) && 2 * C <= 256 * (8 / M);
}

hipError_t launch_gemv_grouped(const uint16_t* x, int64_t ldx, int M, int K, const GemvGroup* groups,
                               int ngroups, hipStream_t stream, const Norm& norm) {
    // M <= 2: the stream kernel (gemv_stream.hip) where it takes the shape, unless tuning knob
    // gemv.multirow selects this one
    if (M <= 2 && tuning().gemv_multirow == 0 && gemv_stream_supported(M, K, norm.w != nullptr))
        return launch_gemv_stream(x, ldx, M, K, groups, ngroups, stream, norm);
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
