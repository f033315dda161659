// Batch-1..8 GEMV for decode: y[b] = W x[b], W row-major (rows x cols), fp32 or bf16.
//
// Replaces the reference's dense -> matmul/weightedSum (domain/graph/.../LayerFeatures.java:785-830,
// compute/algebra/.../MatrixFeatures.java:182-337), which sums each output sequentially over the
// input index; here each output row is reduced by one 64-lane wavefront.
//
// Design (HBM-bound, every weight byte is read exactly once per call):
//  * 256-thread blocks = 4 wavefronts; each wavefront owns RPW consecutive rows (2*RPW for the
//    SwiGLU pair) and streams them with 16-byte loads, UNR column chunks of 64 lanes x 16 B per
//    row issued back to back, so NR*UNR loads per lane are in flight.  Chunk indices past the
//    row end are clamped (the duplicate load hits cache) and their products skipped, so short
//    rows still issue one full batch of loads.
//  * the input vectors are staged once per block in LDS (fp32), in column slices of at most
//    SLICE floats per batch entry; the optional RMSNorm prologue
//    (NormalizationLayerFeatures.java:584-595: y = (w*x) * 1/sqrt(mean(x^2)+eps)) is applied
//    while staging, so the normalised vector never goes to HBM.
//  * epilogues: store (+bias), residual add, SwiGLU (u * g * 1/(exp(-g)+1),
//    ActivationFeatures.java:263-265, ArithmeticFeatures.java:754-756), and greedy argmax
//    (AggregationFeatures.java:111-121, first maximum wins): each block folds its best
//    (value, index) into packed 64-bit keys with atomicMax; the next step's embed kernel reads
//    the maximum after the kernel boundary, so no block ever needs a device-wide fence.
#pragma once
#include "ar_hip_internal.h"

namespace gemv {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsFloats = 8192;  // 32 KB of staged input per block

struct Params {
    const void* w;
    const void* w2;
    int rows, cols, batch;
    const float* x;
    int x_stride;
    const float* norm_w;
    float eps;
    const float* bias;
    float* y;
    int y_stride;
    unsigned long long* keys;  // argmax: [batch][kArgmaxSlots] packed (value, index) maxima
    const uint16_t* x_hi;      // operand planes of the input / output (GemvLaunch), MFMA path only
    const uint16_t* x_lo;
    uint16_t* y_hi;
    uint16_t* y_lo;
    const float* y_gain;
    float* kpart;              // k-split workspace of the MFMA streaming form (GemvLaunch), or null
    int kpart_floats;
    unsigned* kcount;
    int kcount_n;
    const uint16_t* wf;        // fragment-ordered copies of w / w2 (GemvLaunch), or null
    const uint16_t* wf2;
    const float* ss_in;        // per-16-row sums of squares of x / of the residual output (GemvLaunch)
    float* ss_out;
};

template <typename WT>
struct WVec;

// fp32: 4 values per 16-byte load
template <>
struct WVec<float> {
    static constexpr int N = 4;
    using raw = float4;
    __device__ static inline void unpack(const raw& v, float* f) {
        f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
    }
};

// bf16 (stored as uint16): 8 values per 16-byte load
template <>
struct WVec<uint16_t> {
    static constexpr int N = 8;
    using raw = uint4;
    __device__ static inline void unpack(const raw& v, float* f) {
        const unsigned u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            f[2 * i] = __uint_as_float(u[i] << 16);
            f[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
        }
    }
};

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum over the 64 lanes on the DPP network (no LDS round trips): quad swaps, row shifts by 4 and 8,
// then the row totals broadcast across rows; the total lands in lane 63 (the other lanes hold
// partial sums).
template <int CTRL, int ROW_MASK>
__device__ inline float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, true));
}
__device__ inline float dpp_sum_lane63(float v) {
    v = dpp_add<0xB1, 0xF>(v);   // quad_perm 1,0,3,2
    v = dpp_add<0x4E, 0xF>(v);   // quad_perm 2,3,0,1
    v = dpp_add<0x114, 0xF>(v);  // row_shr:4
    v = dpp_add<0x118, 0xF>(v);  // row_shr:8
    v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}
// N independent sums, step by step across all N: each DPP step waits two cycles for the previous
// write of its operand, so N chains written one after the other stall on every step, while steps
// interleaved over N values fill those cycles (each sum is added in the same order as above).
template <int N>
__device__ inline void dpp_sum_lane63_n(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = dpp_add<0xB1, 0xF>(v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = dpp_add<0x4E, 0xF>(v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = dpp_add<0x114, 0xF>(v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = dpp_add<0x118, 0xF>(v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = dpp_add<0x142, 0xA>(v[i]);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = dpp_add<0x143, 0xC>(v[i]);
}

__device__ inline bool better(float v1, int i1, float v2, int i2) {
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

// (value, index) packed so that unsigned 64-bit max = larger value, then lower index:
// high word = order-preserving image of the float (NaN lowest, so it never wins), low word =
// ~index.  Key 0 means "no candidate".
__device__ inline unsigned long long argmax_key(float v, int idx) {
    const unsigned u = __float_as_uint(v);
    const unsigned ord = (v != v) ? 0u : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)idx);
}

template <typename WT, int NB, int RPW, int UNR, int EPI>
__global__ __launch_bounds__(kThreads) void gemv_kernel(Params p) {
    using V = WVec<WT>;
    constexpr int VEC = V::N;
    constexpr int NMAT = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    constexpr int NR = RPW * NMAT;          // weight rows streamed per wavefront
    constexpr int SLICE = kLdsFloats / NB;  // staged columns per batch entry
    constexpr int CH = 64 * VEC;            // columns per wavefront chunk

    __shared__ __attribute__((aligned(16))) float hs[kLdsFloats];
    __shared__ float red[kWaves][NB];
    __shared__ float s_val[kWaves][NB];
    __shared__ int s_idx[kWaves][NB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int cols = p.cols;
    const int row_base = (blockIdx.x * kWaves + wave) * RPW;

    // ---- rows of this wavefront (clamped for loads; results of padding rows dropped) ---
    const WT* wrow[NR];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        const int row = min(row_base + r, p.rows - 1);
        wrow[r] = reinterpret_cast<const WT*>(p.w) + (size_t)row * cols;
        if (NMAT == 2) wrow[RPW + r] = reinterpret_cast<const WT*>(p.w2) + (size_t)row * cols;
    }

    // ---- first batch of weight loads, issued before anything that depends on x ---------
    // (weights do not depend on the previous kernel, so their HBM latency overlaps the
    // input prologue below)
    typename V::raw wv[UNR][NR];
    const int nfull0 = min(SLICE, cols) / CH;
    if (nfull0 > 0) {
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int cc = min(u, nfull0 - 1);
#pragma unroll
            for (int r = 0; r < NR; r++)
                wv[u][r] = *reinterpret_cast<const typename V::raw*>(wrow[r] + cc * CH + lane * VEC);
        }
    }

    // ---- RMSNorm factor per batch entry (whole block cooperates) --------------------
    float rn[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) rn[b] = 1.0f;
    // Short inputs (batch <= 2, cols <= 4096, one slice): x and the gain are read once into
    // registers, reduced, and written normalised to LDS -- one global round trip instead of two.
    constexpr int XV = 4;
    const bool fast = NB <= 2 && cols <= kThreads * 4 * XV && cols <= SLICE;
    if (fast) {
        float4 xr[NB <= 2 ? NB : 1][XV], gr[XV];
#pragma unroll
        for (int j = 0; j < XV; j++) {
            const int i = (tid + j * kThreads) * 4;
            const bool in = i < cols;
            gr[j] = (in && p.norm_w) ? *reinterpret_cast<const float4*>(p.norm_w + i) : make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
            for (int b = 0; b < (NB <= 2 ? NB : 1); b++)
                xr[b][j] = (in && b < p.batch) ? *reinterpret_cast<const float4*>(p.x + (size_t)b * p.x_stride + i)
                                               : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (p.norm_w) {
#pragma unroll
            for (int b = 0; b < (NB <= 2 ? NB : 1); b++) {
                float ss = 0.f;
#pragma unroll
                for (int j = 0; j < XV; j++)
                    ss += xr[b][j].x * xr[b][j].x + xr[b][j].y * xr[b][j].y + xr[b][j].z * xr[b][j].z +
                          xr[b][j].w * xr[b][j].w;
                ss = wave_sum(ss);
                if (lane == 0) red[wave][b] = ss;
            }
            __syncthreads();
#pragma unroll
            for (int b = 0; b < (NB <= 2 ? NB : 1); b++) {
                float ss = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; w++) ss += red[w][b];
                rn[b] = 1.0f / sqrtf(ss / (float)cols + p.eps);
            }
        }
#pragma unroll
        for (int j = 0; j < XV; j++) {
            const int i = (tid + j * kThreads) * 4;
            if (i < cols) {
#pragma unroll
                for (int b = 0; b < (NB <= 2 ? NB : 1); b++) {
                    float4 h = xr[b][j];
                    if (p.norm_w) {
                        h.x = (gr[j].x * h.x) * rn[b];
                        h.y = (gr[j].y * h.y) * rn[b];
                        h.z = (gr[j].z * h.z) * rn[b];
                        h.w = (gr[j].w * h.w) * rn[b];
                    }
                    *reinterpret_cast<float4*>(&hs[b * SLICE + i]) = h;
                }
            }
        }
    } else if (p.norm_w) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float ss = 0.f;
            if (b < p.batch) {
                const float4* xb = reinterpret_cast<const float4*>(p.x + (size_t)b * p.x_stride);
                for (int i = tid; i < cols / 4; i += kThreads) {
                    const float4 v = xb[i];
                    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                }
            }
            ss = wave_sum(ss);
            if (lane == 0) red[wave][b] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float ss = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; w++) ss += red[w][b];
            rn[b] = 1.0f / sqrtf(ss / (float)cols + p.eps);
        }
    }

    float acc[NR][NB];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[r][b] = 0.f;

    for (int s0 = 0; s0 < cols; s0 += SLICE) {
        const int sl = min(SLICE, cols - s0);
        __syncthreads();
        // stage x (normalised if asked) for this slice (already staged on the short-input path)
        for (int i = tid * 4; !fast && i < sl; i += kThreads * 4) {
            float4 gw = make_float4(1.f, 1.f, 1.f, 1.f);
            if (p.norm_w) gw = *reinterpret_cast<const float4*>(p.norm_w + s0 + i);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                float4 h = make_float4(0.f, 0.f, 0.f, 0.f);
                if (b < p.batch) {
                    const float4 xv = *reinterpret_cast<const float4*>(p.x + (size_t)b * p.x_stride + s0 + i);
                    if (p.norm_w) {
                        h.x = (gw.x * xv.x) * rn[b];
                        h.y = (gw.y * xv.y) * rn[b];
                        h.z = (gw.z * xv.z) * rn[b];
                        h.w = (gw.w * xv.w) * rn[b];
                    } else {
                        h = xv;
                    }
                }
                *reinterpret_cast<float4*>(&hs[b * SLICE + i]) = h;
            }
        }
        __syncthreads();

        const int nfull = sl / CH;
        for (int c = 0; c < nfull; c += UNR) {
            if (s0 != 0 || c != 0) {
#pragma unroll
                for (int u = 0; u < UNR; u++) {
                    const int cc = min(c + u, nfull - 1);
#pragma unroll
                    for (int r = 0; r < NR; r++)
                        wv[u][r] = *reinterpret_cast<const typename V::raw*>(wrow[r] + s0 + cc * CH + lane * VEC);
                }
            }
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                if (c + u < nfull) {
                    const int col = (c + u) * CH + lane * VEC;
                    float hv[NB][VEC];
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int j = 0; j < VEC; j += 4) {
                            const float4 t = *reinterpret_cast<const float4*>(&hs[b * SLICE + col + j]);
                            hv[b][j] = t.x; hv[b][j + 1] = t.y; hv[b][j + 2] = t.z; hv[b][j + 3] = t.w;
                        }
#pragma unroll
                    for (int r = 0; r < NR; r++) {
                        float wf[VEC];
                        V::unpack(wv[u][r], wf);
#pragma unroll
                        for (int b = 0; b < NB; b++)
#pragma unroll
                            for (int j = 0; j < VEC; j++) acc[r][b] = fmaf(wf[j], hv[b][j], acc[r][b]);
                    }
                }
            }
        }
        // ragged tail (cols not a multiple of the chunk width)
        const int col = nfull * CH + lane * VEC;
        if (col < sl) {
            float hv[NB][VEC];
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int j = 0; j < VEC; j += 4) {
                    const float4 t = *reinterpret_cast<const float4*>(&hs[b * SLICE + col + j]);
                    hv[b][j] = t.x; hv[b][j + 1] = t.y; hv[b][j + 2] = t.z; hv[b][j + 3] = t.w;
                }
#pragma unroll
            for (int r = 0; r < NR; r++) {
                float wf[VEC];
                V::unpack(*reinterpret_cast<const typename V::raw*>(wrow[r] + s0 + col), wf);
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int j = 0; j < VEC; j++) acc[r][b] = fmaf(wf[j], hv[b][j], acc[r][b]);
            }
        }
    }

#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[r][b] = wave_sum(acc[r][b]);

    // ---- epilogues ----------------------------------------------------------------
    if (EPI != GEMV_EPI_ARGMAX) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int row = row_base + r;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if (lane == r * NB + b && row < p.rows && b < p.batch) {
                    float* yp = p.y + (size_t)b * p.y_stride + row;
                    const float v = acc[r][b];
                    if (EPI == GEMV_EPI_STORE) {
                        *yp = p.bias ? v + p.bias[row] : v;
                    } else if (EPI == GEMV_EPI_RESIDUAL) {
                        *yp = *yp + v;
                    } else {  // SwiGLU: acc[r] = gate, acc[RPW + r] = up
                        const float g = v;
                        const float u = acc[(NMAT == 2) ? RPW + r : r][b];
                        const float sg = 1.0f / (expf(-g) + 1.0f);
                        *yp = u * (g * sg);
                    }
                }
            }
        }
        return;
    }

    // greedy argmax: logits (optional store) and this block's best (value, index) per entry
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int row = row_base + r;
            if (row < p.rows) {
                if (p.y && lane == r && b < p.batch) p.y[(size_t)b * p.y_stride + row] = acc[r][b];
                if (better(acc[r][b], row, bv, bi)) { bv = acc[r][b]; bi = row; }
            }
        }
        if (lane == 0) { s_val[wave][b] = bv; s_idx[wave][b] = bi; }
    }
    __syncthreads();
    if (tid < p.batch) {
        float bv = s_val[0][tid];
        int bi = s_idx[0][tid];
#pragma unroll
        for (int w = 1; w < kWaves; w++)
            if (better(s_val[w][tid], s_idx[w][tid], bv, bi)) { bv = s_val[w][tid]; bi = s_idx[w][tid]; }
        // one device-scope atomic per block and sequence, spread over kArgmaxSlots addresses
        if (bi != 0x7FFFFFFF)
            atomicMax(p.keys + (size_t)tid * kArgmaxSlots + (blockIdx.x & (kArgmaxSlots - 1)), argmax_key(bv, bi));
    }
}

// Launch shape for a GEMV: rows per wavefront and column chunks in flight per row.
struct Shape {
    int rpw, unr, nb;
};

inline int nb_for(int batch) { return batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : 8; }

inline Shape shape_for(int rows, int cols, int batch, int wdtype, int epi) {
    Shape s;
    s.nb = nb_for(batch);
    const int ch = 64 * (wdtype == AR_DTYPE_BF16 ? 8 : 4);
    const int nchunk = (cols + ch - 1) / ch;
    const int nmat = epi == GEMV_EPI_SWIGLU ? 2 : 1;
    if (s.nb == 1) {
        // enough wavefronts to give each of 256 CUs several, then as many rows per wave as fit
        // (SwiGLU streams two matrices per row: one row pair per wave measured fastest below 8192
        // rows, 7.0 vs 8.0 us at 2 x 3072 x 1024 fp32; at 2048 rows one row per wave is faster too:
        // bf16 2048 x 6144 7.8 vs 8.9 us, 2048 x 2048 4.4 vs 4.6 us)
        s.rpw = rows >= 8192 ? 4 : (rows > 2048 && nmat == 1) ? 2 : 1;
        // ~16 loads in flight per lane: UNR chunks x RPW*NMAT rows
        const int budget = 16 / (s.rpw * nmat);
        const int want = nchunk < budget ? nchunk : budget;
        s.unr = want <= 4 ? 4 : want <= 8 ? 8 : 16;
    } else {
        s.rpw = (s.nb <= 4 && rows >= 8192) ? 2 : 1;
        s.unr = 8;
    }
    return s;
}

inline int grid_for(const Shape& s, int rows) {
    const int rpb = kWaves * s.rpw;
    return (rows + rpb - 1) / rpb;
}

template <typename WT, int NB, int RPW, int UNR, int EPI>
int launch_t(const Params& p, int grid, hipStream_t stream) {
    ar_launch((gemv_kernel<WT, NB, RPW, UNR, EPI>), dim3(grid), dim3(kThreads), 0, stream, p);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

template <typename WT, int EPI>
int dispatch(const Params& p, const Shape& s, hipStream_t st) {
    const int grid = grid_for(s, p.rows);
    if (s.nb == 1) {
#define AR_GEMV_U(R)                                                       \
    switch (s.unr) {                                                       \
        case 4: return launch_t<WT, 1, R, 4, EPI>(p, grid, st);            \
        case 8: return launch_t<WT, 1, R, 8, EPI>(p, grid, st);            \
        default: return launch_t<WT, 1, R, 16, EPI>(p, grid, st);          \
    }
        if (s.rpw == 4) { AR_GEMV_U(4) }
        if (s.rpw == 2) { AR_GEMV_U(2) }
        AR_GEMV_U(1)
#undef AR_GEMV_U
    }
#define AR_GEMV_B(NBV)                                                     \
    if (s.nb == NBV) {                                                     \
        if (s.rpw == 2) return launch_t<WT, NBV, 2, 8, EPI>(p, grid, st);  \
        return launch_t<WT, NBV, 1, 8, EPI>(p, grid, st);                  \
    }
    AR_GEMV_B(2)
    AR_GEMV_B(4)
    AR_GEMV_B(8)
#undef AR_GEMV_B
    ar_set_error("GEMV: no kernel for batch group %d", s.nb);
    return AR_HIP_ERR_INVALID;
}

template <typename WT>
int dispatch_epi(const Params& p, int epi, const Shape& s, hipStream_t st) {
    switch (epi) {
        case GEMV_EPI_STORE: return dispatch<WT, GEMV_EPI_STORE>(p, s, st);
        case GEMV_EPI_RESIDUAL: return dispatch<WT, GEMV_EPI_RESIDUAL>(p, s, st);
        case GEMV_EPI_SWIGLU: return dispatch<WT, GEMV_EPI_SWIGLU>(p, s, st);
        case GEMV_EPI_ARGMAX: return dispatch<WT, GEMV_EPI_ARGMAX>(p, s, st);
    }
    ar_set_error("unknown GEMV epilogue %d", epi);
    return AR_HIP_ERR_INVALID;
}

}  // namespace gemv

// per-dtype entry points (gemv_f32.hip, gemv_bf16.hip)
int gemv_launch_f32(const gemv::Params& p, int epi, const gemv::Shape& s, hipStream_t st);
int gemv_launch_bf16(const gemv::Params& p, int epi, const gemv::Shape& s, hipStream_t st);
// Batches of 3..8 sequences (gemv_batched.hip): input slices held in registers, 64/NB rows per block.
int gemv_launch_batched(const gemv::Params& p, int wdtype, int epi, hipStream_t st);
// Batch 1, no argmax, cols a multiple of the 64-lane chunk (gemv_rx.hip): input held in registers.
bool gemv_rx_fits(int rows, int cols, int batch, int wdtype, int epi, bool norm);
int gemv_launch_rx(const gemv::Params& p, int wdtype, int epi, hipStream_t st);
// Argmax epilogue (final RMSNorm + logits + greedy keys), batch 1-2, cols = 1, 2 or 4 full 64-lane
// chunks (gemv_argmax.hip): persistent grid, input in registers.
bool gemv_argmax_fits(int cols, int batch, int wdtype);
int gemv_launch_argmax(const gemv::Params& p, int wdtype, hipStream_t st);
// bf16 weights, batches of 3..16, cols % 32 == 0 (gemv_mfma.hip): 16-row tiles on the MFMA units.
int gemv_launch_mfma(const gemv::Params& p, int epi, hipStream_t st);
// Fragment-ordered bf16 weights, batches of 1..8, store / residual / SwiGLU (gemv_frag.hip).
int gemv_launch_frag(const gemv::Params& p, int epi, hipStream_t st);
