// Batch-1..8 GEMV for decode: y[b] = W x[b], W row-major (rows x cols), fp32 or bf16.
//
// Replaces the reference's dense -> matmul/weightedSum (domain/graph/.../LayerFeatures.java:785-830,
// compute/algebra/.../MatrixFeatures.java:182-337), which sums each output sequentially over the
// input index; here each output row is reduced by one 64-lane wavefront.
//
// Design (HBM-bound, every weight byte is read exactly once per call):
//  * 256-thread blocks = 4 wavefronts; each wavefront owns RPW consecutive rows (2*RPW for the
//    SwiGLU pair) and streams them with 16-byte loads, UNR column chunks in flight per row.
//  * the input vectors are staged once per block in LDS (fp32), in column slices of at most
//    SLICE floats per batch entry; the optional RMSNorm prologue
//    (NormalizationLayerFeatures.java:584-595: y = (w*x) * 1/sqrt(mean(x^2)+eps)) is applied
//    while staging, so the normalised vector never goes to HBM.
//  * epilogues: store (+bias), residual add, SwiGLU (u * g * 1/(exp(-g)+1),
//    ActivationFeatures.java:263-265, ArithmeticFeatures.java:754-756), and greedy argmax
//    (AggregationFeatures.java:111-121, first maximum wins) finished by the last block to arrive.
#include "ar_hip_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsFloats = 8192;  // 32 KB of staged input per block

struct GemvParams {
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
    float* part_val;
    int* part_idx;
    unsigned* counter;
    int* tokens;
    int token_stride;
    int* state;     // {position, prompt length}
    int advance;
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

__device__ inline bool better(float v1, int i1, float v2, int i2) {
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

template <typename WT, int NB, int RPW, int EPI>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
    using V = WVec<WT>;
    constexpr int VEC = V::N;
    constexpr int NMAT = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    constexpr int NR = RPW * NMAT;                  // weight rows streamed per wavefront
    constexpr int UNR = (16 / NR) > 0 ? 16 / NR : 1;  // column chunks in flight per row
    constexpr int SLICE = kLdsFloats / NB;          // staged columns per batch entry

    __shared__ __attribute__((aligned(16))) float hs[kLdsFloats];
    __shared__ float red[kWaves][NB];
    __shared__ float s_val[kWaves][NB];
    __shared__ int s_idx[kWaves][NB];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int cols = p.cols;
    const int row_base = (blockIdx.x * kWaves + wave) * RPW;

    // ---- RMSNorm factor per batch entry (whole block cooperates) --------------------
    float rn[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) rn[b] = 1.0f;
    if (p.norm_w) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float ss = 0.f;
            if (b < p.batch) {
                const float* xb = p.x + (size_t)b * p.x_stride;
                for (int i = tid; i < cols; i += kThreads) {
                    float v = xb[i];
                    ss += v * v;
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

    // ---- rows of this wavefront (clamped for loads; results of padding rows dropped) ---
    const WT* wrow[NR];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        int row = min(row_base + r, p.rows - 1);
        wrow[r] = reinterpret_cast<const WT*>(p.w) + (size_t)row * cols;
        if (NMAT == 2) wrow[RPW + r] = reinterpret_cast<const WT*>(p.w2) + (size_t)row * cols;
    }

    float acc[NR][NB];
#pragma unroll
    for (int r = 0; r < NR; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[r][b] = 0.f;

    for (int s0 = 0; s0 < cols; s0 += SLICE) {
        const int sl = min(SLICE, cols - s0);
        __syncthreads();
        // stage x (normalised if asked) for this slice
        for (int i = tid * 4; i < sl; i += kThreads * 4) {
            float4 wv = make_float4(1.f, 1.f, 1.f, 1.f);
            if (p.norm_w) wv = *reinterpret_cast<const float4*>(p.norm_w + s0 + i);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                float4 h = make_float4(0.f, 0.f, 0.f, 0.f);
                if (b < p.batch) {
                    float4 xv = *reinterpret_cast<const float4*>(p.x + (size_t)b * p.x_stride + s0 + i);
                    if (p.norm_w) {
                        h.x = (wv.x * xv.x) * rn[b];
                        h.y = (wv.y * xv.y) * rn[b];
                        h.z = (wv.z * xv.z) * rn[b];
                        h.w = (wv.w * xv.w) * rn[b];
                    } else {
                        h = xv;
                    }
                }
                *reinterpret_cast<float4*>(&hs[b * SLICE + i]) = h;
            }
        }
        __syncthreads();

        constexpr int CH = 64 * VEC;  // columns per wavefront chunk
        const int nfull = sl / CH;
        int c = 0;
        for (; c + UNR <= nfull; c += UNR) {
            typename V::raw wv[UNR][NR];
#pragma unroll
            for (int u = 0; u < UNR; u++)
#pragma unroll
                for (int r = 0; r < NR; r++)
                    wv[u][r] = *reinterpret_cast<const typename V::raw*>(wrow[r] + s0 + (c + u) * CH + lane * VEC);
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int col = (c + u) * CH + lane * VEC;
                float hv[NB][VEC];
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int j = 0; j < VEC; j += 4) {
                        float4 t = *reinterpret_cast<const float4*>(&hs[b * SLICE + col + j]);
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
        // remaining full chunks one at a time, then the ragged tail
        for (; c * CH < sl; c++) {
            const int col = c * CH + lane * VEC;
            if (col < sl) {
                float hv[NB][VEC];
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int j = 0; j < VEC; j += 4) {
                        float4 t = *reinterpret_cast<const float4*>(&hs[b * SLICE + col + j]);
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
                    float v = acc[r][b];
                    if (EPI == GEMV_EPI_STORE) {
                        if (p.bias) v += p.bias[row];
                        *yp = v;
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

    // greedy argmax: logits (optional store), block best, last block picks the token
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
    if (tid < NB) {
        float bv = s_val[0][tid];
        int bi = s_idx[0][tid];
#pragma unroll
        for (int w = 1; w < kWaves; w++)
            if (better(s_val[w][tid], s_idx[w][tid], bv, bi)) { bv = s_val[w][tid]; bi = s_idx[w][tid]; }
        p.part_val[(size_t)blockIdx.x * NB + tid] = bv;
        p.part_idx[(size_t)blockIdx.x * NB + tid] = bi;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        unsigned prev = atomicAdd(p.counter, 1u);
        s_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    // last block: reduce the per-block partials of every batch entry
    const int nblk = gridDim.x;
    for (int b = 0; b < NB; b++) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int i = tid; i < nblk; i += kThreads) {
            float v = p.part_val[(size_t)i * NB + b];
            int ix = p.part_idx[(size_t)i * NB + b];
            if (better(v, ix, bv, bi)) { bv = v; bi = ix; }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            float ov = __shfl_xor(bv, off, 64);
            int oi = __shfl_xor(bi, off, 64);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { s_val[wave][b] = bv; s_idx[wave][b] = bi; }
    }
    __syncthreads();
    if (tid == 0) {
        const int pos = p.state ? p.state[0] : 0;
        const int plen = p.state ? p.state[1] : 0;
        for (int b = 0; b < p.batch; b++) {
            float bv = s_val[0][b];
            int bi = s_idx[0][b];
            for (int w = 1; w < kWaves; w++)
                if (better(s_val[w][b], s_idx[w][b], bv, bi)) { bv = s_val[w][b]; bi = s_idx[w][b]; }
            if (bi == 0x7FFFFFFF) bi = 0;  // every logit NaN: the reference keeps index 0
            if (p.tokens) {
                if (p.state) {
                    if (pos + 1 >= plen) p.tokens[(size_t)b * p.token_stride + pos + 1] = bi;
                } else {
                    p.tokens[(size_t)b * p.token_stride] = bi;
                }
            }
        }
        if (p.advance && p.state) p.state[0] = pos + 1;
        *p.counter = 0u;
    }
}

template <typename WT, int NB, int RPW, int EPI>
int launch_t(const GemvLaunch& a, hipStream_t stream) {
    GemvParams p;
    p.w = a.w; p.w2 = a.w2; p.rows = a.rows; p.cols = a.cols; p.batch = a.batch;
    p.x = a.x; p.x_stride = a.x_stride; p.norm_w = a.norm_w; p.eps = a.eps; p.bias = a.bias;
    p.y = a.y; p.y_stride = a.y_stride; p.part_val = a.part_val; p.part_idx = a.part_idx;
    p.counter = a.counter; p.tokens = a.tokens; p.token_stride = a.token_stride; p.state = a.state;
    p.advance = a.advance;
    const int rows_per_block = kWaves * RPW;
    const int grid = (a.rows + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((gemv_kernel<WT, NB, RPW, EPI>), dim3(grid), dim3(kThreads), 0, stream, p);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

template <typename WT, int NB, int EPI>
int pick_rpw(const GemvLaunch& a, hipStream_t s) {
    // Enough wavefronts to cover 256 CUs several times over, with RPW rows each.
    if (NB == 1) {
        if (a.rows >= 16384) return launch_t<WT, NB, 4, EPI>(a, s);
        if (a.rows >= 4096) return launch_t<WT, NB, 2, EPI>(a, s);
        return launch_t<WT, NB, 1, EPI>(a, s);
    }
    if (NB <= 4 && a.rows >= 8192) return launch_t<WT, NB, 2, EPI>(a, s);
    return launch_t<WT, NB, 1, EPI>(a, s);
}

template <typename WT, int EPI>
int pick_nb(const GemvLaunch& a, hipStream_t s) {
    if (a.batch <= 1) return pick_rpw<WT, 1, EPI>(a, s);
    if (a.batch <= 2) return pick_rpw<WT, 2, EPI>(a, s);
    if (a.batch <= 4) return pick_rpw<WT, 4, EPI>(a, s);
    return pick_rpw<WT, 8, EPI>(a, s);
}

template <typename WT>
int pick_epi(const GemvLaunch& a, hipStream_t s) {
    switch (a.epilogue) {
        case GEMV_EPI_STORE: return pick_nb<WT, GEMV_EPI_STORE>(a, s);
        case GEMV_EPI_RESIDUAL: return pick_nb<WT, GEMV_EPI_RESIDUAL>(a, s);
        case GEMV_EPI_SWIGLU: return pick_nb<WT, GEMV_EPI_SWIGLU>(a, s);
        case GEMV_EPI_ARGMAX: return pick_nb<WT, GEMV_EPI_ARGMAX>(a, s);
    }
    ar_set_error("unknown GEMV epilogue %d", a.epilogue);
    return AR_HIP_ERR_INVALID;
}

int rpw_for(int rows, int batch) {
    if (batch <= 1) return rows >= 16384 ? 4 : (rows >= 4096 ? 2 : 1);
    if (batch <= 4 && rows >= 8192) return 2;
    return 1;
}

}  // namespace

int gemv_argmax_partials(int rows, int batch) {
    const int rpb = kWaves * rpw_for(rows, batch);
    const int nb = batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : 8;
    return ((rows + rpb - 1) / rpb) * nb;
}

int launch_gemv(const GemvLaunch& a, hipStream_t stream) {
    AR_CHECK_ARG(a.w && a.x, "GEMV: null weight or input");
    AR_CHECK_ARG(a.rows > 0 && a.cols > 0, "GEMV: empty shape %dx%d", a.rows, a.cols);
    AR_CHECK_ARG(a.batch >= 1 && a.batch <= 8, "GEMV: batch %d outside 1..8", a.batch);
    AR_CHECK_ARG(a.cols % 8 == 0, "GEMV: cols %d must be a multiple of 8", a.cols);
    AR_CHECK_ARG(a.x_stride % 4 == 0 && a.x_stride >= a.cols, "GEMV: bad input stride %d", a.x_stride);
    AR_CHECK_ARG((reinterpret_cast<uintptr_t>(a.w) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0,
                 "GEMV: weight and input must be 16-byte aligned");
    AR_CHECK_ARG(!a.norm_w || (reinterpret_cast<uintptr_t>(a.norm_w) & 15) == 0, "GEMV: norm gain not aligned");
    if (a.epilogue == GEMV_EPI_SWIGLU)
        AR_CHECK_ARG(a.w2 && (reinterpret_cast<uintptr_t>(a.w2) & 15) == 0, "GEMV: SwiGLU needs an aligned up matrix");
    if (a.epilogue == GEMV_EPI_ARGMAX) {
        AR_CHECK_ARG(a.part_val && a.part_idx && a.counter, "GEMV argmax: missing partial buffers");
    } else {
        AR_CHECK_ARG(a.y && a.y_stride >= a.rows, "GEMV: null output or short stride");
    }
    if (a.wdtype == AR_DTYPE_F32) return pick_epi<float>(a, stream);
    if (a.wdtype == AR_DTYPE_BF16) return pick_epi<uint16_t>(a, stream);
    ar_set_error("GEMV: unknown weight dtype %d", a.wdtype);
    return AR_HIP_ERR_INVALID;
}
