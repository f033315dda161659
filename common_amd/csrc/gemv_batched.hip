// Batched decode GEMV (3..8 sequences): y[b] = W x[b] for every sequence b of the batch.
//
// Same contract as the batch-1/2 GEMV (gemv_impl.h): the reference's dense -> matmul/weightedSum
// (domain/graph/.../LayerFeatures.java:785-830, compute/algebra/.../MatrixFeatures.java:182-337)
// with the RMSNorm prologue (NormalizationLayerFeatures.java:584-595) and the store / residual /
// SwiGLU / greedy-argmax epilogues.  With 8 input vectors every weight element feeds 8 FMAs, so
// the batch-1 design (vectors staged in LDS, re-read per row) turns into LDS and prologue traffic
// larger than the weight stream.  Here instead:
//  * a block owns R weight rows (R/2 row pairs for SwiGLU) over the whole input width; each lane
//    owns 16-byte column chunks (one per pass) and holds the matching slice of all NB input
//    vectors in registers, so every x value is loaded once per block and reused for R rows;
//  * the RMSNorm factor 1/rms(x[b]) is a per-sequence scalar, so it is applied to the finished
//    dot products: the lanes multiply only the gain into x and accumulate sum(x^2) alongside;
//  * the R*NB = 64 partial sums of a lane are reduced over the wavefront by a halving butterfly
//    (after it, lane l holds total l), then over the block's wavefronts through LDS.
#include "gemv_impl.h"

namespace {

using gemv::Params;
using gemv::WVec;

constexpr int kMaxThreads = 512;

// One halving step over entries v[0..2*HALF): lanes with the HALF bit set keep the upper half,
// the others the lower half, and each adds the copy that partner lane l^OFF sends over.
template <int HALF, int OFF, int N>
__device__ inline void halve(float (&v)[N], int lane) {
    const bool upper = lane & OFF;
#pragma unroll
    for (int i = 0; i < HALF; i++) {
        const float send = upper ? v[i] : v[i + HALF];
        const float keep = upper ? v[i + HALF] : v[i];
        v[i] = keep + __shfl_xor(send, OFF, 64);
    }
}

// Halving butterfly: 64 entries on every lane -> lane l holds the wavefront total of entry l.
__device__ inline float wave_transpose_sum(float (&v)[64], int lane) {
    halve<32, 32>(v, lane);
    halve<16, 16>(v, lane);
    halve<8, 8>(v, lane);
    halve<4, 4>(v, lane);
    halve<2, 2>(v, lane);
    halve<1, 1>(v, lane);
    return v[0];
}

// NB (4 or 8) entries on every lane -> lane l holds the wavefront total of entry l / (64/NB).
template <int NB>
__device__ inline float wave_sum_small(float (&v)[NB], int lane) {
    static_assert(NB == 4 || NB == 8, "batch tile");
    if constexpr (NB == 8) {
        halve<4, 32>(v, lane);
        halve<2, 16>(v, lane);
        halve<1, 8>(v, lane);
    } else {
        halve<2, 32>(v, lane);
        halve<1, 16>(v, lane);
    }
    float s = v[0];
#pragma unroll
    for (int off = 64 / NB / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
    return s;
}

template <typename WT, int NB, int EPI>
__global__ __launch_bounds__(kMaxThreads) void gemv_batched_kernel(Params p, int passes) {
    using V = WVec<WT>;
    constexpr int VEC = V::N;
    constexpr int NMAT = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    constexpr int R = 64 / NB;       // weight rows streamed per block (both matrices together)
    constexpr int RB = R / NMAT;     // output rows per block
    __shared__ float red[kMaxThreads / 64][64];
    __shared__ float red_ss[kMaxThreads / 64][NB];
    __shared__ float tot[64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int row0 = blockIdx.x * RB;
    const int nchunks = p.cols / VEC;

    const WT* wrow[R];
#pragma unroll
    for (int r = 0; r < RB; r++) {
        const int row = min(row0 + r, p.rows - 1);
        wrow[r] = reinterpret_cast<const WT*>(p.w) + (size_t)row * p.cols;
        if (NMAT == 2) wrow[RB + r] = reinterpret_cast<const WT*>(p.w2) + (size_t)row * p.cols;
    }

    float acc[R][NB], ss[NB];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[r][b] = 0.f;
#pragma unroll
    for (int b = 0; b < NB; b++) ss[b] = 0.f;

    for (int ps = 0; ps < passes; ps++) {
        const int c = ps * blockDim.x + tid;
        if (c >= nchunks) break;
        const int col = c * VEC;
        // weights first: they do not depend on x, so their latency overlaps the x loads
        typename V::raw wv[R];
#pragma unroll
        for (int r = 0; r < R; r++) wv[r] = *reinterpret_cast<const typename V::raw*>(wrow[r] + col);
        float g[VEC];
#pragma unroll
        for (int j = 0; j < VEC; j += 4) {
            const float4 t = p.norm_w ? *reinterpret_cast<const float4*>(p.norm_w + col + j)
                                      : make_float4(1.f, 1.f, 1.f, 1.f);
            g[j] = t.x; g[j + 1] = t.y; g[j + 2] = t.z; g[j + 3] = t.w;
        }
        float xg[NB][VEC];
#pragma unroll
        for (int b = 0; b < NB; b++) {
#pragma unroll
            for (int j = 0; j < VEC; j += 4) {
                const float4 t = b < p.batch ? *reinterpret_cast<const float4*>(p.x + (size_t)b * p.x_stride + col + j)
                                             : make_float4(0.f, 0.f, 0.f, 0.f);
                xg[b][j] = t.x; xg[b][j + 1] = t.y; xg[b][j + 2] = t.z; xg[b][j + 3] = t.w;
            }
            if (p.norm_w) {
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    ss[b] = fmaf(xg[b][j], xg[b][j], ss[b]);
                    xg[b][j] *= g[j];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            float wf[VEC];
            V::unpack(wv[r], wf);
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int j = 0; j < VEC; j++) acc[r][b] = fmaf(wf[j], xg[b][j], acc[r][b]);
        }
    }

    // ---- reductions: wavefront butterfly, then the block's wavefronts through LDS -----------
    float flat[64];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int b = 0; b < NB; b++) flat[r * NB + b] = acc[r][b];
    red[wave][lane] = wave_transpose_sum(flat, lane);
    if (p.norm_w) {
        const float s = wave_sum_small<NB>(ss, lane);
        if ((lane & (64 / NB - 1)) == 0) red_ss[wave][lane / (64 / NB)] = s;
    }
    __syncthreads();
    if (tid < 64) {
        float t = 0.f;
        for (int w = 0; w < nwaves; w++) t += red[w][tid];
        float rn = 1.0f;
        if (p.norm_w) {
            const int b = tid % NB;
            float s = 0.f;
            for (int w = 0; w < nwaves; w++) s += red_ss[w][b];
            rn = 1.0f / sqrtf(s / (float)p.cols + p.eps);
        }
        tot[tid] = t * rn;  // entry tid = weight row tid / NB of the block, sequence tid % NB
    }
    __syncthreads();

    // ---- epilogues ----------------------------------------------------------------------
    if (EPI != GEMV_EPI_ARGMAX) {
        if (tid < RB * NB) {
            const int r = tid / NB, b = tid % NB, row = row0 + r;
            if (row < p.rows && b < p.batch) {
                float* yp = p.y + (size_t)b * p.y_stride + row;
                const float v = tot[tid];
                if (EPI == GEMV_EPI_STORE) {
                    *yp = p.bias ? v + p.bias[row] : v;
                } else if (EPI == GEMV_EPI_RESIDUAL) {
                    *yp = *yp + v;
                } else {  // SwiGLU: rows 0..RB-1 gate, RB..2RB-1 up
                    const float u = tot[(RB + r) * NB + b];
                    const float sg = 1.0f / (expf(-v) + 1.0f);
                    *yp = u * (v * sg);
                }
            }
        }
        return;
    }
    if (p.y && tid < RB * NB) {
        const int r = tid / NB, b = tid % NB, row = row0 + r;
        if (row < p.rows && b < p.batch) p.y[(size_t)b * p.y_stride + row] = tot[tid];
    }
    if (tid < p.batch) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int r = 0; r < RB; r++) {
            const int row = row0 + r;
            if (row < p.rows && gemv::better(tot[r * NB + tid], row, bv, bi)) {
                bv = tot[r * NB + tid];
                bi = row;
            }
        }
        if (bi != 0x7FFFFFFF)
            atomicMax(p.keys + (size_t)tid * kArgmaxSlots + (blockIdx.x & (kArgmaxSlots - 1)), gemv::argmax_key(bv, bi));
    }
}

template <typename WT, int NB>
int launch_nb(const Params& p, int epi, hipStream_t st) {
    constexpr int VEC = WVec<WT>::N;
    const int nchunks = p.cols / VEC;
    const int passes = (nchunks + kMaxThreads - 1) / kMaxThreads;
    const int per = (nchunks + passes - 1) / passes;
    const int threads = (per + 63) / 64 * 64;
    const int rb = (64 / NB) / (epi == GEMV_EPI_SWIGLU ? 2 : 1);
    const dim3 grid((p.rows + rb - 1) / rb), block(threads);
    switch (epi) {
        case GEMV_EPI_STORE: ar_launch((gemv_batched_kernel<WT, NB, GEMV_EPI_STORE>), grid, block, 0, st, p, passes); break;
        case GEMV_EPI_RESIDUAL: ar_launch((gemv_batched_kernel<WT, NB, GEMV_EPI_RESIDUAL>), grid, block, 0, st, p, passes); break;
        case GEMV_EPI_SWIGLU: ar_launch((gemv_batched_kernel<WT, NB, GEMV_EPI_SWIGLU>), grid, block, 0, st, p, passes); break;
        case GEMV_EPI_ARGMAX: ar_launch((gemv_batched_kernel<WT, NB, GEMV_EPI_ARGMAX>), grid, block, 0, st, p, passes); break;
        default: ar_set_error("GEMV: unknown epilogue %d", epi); return AR_HIP_ERR_INVALID;
    }
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

}  // namespace

int gemv_launch_batched(const Params& p, int wdtype, int epi, hipStream_t stream) {
    AR_CHECK_ARG(p.batch >= 3 && p.batch <= 8, "batched GEMV: batch %d outside 3..8", p.batch);
    const bool nb4 = p.batch <= 4;
    if (wdtype == AR_DTYPE_BF16) return nb4 ? launch_nb<uint16_t, 4>(p, epi, stream) : launch_nb<uint16_t, 8>(p, epi, stream);
    return nb4 ? launch_nb<float, 4>(p, epi, stream) : launch_nb<float, 8>(p, epi, stream);
}
