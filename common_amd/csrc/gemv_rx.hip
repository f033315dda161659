// Batch-1 decode GEMV with the input vector held in registers: y = W x (+ epilogue).
//
// Same contract as the LDS-staged kernel in gemv_impl.h (the reference's dense -> matmul /
// weightedSum, domain/graph/.../LayerFeatures.java:785-830, compute/algebra/.../MatrixFeatures.java:
// 182-337, with the RMSNorm prologue of NormalizationLayerFeatures.java:584-595 and the store /
// residual / SwiGLU epilogues).  The per-layer decode GEMVs of a 0.6B-4B model read 8-25 MB each and
// run at a few microseconds, where the fixed cost of the kernel matters as much as the streaming:
// the LDS-staged kernel spends ~1.5-2 us per launch above a plain streaming kernel over the same
// bytes (block-wide input staging, two barriers, LDS reads).  Here instead:
//  * one wavefront owns NR weight rows (a gate/up row pair for SwiGLU) over the whole input width
//    and issues all NR x nch 16-byte weight loads at once;
//  * each lane loads the input slices matching its weight columns straight into registers, and
//    the residual value of its output row, before the weight loads (loads return in issue order,
//    so the input is ready first and the RMSNorm sum of squares overlaps the weight stream);
//  * the RMSNorm factor is computed per wavefront from the same registers (the whole row is
//    covered, so no block-wide reduction) and applied to the finished dot product;
//  * no LDS and no barrier; each row (and the sum of squares) is summed over the lanes on the DPP
//    network into lane 63, which applies the epilogue and stores.
// Shapes: cols a multiple of the 64-lane chunk (256 fp32 / 512 bf16 columns), at most 16 fp32 or
// 12 bf16 chunks (8 with the RMSNorm prologue).
#include "gemv_impl.h"

namespace {

using gemv::Params;
using gemv::WVec;

constexpr int kRxWaves = 4;
constexpr int kRxMaxChunks = 16;  // 64-lane chunks per row: 4096 fp32 / 8192 bf16 columns

template <typename WT, int NR, int NCH, int EPI>
__global__ __launch_bounds__(kRxWaves * 64) void gemv_rx_kernel(Params p, int nch) {
    using V = WVec<WT>;
    constexpr int VEC = V::N;
    constexpr int CH = 64 * VEC;
    constexpr int NM = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    constexpr int RW = NR / NM;  // output rows per wavefront
    static_assert(NR % NM == 0, "SwiGLU streams row pairs");

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * kRxWaves + wave) * RW;
    const bool norm = p.norm_w != nullptr;

    float res[RW];  // residual epilogue: lane 63 (which finishes the row sums) holds the old rows
#pragma unroll
    for (int r = 0; r < RW; r++)
        res[r] = (EPI == GEMV_EPI_RESIDUAL && lane == 63 && row0 + r < p.rows) ? p.y[row0 + r] : 0.f;

    // input (and gain) slices of this lane: VEC values at column c * CH + lane * VEC
    float xv[NCH][VEC];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int cc = min(c, nch - 1);
#pragma unroll
        for (int j = 0; j < VEC; j += 4) {
            const float4 t = *reinterpret_cast<const float4*>(p.x + cc * CH + lane * VEC + j);
            xv[c][j] = t.x; xv[c][j + 1] = t.y; xv[c][j + 2] = t.z; xv[c][j + 3] = t.w;
        }
    }
    float gv[NCH][VEC];
    if (norm) {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int cc = min(c, nch - 1);
#pragma unroll
            for (int j = 0; j < VEC; j += 4) {
                const float4 t = *reinterpret_cast<const float4*>(p.norm_w + cc * CH + lane * VEC + j);
                gv[c][j] = t.x; gv[c][j + 1] = t.y; gv[c][j + 2] = t.z; gv[c][j + 3] = t.w;
            }
        }
    }

    const WT* wr[NR];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int row = min(row0 + r, p.rows - 1);
        wr[r] = reinterpret_cast<const WT*>(p.w) + (size_t)row * p.cols + lane * VEC;
        if (NM == 2) wr[RW + r] = reinterpret_cast<const WT*>(p.w2) + (size_t)row * p.cols + lane * VEC;
    }
    typename V::raw wv[NR][NCH];
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int cc = min(c, nch - 1);  // chunks past the row end re-read the last one (cache hit)
#pragma unroll
        for (int r = 0; r < NR; r++) wv[r][c] = *reinterpret_cast<const typename V::raw*>(wr[r] + cc * CH);
    }

    float rn = 1.0f;
    if (norm) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < NCH; c++)
            if (c < nch) {
#pragma unroll
                for (int j = 0; j < VEC; j++) {
                    ss = fmaf(xv[c][j], xv[c][j], ss);
                    xv[c][j] *= gv[c][j];
                }
            }
        ss = gemv::dpp_sum_lane63(ss);  // lane 63 alone finishes and stores the rows
        rn = 1.0f / sqrtf(ss / (float)p.cols + p.eps);
    }

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        float a = 0.f;
#pragma unroll
        for (int c = 0; c < NCH; c++)
            if (c < nch) {
                float wf[VEC];
                V::unpack(wv[r][c], wf);
#pragma unroll
                for (int j = 0; j < VEC; j++) a = fmaf(wf[j], xv[c][j], a);
            }
        acc[r] = gemv::dpp_sum_lane63(a) * rn;  // meaningful in lane 63 only
    }

#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int row = row0 + r;
        if (lane == 63 && row < p.rows) {
            float* yp = p.y + row;
            if (EPI == GEMV_EPI_STORE) {
                *yp = p.bias ? acc[r] + p.bias[row] : acc[r];
            } else if (EPI == GEMV_EPI_RESIDUAL) {
                *yp = res[r] + acc[r];
            } else {  // SwiGLU: acc[r] = gate, acc[RW + r] = up
                const float g = acc[r];
                const float sg = 1.0f / (expf(-g) + 1.0f);
                *yp = acc[(NM == 2) ? RW + r : r] * (g * sg);
            }
        }
    }
}

template <typename WT, int NR, int NCH>
int launch_nch(const Params& p, int epi, int nch, hipStream_t st) {
    const int rw = (epi == GEMV_EPI_SWIGLU) ? NR / 2 : NR;
    const dim3 grid((p.rows + kRxWaves * rw - 1) / (kRxWaves * rw)), block(kRxWaves * 64);
    switch (epi) {
        case GEMV_EPI_STORE: ar_launch((gemv_rx_kernel<WT, NR, NCH, GEMV_EPI_STORE>), grid, block, 0, st, p, nch); break;
        case GEMV_EPI_RESIDUAL: ar_launch((gemv_rx_kernel<WT, NR, NCH, GEMV_EPI_RESIDUAL>), grid, block, 0, st, p, nch); break;
        case GEMV_EPI_SWIGLU:
            if constexpr (NR % 2 == 0) {
                ar_launch((gemv_rx_kernel<WT, NR, NCH, GEMV_EPI_SWIGLU>), grid, block, 0, st, p, nch);
                break;
            }
            ar_set_error("register-input GEMV: SwiGLU needs a row pair per wavefront");
            return AR_HIP_ERR_INVALID;
        default: ar_set_error("register-input GEMV: epilogue %d not supported", epi); return AR_HIP_ERR_INVALID;
    }
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

template <typename WT, int NR>
int launch_nr(const Params& p, int epi, int nch, hipStream_t st) {
    if (nch <= 2) return launch_nch<WT, NR, 2>(p, epi, nch, st);
    if (nch <= 4) return launch_nch<WT, NR, 4>(p, epi, nch, st);
    if (nch <= 8) return launch_nch<WT, NR, 8>(p, epi, nch, st);
    if constexpr (sizeof(WT) == 4) {
        if (nch <= 12) return launch_nch<WT, NR, 12>(p, epi, nch, st);
        return launch_nch<WT, NR, 16>(p, epi, nch, st);
    } else {
        return launch_nch<WT, NR, 12>(p, epi, nch, st);
    }
}

}  // namespace

bool gemv_rx_fits(int rows, int cols, int batch, int wdtype, int epi, bool norm) {
    const int ch = 64 * (wdtype == AR_DTYPE_BF16 ? 8 : 4);
    // bf16 chunks hold 8 inputs per lane: 12 chunks without the RMSNorm gain, 8 with it, keep the
    // input, gain and weight registers of a row pair within the register file
    const int max_chunks = wdtype == AR_DTYPE_BF16 ? (norm ? 8 : 12) : kRxMaxChunks;
    return batch == 1 && rows > 0 && epi != GEMV_EPI_ARGMAX && cols % ch == 0 && cols / ch >= 1 &&
           cols / ch <= max_chunks;
}

int gemv_launch_rx(const Params& p, int wdtype, int epi, hipStream_t st) {
    AR_CHECK_ARG(gemv_rx_fits(p.rows, p.cols, p.batch, wdtype, epi, p.norm_w != nullptr), "register-input GEMV: shape %dx%d batch %d outside its range",
                 p.rows, p.cols, p.batch);
    const int ch = 64 * (wdtype == AR_DTYPE_BF16 ? 8 : 4);
    const int nch = p.cols / ch;
    // two rows per wavefront (a row pair for SwiGLU) while that keeps <= 8 loads per lane in flight
    // and leaves >= 4 wavefronts per CU at 256 CUs; one otherwise (swept on the 0.6B decode shapes:
    // 4096 x 1024 fp32 5.19 vs 5.36 us, 1024 x 2048 one row 3.43 us)
    const bool two = epi == GEMV_EPI_SWIGLU || (nch <= 4 && p.rows >= 4096);
    if (wdtype == AR_DTYPE_BF16)
        return two ? launch_nr<uint16_t, 2>(p, epi, nch, st) : launch_nr<uint16_t, 1>(p, epi, nch, st);
    return two ? launch_nr<float, 2>(p, epi, nch, st) : launch_nr<float, 1>(p, epi, nch, st);
}
