// Final RMSNorm + logits GEMV + greedy argmax for batch 1-2 (Qwen3.java:401-405,
// AutoregressiveModel.java:412-421), as a persistent kernel: the largest single launch of a decode
// step (C3: 151,936 x 1,024 fp32 = 622 MB), so it is built to stream at the read bandwidth a plain
// sum over the same bytes reaches (6.5 TB/s measured on MI355X).
//
// A fixed grid of 256-thread blocks (as many as are resident at once) walks the rows: wavefront w
// of the grid takes rows (it * W + w) * RPW .. + RPW - 1 at iteration it.  Every wavefront holds the whole normalised input in registers (lane l
// owns columns k * 64 * VEC + l * VEC .. + VEC - 1 of each chunk k), computed once from x and the
// RMSNorm gain with its own sum of squares, so the loop touches no LDS and has no barrier.  Each
// row's dot product is summed over the lanes on the DPP network, and lane 63 keeps the wavefront's
// best (value, index) -- the first maximum, rows being visited in increasing order per
// wavefront -- and the block adds one packed key per sequence to the greedy-token slots
// (the same keys as the other GEMV argmax epilogues; ties across blocks resolve to the lowest
// index).  The logits themselves are stored when asked.
#include <algorithm>

#include "gemv_impl.h"

namespace {
using namespace gemv;

constexpr int kAmThreads = 256, kAmWaves = kAmThreads / 64;

template <typename WT, int NB, int RPW, int NCH>
__global__ __launch_bounds__(kAmThreads) void gemv_argmax_kernel(Params p) {
    using V = WVec<WT>;
    using raw = typename V::raw;
    constexpr int VEC = V::N, CH = 64 * VEC;
    __shared__ float s_val[kAmWaves][NB];
    __shared__ int s_idx[kAmWaves][NB];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gw = blockIdx.x * kAmWaves + wave, W = gridDim.x * kAmWaves;
    const WT* w = reinterpret_cast<const WT*>(p.w);
    const int cols = p.cols;

    // rows of iteration `it` for this wavefront (clamped: a padding row reloads the last row)
    auto load_rows = [&](int it, raw (&buf)[RPW][NCH]) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int row = min((it * W + gw) * RPW + r, p.rows - 1);
            const WT* wr = w + (size_t)row * cols + lane * VEC;
#pragma unroll
            for (int k = 0; k < NCH; k++) buf[r][k] = *reinterpret_cast<const raw*>(wr + k * CH);
        }
    };
    raw b0[RPW][NCH];
    load_rows(0, b0);

    // the normalised input, in registers: h = (g * x) * r with r = 1 / sqrt(mean(x^2) + eps)
    float h[NB][NCH][VEC];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const float* xb = p.x + (size_t)min(b, p.batch - 1) * p.x_stride;
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < NCH; k++)
#pragma unroll
            for (int j = 0; j < VEC; j += 4) {
                const float4 v = *reinterpret_cast<const float4*>(xb + k * CH + lane * VEC + j);
                h[b][k][j] = v.x; h[b][k][j + 1] = v.y; h[b][k][j + 2] = v.z; h[b][k][j + 3] = v.w;
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        if (p.norm_w) {
            const float rn = 1.0f / sqrtf(wave_sum(ss) / (float)cols + p.eps);
#pragma unroll
            for (int k = 0; k < NCH; k++)
#pragma unroll
                for (int j = 0; j < VEC; j += 4) {
                    const float4 g = *reinterpret_cast<const float4*>(p.norm_w + k * CH + lane * VEC + j);
                    h[b][k][j] = (g.x * h[b][k][j]) * rn;
                    h[b][k][j + 1] = (g.y * h[b][k][j + 1]) * rn;
                    h[b][k][j + 2] = (g.z * h[b][k][j + 2]) * rn;
                    h[b][k][j + 3] = (g.w * h[b][k][j + 3]) * rn;
                }
        }
    }

    float bv[NB];
    int bi[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        bv[b] = -INFINITY;
        bi[b] = 0x7FFFFFFF;
    }
    auto consume = [&](int it, const raw (&buf)[RPW][NCH]) {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            float acc[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) acc[b] = 0.f;
#pragma unroll
            for (int k = 0; k < NCH; k++) {
                float wf[VEC];
                V::unpack(buf[r][k], wf);
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int j = 0; j < VEC; j++) acc[b] = fmaf(wf[j], h[b][k][j], acc[b]);
            }
            const int row = (it * W + gw) * RPW + r;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float v = dpp_sum_lane63(acc[b]);  // meaningful in lane 63 only
                if (lane == 63 && row < p.rows && b < p.batch) {
                    if (p.y) p.y[(size_t)b * p.y_stride + row] = v;
                    if (v > bv[b]) {  // rows ascend within a wavefront: the first maximum stays
                        bv[b] = v;
                        bi[b] = row;
                    }
                }
            }
        }
    };
    // one buffer of rows per wavefront: the other resident wavefronts of the CU keep the memory
    // pipeline full while this one reduces
    const int iters = (p.rows + W * RPW - 1) / (W * RPW);
    for (int it = 0; it < iters; it++) {
        if (it) load_rows(it, b0);
        consume(it, b0);
    }

    if (lane == 63)
#pragma unroll
        for (int b = 0; b < NB; b++) {
            s_val[wave][b] = bv[b];
            s_idx[wave][b] = bi[b];
        }
    __syncthreads();
    if (tid < p.batch && tid < NB) {
        float v = s_val[0][tid];
        int i = s_idx[0][tid];
#pragma unroll
        for (int ww = 1; ww < kAmWaves; ww++)
            if (better(s_val[ww][tid], s_idx[ww][tid], v, i)) {
                v = s_val[ww][tid];
                i = s_idx[ww][tid];
            }
        if (i != 0x7FFFFFFF)
            atomicMax(p.keys + (size_t)tid * kArgmaxSlots + (blockIdx.x & (kArgmaxSlots - 1)), argmax_key(v, i));
    }
}

template <typename WT, int NB, int NCH>
int launch_nch(const Params& p, hipStream_t st) {
    constexpr int RPW = 1;  // one row per wavefront per step measured fastest (C3 logits: 100.9 us vs 101.7-104.3 for 2, 108-110 for 4-8)
    // as many blocks as are resident at once, so every block is running from the start
    // (cached per device: the resident count depends on the device the stream launches to)
    static std::atomic<int> grid_cache[kMaxDevices];
    const int slot = ar_device_slot(st);
    int grid = slot >= 0 ? grid_cache[slot].load(std::memory_order_relaxed) : 0;
    if (!grid) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_argmax_kernel<WT, NB, RPW, NCH>, kAmThreads, 0) !=
                hipSuccess || per_cu < 1)
            per_cu = 2;
        grid = per_cu * ar_device_cus(st);
        if (slot >= 0) grid_cache[slot].store(grid, std::memory_order_relaxed);
    }
    const int g = std::min(grid, (p.rows + kAmWaves * RPW - 1) / (kAmWaves * RPW));
    ar_launch((gemv_argmax_kernel<WT, NB, RPW, NCH>), dim3(g), dim3(kAmThreads), 0, st, p);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

template <typename WT, int NB>
int launch_nb(const Params& p, int nch, hipStream_t st) {
    switch (nch) {
        case 1: return launch_nch<WT, NB, 1>(p, st);
        case 2: return launch_nch<WT, NB, 2>(p, st);
        case 3: return launch_nch<WT, NB, 3>(p, st);
        case 4: return launch_nch<WT, NB, 4>(p, st);
    }
    ar_set_error("argmax GEMV: %d column chunks not supported", nch);
    return AR_HIP_ERR_INVALID;
}

}  // namespace

bool gemv_argmax_fits(int cols, int batch, int wdtype) {
    const int ch = 64 * (wdtype == AR_DTYPE_BF16 ? 8 : 4);
    const int nch = cols / ch;
    return batch >= 1 && batch <= 2 && cols % ch == 0 && nch >= 1 && nch <= 4;
}

int gemv_launch_argmax(const gemv::Params& p, int wdtype, hipStream_t st) {
    const int ch = 64 * (wdtype == AR_DTYPE_BF16 ? 8 : 4);
    const int nch = p.cols / ch;
    if (wdtype == AR_DTYPE_BF16)
        return p.batch == 1 ? launch_nb<uint16_t, 1>(p, nch, st) : launch_nb<uint16_t, 2>(p, nch, st);
    return p.batch == 1 ? launch_nb<float, 1>(p, nch, st) : launch_nb<float, 2>(p, nch, st);
}
