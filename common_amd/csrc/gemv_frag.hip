// Batched decode GEMV over fragment-ordered bf16 weights, 3..8 sequences, on the MFMA units.
//
// Same contract as the MFMA GEMV (gemv_mfma.hip) for the store, residual and SwiGLU epilogues -- the
// reference's dense -> matmul/weightedSum (domain/graph/.../LayerFeatures.java:785-830,
// compute/algebra/.../MatrixFeatures.java:182-337) with the RMSNorm prologue
// (NormalizationLayerFeatures.java:584-595) -- but the weights are read from a copy laid out for
// the matrix cores, and the work is split so that every wavefront streams the same number of bytes.
//
// Fragment order: the 16 x 32 block of rows 16t.. and columns 32k.. is fragment (t, k), stored as
// 64 lanes x 8 bf16 (lane l: row l % 16, columns 8 (l / 16) .. + 7) = 1 KB contiguous, fragments of
// a tile in k order, tiles in row order.  A wavefront's 16-byte load of a fragment is one 1 KB
// burst (row-major 16-row tiles scatter every load over 16 rows, measured 20-35% slower).
//
// Work split: the tiles x (cols / 32) fragments, in tile-major order, are divided evenly over all
// wavefronts of a one-block-per-CU grid (2 wavefronts per block); each streams its range with D
// fragments of loads in flight (8; 6 fragment pairs for SwiGLU).  A tile that lies inside one wavefront's range is finished by that
// wavefront; a tile shared by several (at most the first and the last tile of each range) is
// summed through the workspace: each contributor stores its 16 x 16 partial tile in slot
// (wavefront + tile) and bumps the tile's arrival counter; the last to arrive adds the partials in
// wavefront order (so the sum does not depend on timing) and applies the epilogue.  The partials
// go through agent-scope atomic accesses and the counter is bumped after this wavefront's stores
// have completed, as in the k-split form of gemv_mfma.hip; no wavefront ever waits on another.
//
// Input operand: lanes 0-7 of each 16-lane row of the B fragment take the hi plane of sequences
// 0..7 and lanes 8-15 the lo plane (hi = bf16(v), lo = bf16(v - hi), written by the kernel that
// produced the input), so one v_mfma_f32_16x16x32_bf16 per fragment gives W hi in columns 0-7 and
// W lo in columns 8-15; column s + 8 is added to column s at the end.
//
// RMSNorm prologue: 1/sqrt(mean(x^2) + eps) per sequence scales the finished dot products; the
// sum of squares comes from per-16-row partial sums that the producer of x published (ss_in,
// [cols / 16][16] floats), loaded by every wavefront with its first fragments and added in a fixed
// order at its first epilogue (no block-wide wait).  The residual epilogue publishes the same sums
// of its output (ss_out), for the next normalised GEMV, and its old values are loaded when a
// wavefront starts a tile, not at the tile's end.
#include <algorithm>

#include "gemv_impl.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// wavefronts per block (one block per CU): 2 measured faster than 4 on every C5 projection (QKV
// 12.9 vs 13.7 us, O 11.9 vs 12.9, gate/up 24.6 vs 26.2, down 17.5 vs 19.6: fewer wavefronts share
// each tile) and than 1 (too few loads in flight)
constexpr int kWaves = 2;
constexpr int kSsPerLane = 32;  // RMSNorm inputs of up to 8 * 32 16-row tiles (cols <= 4096)

struct Geo {
    int ns;       // fragments per tile (cols / 32)
    int tiles;    // 16-row tiles
    long long U;  // fragments
    int nwt;      // wavefronts of the grid
    // first and last wavefront whose range holds a fragment of tile t
    __device__ inline void contributors(int t, int& i0, int& i1) const {
        const long long s = (long long)t * ns, e = s + ns - 1;
        i0 = (int)(((s + 1) * nwt - 1) / U);
        i1 = (int)(((e + 1) * nwt - 1) / U);
    }
};

// Epilogue of tile t from its finished (unnormalised) 16 x 16 product(s): lane l holds rows
// 4 (l / 16) + e (e < 4), column l % 16.  Columns 8..15 (the lo plane's products) are added to
// columns 0..7 first; lanes of column s < batch then write rows 16t + 4q .. + 3 of sequence s.
template <int EPI>
__device__ inline void emit(const gemv::Params& p, floatx4 (&v)[EPI == GEMV_EPI_SWIGLU ? 2 : 1], int t, int lane,
                            float rn, float4 old) {
    constexpr int NMAT = EPI == GEMV_EPI_SWIGLU ? 2 : 1;
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int e = 0; e < 4; e++) v[m][e] += __shfl_xor(v[m][e], 8, 64);
    const int s = lane & 15, q = lane >> 4, row0 = t * 16 + 4 * q;
    const bool live = s < 8 && s < p.batch;
    float val[4];
    float* yp = p.y + (size_t)(s & 7) * p.y_stride + row0;
    const float o4[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float g = v[0][e] * rn;
        if (EPI == GEMV_EPI_STORE) {
            val[e] = p.bias ? g + p.bias[row0 + e] : g;
        } else if (EPI == GEMV_EPI_RESIDUAL) {
            val[e] = o4[e] + g;
        } else {  // SwiGLU: u * (g * 1/(exp(-g)+1))
            const float u = v[NMAT - 1][e] * rn;
            const float sg = 1.0f / (expf(-g) + 1.0f);
            val[e] = u * (g * sg);
        }
    }
    if (EPI == GEMV_EPI_RESIDUAL && p.ss_out) {  // per-tile sum of squares of the new residual row
        float s2 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) s2 = fmaf(val[e], val[e], s2);
        s2 += __shfl_xor(s2, 16, 64);
        s2 += __shfl_xor(s2, 32, 64);
        if (live && q == 0) p.ss_out[(size_t)t * 16 + s] = s2;
    }
    if (!live) return;
    *reinterpret_cast<float4*>(yp) = make_float4(val[0], val[1], val[2], val[3]);
    if (p.y_hi) {  // operand planes of the next GEMV's input
        unsigned short hs[4], ls[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint16_t h, l;
            bf16_planes(p.y_gain ? val[e] * p.y_gain[row0 + e] : val[e], &h, &l);
            hs[e] = h;
            ls[e] = l;
        }
        const size_t o = (size_t)s * p.y_stride + row0;
        *reinterpret_cast<uint2*>(p.y_hi + o) = make_uint2(hs[0] | ((unsigned)hs[1] << 16), hs[2] | ((unsigned)hs[3] << 16));
        *reinterpret_cast<uint2*>(p.y_lo + o) = make_uint2(ls[0] | ((unsigned)ls[1] << 16), ls[2] | ((unsigned)ls[3] << 16));
    }
}

template <int NMAT>
__device__ inline void part_store(const gemv::Params& p, int slot, const floatx4 (&acc)[NMAT], int lane) {
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int e = 0; e < 4; e++)
            __hip_atomic_store(p.kpart + ((size_t)slot * NMAT + m) * 256 + e * 64 + lane, acc[m][e], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}

template <int EPI, int D, int NW>
__global__ __launch_bounds__(NW * 64) void gemv_frag_kernel(gemv::Params p) {
    constexpr int NMAT = EPI == GEMV_EPI_SWIGLU ? 2 : 1;
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, q = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wavefront-uniform: scalar loop control
    Geo geo;
    geo.ns = p.cols / 32;
    geo.tiles = p.rows / 16;
    geo.U = (long long)geo.tiles * geo.ns;
    geo.nwt = gridDim.x * NW;
    const int ns = geo.ns;
    const int g = blockIdx.x * NW + w;
    const int a = (int)(geo.U * g / geo.nwt), b = (int)(geo.U * (g + 1) / geo.nwt);  // fragments [a, b)

    // B operand: lane (r, q) holds columns 8q..8q+7 of k-step k from the hi plane of sequence r
    // (r < 8) or the lo plane of sequence r - 8
    const int ps = min(r & 7, p.batch - 1);
    const uint16_t* xp = (r < 8 ? p.x_hi : p.x_lo) + (size_t)ps * p.x_stride + 8 * q;
    const uint16_t* w0 = p.wf + lane * 8;
    const uint16_t* w1 = NMAT == 2 ? p.wf2 + lane * 8 : nullptr;
    u32x4 wv[D][NMAT], xv[D];
    int lk = a % ns, lu = a;  // next fragment to load (k-step lk of its tile); stays at b - 1 past the end
    auto load = [&](int j) {
        wv[j][0] = *reinterpret_cast<const u32x4*>(w0 + (size_t)lu * 512);
        if (NMAT == 2) wv[j][NMAT - 1] = *reinterpret_cast<const u32x4*>(w1 + (size_t)lu * 512);
        xv[j] = *reinterpret_cast<const u32x4*>(xp + lk * 32);
        if (lu + 1 < b) {
            lu++;
            if (++lk == ns) lk = 0;
        }
    };
#pragma unroll
    for (int j = 0; j < D; j++) load(j);

    int ct = a / ns, ck = a % ns;          // tile and k-step of the next fragment multiplied
    // residual epilogue: the old values of a tile's outputs are loaded when the wavefront starts the
    // tile, so they have arrived by its end (loads complete in issue order)
    const int es = lane & 15;
    const bool elive = es < 8 && es < p.batch;
    const float* yrow = p.y + (size_t)(es & 7) * p.y_stride + 4 * q;
    auto load_old = [&](int t) {
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        if (EPI == GEMV_EPI_RESIDUAL && elive) o = *reinterpret_cast<const float4*>(yrow + t * 16);
        return o;
    };
    float4 old_cur = load_old(ct), old_first = make_float4(0.f, 0.f, 0.f, 0.f);
    // RMSNorm: the producer's per-16-row sums of squares of sequence lane % 8, entries lane / 8 + 8 i,
    // loaded now and reduced (in a fixed order) at the first epilogue
    float ssv[kSsPerLane];
    const int nt = p.cols / 16;
    if (p.norm_w) {
#pragma unroll
        for (int i = 0; i < kSsPerLane; i++) {
            const int t = (lane >> 3) + 8 * i;
            ssv[i] = (t < nt && (lane & 7) < p.batch) ? p.ss_in[(size_t)t * 16 + (lane & 7)] : 0.f;
        }
    }
    float rn = 1.0f;
    bool rn_done = p.norm_w == nullptr;
    auto norm_factor = [&]() {
        if (!rn_done) {
            float tot = 0.f;
#pragma unroll
            for (int i = 0; i < kSsPerLane; i++) tot += ssv[i];
            tot += __shfl_xor(tot, 8, 64);
            tot += __shfl_xor(tot, 16, 64);
            tot += __shfl_xor(tot, 32, 64);
            rn = 1.0f / sqrtf(tot / (float)p.cols + p.eps);
            rn_done = true;
        }
        return rn;
    };

    const bool first_partial = ck != 0;    // the range starts inside a tile
    int t_first = -1;                      // that tile, once its part is complete (held in acc_first)
    floatx4 acc[NMAT], acc_first[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) acc[m] = acc_first[m] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto step = [&](int j) {
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv[j][m]),
                                                             __builtin_bit_cast(bf16x8, xv[j]), acc[m], 0, 0, 0);
        if (++ck == ns) {  // end of tile ct
            if (first_partial && t_first < 0) {
                t_first = ct;
                old_first = old_cur;
#pragma unroll
                for (int m = 0; m < NMAT; m++) acc_first[m] = acc[m];
            } else {
                emit<EPI>(p, acc, ct, lane, norm_factor(), old_cur);
            }
#pragma unroll
            for (int m = 0; m < NMAT; m++) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
            ck = 0;
            ct++;
            if (ct < geo.tiles) old_cur = load_old(ct);
        }
    };
    int base = a;
    for (; base + D <= b; base += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            step(j);
            load(j);
        }
    }
#pragma unroll
    for (int j = 0; j < D; j++)
        if (base + j < b) step(j);

    // shared tiles: the first (complete part held in acc_first) and the last (range ends inside it)
    const bool last_partial = ck > 0;
    if (t_first >= 0) part_store<NMAT>(p, g + t_first, acc_first, lane);
    if (last_partial) part_store<NMAT>(p, g + ct, acc, lane);
    if (t_first < 0 && !last_partial) return;
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial stores have completed
    auto fold = [&](int t, float4 old) {
        int i0, i1;
        geo.contributors(t, i0, i1);
        unsigned prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(p.kcount + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __shfl(prev, 0, 64);
        if (prev != (unsigned)(i1 - i0)) return;  // not the last contributor
        if (lane == 0) __hip_atomic_store(p.kcount + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        floatx4 v[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; m++) v[m] = floatx4{0.f, 0.f, 0.f, 0.f};
        for (int i = i0; i <= i1; i += 4) {  // four contributors' loads in flight together
            float tmp[4][NMAT][4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int ii = min(i + jj, i1);
#pragma unroll
                for (int m = 0; m < NMAT; m++)
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        tmp[jj][m][e] = __hip_atomic_load(p.kpart + ((size_t)(ii + t) * NMAT + m) * 256 + e * 64 + lane,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                if (i + jj <= i1)
#pragma unroll
                    for (int m = 0; m < NMAT; m++)
#pragma unroll
                        for (int e = 0; e < 4; e++) v[m][e] += tmp[jj][m][e];
        }
        emit<EPI>(p, v, t, lane, norm_factor(), old);
    };
    if (t_first >= 0) fold(t_first, old_first);
    if (last_partial) fold(ct, old_cur);
}

// row-major bf16 (rows x cols) -> fragment order; rows past the end of the last tile are zero
__global__ void frag_copy_kernel(const uint16_t* w, uint16_t* out, int rows, int cols) {
    const int ns = cols / 32, tiles = (rows + 15) / 16;
    const size_t lanes = (size_t)tiles * ns * 64;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < lanes; i += (size_t)gridDim.x * blockDim.x) {
        const size_t f = i / 64;
        const int l = (int)(i % 64), t = (int)(f / ns), k = (int)(f % ns);
        const int row = t * 16 + (l & 15);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < rows) v = *reinterpret_cast<const u32x4*>(w + (size_t)row * cols + k * 32 + 8 * (l >> 4));
        *reinterpret_cast<u32x4*>(out + i * 8) = v;
    }
}

template <int EPI, int D>
int launch_epi(const gemv::Params& p, int grid, hipStream_t st) {
    ar_launch((gemv_frag_kernel<EPI, D, kWaves>), dim3(grid), dim3(kWaves * 64), 0, st, p);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

}  // namespace

size_t gemv_frag_elems(int rows, int cols) { return (size_t)((rows + 15) / 16) * 16 * cols; }

size_t gemv_frag_part_floats(int rows, int cus, int nmat) {
    return ((size_t)cus * kWaves + (rows + 15) / 16) * nmat * 256;
}

bool gemv_frag_fits(int rows, int cols, int batch, int cus) {
    return batch >= 1 && batch <= 8 && rows % 16 == 0 && cols % 32 == 0 &&
           (long long)(rows / 16) * (cols / 32) >= (long long)cus * kWaves && (long long)(rows / 16) * (cols / 32) < (1ll << 31);
}

int launch_frag_copy(const uint16_t* w, uint16_t* out, int rows, int cols, hipStream_t st) {
    AR_CHECK_ARG(w && out && rows > 0 && cols > 0 && cols % 32 == 0, "fragment copy: bad arguments");
    hipLaunchKernelGGL(frag_copy_kernel, dim3(2048), dim3(256), 0, st, w, out, rows, cols);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int gemv_launch_frag(const gemv::Params& p, int epi, hipStream_t st) {
    const int cus = ar_device_cus(st);
    AR_CHECK_ARG(gemv_frag_fits(p.rows, p.cols, p.batch, cus), "fragment GEMV: shape %dx%d / batch %d unsupported",
                 p.rows, p.cols, p.batch);
    AR_CHECK_ARG(p.wf && (epi != GEMV_EPI_SWIGLU || p.wf2), "fragment GEMV: missing fragment-ordered weights");
    AR_CHECK_ARG(p.x_hi && p.x_lo, "fragment GEMV: needs the input's operand planes");
    AR_CHECK_ARG(!p.norm_w || (p.ss_in && p.cols / 16 <= 8 * kSsPerLane),
                 "fragment GEMV: RMSNorm needs the input's per-tile sums of squares (cols <= %d)", 128 * kSsPerLane);
    AR_CHECK_ARG(p.y && p.y_stride % 4 == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0,
                 "fragment GEMV: output must be 16-byte aligned rows");
    AR_CHECK_ARG(epi == GEMV_EPI_STORE || epi == GEMV_EPI_RESIDUAL || epi == GEMV_EPI_SWIGLU,
                 "fragment GEMV: epilogue %d unsupported", epi);
    const int nmat = epi == GEMV_EPI_SWIGLU ? 2 : 1;
    AR_CHECK_ARG(p.kpart && p.kcount && (size_t)p.kpart_floats >= gemv_frag_part_floats(p.rows, cus, nmat) &&
                     p.kcount_n >= p.rows / 16,
                 "fragment GEMV: workspace too small");
    switch (epi) {
        case GEMV_EPI_STORE: return launch_epi<GEMV_EPI_STORE, 8>(p, cus, st);
        case GEMV_EPI_RESIDUAL: return launch_epi<GEMV_EPI_RESIDUAL, 8>(p, cus, st);
        default: return launch_epi<GEMV_EPI_SWIGLU, 6>(p, cus, st);
    }
}
