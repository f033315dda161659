// Batched decode GEMV on the MFMA units: bf16 weights, 3..16 sequences.
//
// Same contract as the batch-1/2 GEMV (gemv_impl.h): the reference's dense -> matmul/weightedSum
// (domain/graph/.../LayerFeatures.java:785-830, compute/algebra/.../MatrixFeatures.java:182-337)
// with the RMSNorm prologue (NormalizationLayerFeatures.java:584-595) and the store / residual /
// SwiGLU / greedy-argmax epilogues.  With 8 sequences each weight element feeds 8 multiply-adds,
// which on the vector ALUs (fp32, 16 FMA lanes per SIMD per clock) costs about as much time as
// streaming the weight from HBM; the matrix cores take that work off the critical path.
//
// Product: one v_mfma_f32_16x16x32_bf16 per operand plane and 32-wide k-step.  A = 16 weight rows
// (lane l supplies row l%16, k = (l/16)*8 .. +7: one 16-byte load straight from the row-major bf16
// matrix); B = the batch as 16 columns (lane l supplies sequence l%16 at the same k; columns past
// the batch are 0).  The fp32 input is gain-scaled and split into bf16 planes hi = bf16(v),
// lo = bf16(v - hi), so hi + lo keeps 16 significant bits and the products accumulate in fp32.
// RMSNorm's 1/sqrt(mean(x^2) + eps) is a per-sequence scalar: the lanes accumulate sum(x^2) from
// the same loads and the factor scales the finished dot products.
//
// A block's wavefronts split the k-steps of a 16-row tile (a gate tile and an up tile for SwiGLU)
// and sum their 16 x 16 partial tiles through LDS in a fixed order.  Two forms:
//  * persistent (up to 16 k-steps per wavefront, 12 for SwiGLU: cols <= 4096 / 3072): one
//    block per CU loops over tiles; each wavefront converts its slice of every input once and keeps
//    the planes in registers for all tiles; the next tile's weight loads are issued before the
//    current tile's reduction, so they overlap it;
//  * streaming (wider inputs, or fewer tiles than CUs): one tile per 16-wavefront block; each
//    chunk of k-steps issues its weight and input loads together, and the next chunk's loads are in
//    flight while the current chunk is converted and multiplied.
#include <algorithm>

#include "gemv_impl.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPersistWaves = 8;
constexpr int kStreamWaves = 16;
constexpr int kStreamChunk = 2;  // k-steps per load chunk (two chunks in flight)
constexpr int kMaxKSplit = 4;    // k-slices per tile in the split streaming form

__device__ inline unsigned bf16_bits(float f) {  // round to nearest even; NaN stays NaN
    unsigned u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// 8 consecutive inputs of one sequence: gain applied when gp is given (sum of squares of the raw
// values added to ss), then split into hi and lo planes as MFMA B fragments.
__device__ inline void make_planes(float4 a, float4 b, const float* gp, float& ss, u32x4& hi, u32x4& lo) {
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (gp) {
        const float4 ga = *reinterpret_cast<const float4*>(gp);
        const float4 gb = *reinterpret_cast<const float4*>(gp + 4);
        const float g[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            ss = fmaf(v[j], v[j], ss);
            v[j] *= g[j];
        }
    }
    unsigned h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const unsigned h0 = bf16_bits(v[2 * j]), h1 = bf16_bits(v[2 * j + 1]);
        h[j] = h0 | (h1 << 16);
        l[j] = bf16_bits(v[2 * j] - __uint_as_float(h0 << 16)) |
               (bf16_bits(v[2 * j + 1] - __uint_as_float(h1 << 16)) << 16);
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
}

// sum of squares of 8 inputs added to ss, in the order make_planes adds them
__device__ inline void sumsq8(float4 a, float4 b, float& ss) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; j++) ss = fmaf(v[j], v[j], ss);
}

__device__ inline float4 load4(const float* p, bool live) {
    return live ? *reinterpret_cast<const float4*>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
}

__device__ inline floatx4 mac2(const u32x4& w, const u32x4& hi, const u32x4& lo, floatx4 acc) {
    const bf16x8 a = __builtin_bit_cast(bf16x8, w);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, hi), acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, lo), acc, 0, 0, 0);
}

// Sums the per-wavefront partial tiles and applies the epilogue to output (row0 + t/16, sequence
// t%16) for threads t < 256, after the partials are in LDS.  For the argmax epilogue the values go
// to `tot`, and after a barrier one thread per sequence scans the tile's 16 rows.
template <int NW, int NMAT, int EPI>
struct Finish {
    __device__ static inline void sum(float (*cpart)[NMAT][256], int tid, float (&v)[NMAT]) {
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) t += cpart[w][m][tid];
            v[m] = t;
        }
    }
    __device__ static inline void outputs(const gemv::Params& p, float (*cpart)[NMAT][256], float (*ssw)[16],
                                          bool norm, int row0, int tid, float* tot) {
        if (tid >= 256) return;
        const int b = tid & 15;
        float v[NMAT];
        sum(cpart, tid, v);
        if (norm) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) s += ssw[w][b];
            const float rn = 1.0f / sqrtf(s / (float)p.cols + p.eps);
#pragma unroll
            for (int m = 0; m < NMAT; m++) v[m] *= rn;
        }
        emit(p, v, row0, tid, tot);
    }
    // epilogue of output (row0 + tid/16, sequence tid%16) given its finished dot products
    __device__ static inline void emit(const gemv::Params& p, float (&v)[NMAT], int row0, int tid, float* tot) {
        const int ri = tid >> 4, b = tid & 15, row = row0 + ri;
        const bool out = row < p.rows && b < p.batch;
        if (EPI == GEMV_EPI_ARGMAX) {
            if (p.y && out) p.y[(size_t)b * p.y_stride + row] = v[0];
            tot[tid] = v[0];
            return;
        }
        if (!out) return;
        float* yp = p.y + (size_t)b * p.y_stride + row;
        float val;
        if (EPI == GEMV_EPI_STORE) {
            val = p.bias ? v[0] + p.bias[row] : v[0];
        } else if (EPI == GEMV_EPI_RESIDUAL) {
            val = *yp + v[0];
        } else {  // SwiGLU: u * (g * 1/(exp(-g)+1))
            const float g = v[0], u = v[NMAT - 1];
            const float sg = 1.0f / (expf(-g) + 1.0f);
            val = u * (g * sg);
        }
        *yp = val;
        if (p.y_hi) {  // operand planes of the next GEMV's input
            const size_t o = (size_t)b * p.y_stride + row;
            bf16_planes(p.y_gain ? val * p.y_gain[row] : val, p.y_hi + o, p.y_lo + o);
        }
    }
    __device__ static inline void argmax(const gemv::Params& p, const float* tot, int row0, int tile, int tid) {
        if (tid >= p.batch) return;
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int i = 0; i < 16; i++) {
            const int rr = row0 + i;
            if (rr < p.rows && gemv::better(tot[i * 16 + tid], rr, bv, bi)) {
                bv = tot[i * 16 + tid];
                bi = rr;
            }
        }
        if (bi != 0x7FFFFFFF)
            atomicMax(p.keys + (size_t)tid * kArgmaxSlots + (tile & (kArgmaxSlots - 1)), gemv::argmax_key(bv, bi));
    }
};

// KS: k-steps per wavefront whose planes stay in registers (>= kpw)
template <int EPI, int KS>
__global__ __launch_bounds__(kPersistWaves * 64) void gemv_mfma_persist_kernel(gemv::Params p, int kpw, int tiles) {
    constexpr int NW = kPersistWaves, NMAT = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    using F = Finish<NW, NMAT, EPI>;
    __shared__ float cpart[NW][NMAT][256];
    __shared__ float ssw[NW][16];
    __shared__ float tot[256];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, q = lane >> 4;
    const int nsteps = p.cols / 32;
    const int s0 = w * kpw, ns = max(0, min(kpw, nsteps - s0));  // this wavefront's k-steps
    const bool live = r < p.batch;
    const bool norm = p.norm_w != nullptr;

    const uint16_t* wbase[NMAT];
    wbase[0] = reinterpret_cast<const uint16_t*>(p.w) + (size_t)s0 * 32 + 8 * q;
    if (NMAT == 2) wbase[NMAT - 1] = reinterpret_cast<const uint16_t*>(p.w2) + (size_t)s0 * 32 + 8 * q;
    u32x4 wv[NMAT][KS];
#define AR_MFMA_LOAD_TILE(t_)                                                                         \
    do {                                                                                              \
        const size_t ro = (size_t)min((t_) * 16 + r, p.rows - 1) * p.cols;                            \
        _Pragma("unroll") for (int i = 0; i < KS; i++) if (i < ns) _Pragma("unroll") for (int m = 0; \
                                                                                         m < NMAT;   \
                                                                                         m++)        \
            wv[m][i] = *reinterpret_cast<const u32x4*>(wbase[m] + ro + i * 32);                       \
    } while (0)
    int t = blockIdx.x;
    if (t < tiles) AR_MFMA_LOAD_TILE(t);  // weights do not depend on x: their latency overlaps the planes
    // input planes of this wavefront's k-steps, once for all tiles: read as written by the kernel
    // that produced the input (the RMSNorm sum of squares still comes from the fp32 input), or
    // converted here
    u32x4 hv[KS], lv[KS];
    float ss = 0.f;
    {
        const float* xp = p.x + (size_t)min(r, p.batch - 1) * p.x_stride + (size_t)s0 * 32 + 8 * q;
        if (p.x_hi) {
            const size_t po = (size_t)min(r, p.batch - 1) * p.x_stride + (size_t)s0 * 32 + 8 * q;
            const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int i = 0; i < KS; i++)
                if (i < ns) {
                    hv[i] = live ? *reinterpret_cast<const u32x4*>(p.x_hi + po + i * 32) : zero;
                    lv[i] = live ? *reinterpret_cast<const u32x4*>(p.x_lo + po + i * 32) : zero;
                }
            if (norm) {
#pragma unroll
                for (int i = 0; i < KS; i++)
                    if (i < ns) sumsq8(load4(xp + i * 32, live), load4(xp + i * 32 + 4, live), ss);
            }
        } else {
            const float* gp = norm ? p.norm_w + (size_t)s0 * 32 + 8 * q : nullptr;
#pragma unroll
            for (int i = 0; i < KS; i++)
                if (i < ns)
                    make_planes(load4(xp + i * 32, live), load4(xp + i * 32 + 4, live), gp ? gp + i * 32 : nullptr,
                                ss, hv[i], lv[i]);
        }
    }
    if (norm) {
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (q == 0) ssw[w][r] = ss;
    }

    for (; t < tiles; t += gridDim.x) {
        floatx4 acc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; m++) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < KS; i++)
            if (i < ns)
#pragma unroll
                for (int m = 0; m < NMAT; m++) acc[m] = mac2(wv[m][i], hv[i], lv[i], acc[m]);
        if (t + (int)gridDim.x < tiles) AR_MFMA_LOAD_TILE(t + (int)gridDim.x);  // in flight during the reduction
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
            for (int j = 0; j < 4; j++) cpart[w][m][(4 * q + j) * 16 + r] = acc[m][j];
        __syncthreads();
        F::outputs(p, cpart, ssw, norm, t * 16, tid, tot);
        if (EPI == GEMV_EPI_ARGMAX) {
            __syncthreads();
            F::argmax(p, tot, t * 16, t, tid);
        }
        __syncthreads();  // cpart / tot are rewritten by the next tile
    }
#undef AR_MFMA_LOAD_TILE
}

// NWS wavefronts per block; ks blocks per 16-row tile (block = tile * ks + k-slice), each taking
// a contiguous share of the k-steps.  With ks > 1 the blocks store their partial tiles in the
// workspace and the last one to arrive adds the ks partials in k-slice order and applies the
// epilogue (partials through agent-scope atomic accesses, as the attention merge would need; no
// device-wide fence).
template <int EPI, int NWS>
__global__ __launch_bounds__(NWS * 64, NWS == 8 ? 4 : 1) void gemv_mfma_stream_kernel(gemv::Params p, int kpw, int ks) {
    constexpr int NW = NWS, NMAT = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1, KC = kStreamChunk;
    using F = Finish<NW, NMAT, EPI>;
    __shared__ float cpart[NW][NMAT][256];
    __shared__ float ssw[NW][16];
    __shared__ float tot[256];
    __shared__ int last_s;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 15, q = lane >> 4;
    const int tile = blockIdx.x / ks, kh = blockIdx.x - tile * ks;
    const int row0 = tile * 16;
    const int nsteps = p.cols / 32;
    const int per = (nsteps + ks - 1) / ks;  // k-steps of this block: [kh*per, min((kh+1)*per, nsteps))
    const int kend = min((kh + 1) * per, nsteps);
    const int s0 = kh * per + w * kpw, s1 = min(s0 + kpw, kend);
    const bool live = r < p.batch;
    const bool norm = p.norm_w != nullptr;
    const size_t wrow = (size_t)min(row0 + r, p.rows - 1) * p.cols + 8 * q;
    const uint16_t* wa = reinterpret_cast<const uint16_t*>(p.w) + wrow;
    const uint16_t* wb = NMAT == 2 ? reinterpret_cast<const uint16_t*>(p.w2) + wrow : nullptr;
    const float* xp = p.x + (size_t)min(r, p.batch - 1) * p.x_stride + 8 * q;
    const float* gp = norm ? p.norm_w + 8 * q : nullptr;

    floatx4 acc[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) acc[m] = floatx4{0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
    // two chunk buffers: the next chunk's loads are in flight while the current one is multiplied
    u32x4 wv[2][NMAT][KC];
    float4 xa[2][KC], xb[2][KC];
    u32x4 ph[2][KC], pl[2][KC];  // operand planes read as written by the input's producer
    const bool planes = p.x_hi != nullptr;
    const uint16_t* phs = planes ? p.x_hi + (size_t)min(r, p.batch - 1) * p.x_stride + 8 * q : nullptr;
    const uint16_t* pls = planes ? p.x_lo + (size_t)min(r, p.batch - 1) * p.x_stride + 8 * q : nullptr;
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
#define AR_MFMA_LOAD_CHUNK(buf_, sb_)                                                    \
    _Pragma("unroll") for (int i = 0; i < KC; i++) {                                     \
        const int k = min((sb_) + i, s1 - 1) * 32;                                       \
        wv[buf_][0][i] = *reinterpret_cast<const u32x4*>(wa + k);                        \
        if (NMAT == 2) wv[buf_][NMAT - 1][i] = *reinterpret_cast<const u32x4*>(wb + k);  \
        if (planes) {                                                                    \
            ph[buf_][i] = live ? *reinterpret_cast<const u32x4*>(phs + k) : zero4;       \
            pl[buf_][i] = live ? *reinterpret_cast<const u32x4*>(pls + k) : zero4;       \
        }                                                                                \
        if (!planes || norm) {                                                           \
            xa[buf_][i] = load4(xp + k, live);                                           \
            xb[buf_][i] = load4(xp + k + 4, live);                                       \
        }                                                                                \
    }
#define AR_MFMA_MUL_CHUNK(buf_, sb_)                                                                     \
    _Pragma("unroll") for (int i = 0; i < KC; i++) {                                                     \
        if ((sb_) + i < s1) { /* uniform over the wavefront */                                           \
            u32x4 hi, lo;                                                                                \
            if (planes) {                                                                                \
                hi = ph[buf_][i];                                                                        \
                lo = pl[buf_][i];                                                                        \
                if (norm) sumsq8(xa[buf_][i], xb[buf_][i], ss);                                         \
            } else {                                                                                     \
                make_planes(xa[buf_][i], xb[buf_][i], gp ? gp + ((sb_) + i) * 32 : nullptr, ss, hi, lo); \
            }                                                                                            \
            _Pragma("unroll") for (int m = 0; m < NMAT; m++) acc[m] = mac2(wv[buf_][m][i], hi, lo, acc[m]); \
        }                                                                                                \
    }
    if (s0 < s1) AR_MFMA_LOAD_CHUNK(0, s0)
    for (int sb = s0; sb < s1; sb += 2 * KC) {
        if (sb + KC < s1) AR_MFMA_LOAD_CHUNK(1, sb + KC)
        AR_MFMA_MUL_CHUNK(0, sb)
        if (sb + 2 * KC < s1) AR_MFMA_LOAD_CHUNK(0, sb + 2 * KC)
        if (sb + KC < s1) AR_MFMA_MUL_CHUNK(1, sb + KC)
    }
#undef AR_MFMA_LOAD_CHUNK
#undef AR_MFMA_MUL_CHUNK
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int j = 0; j < 4; j++) cpart[w][m][(4 * q + j) * 16 + r] = acc[m][j];
    if (norm) {
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (q == 0) ssw[w][r] = ss;
    }
    __syncthreads();
    if (ks == 1) {
        F::outputs(p, cpart, ssw, norm, row0, tid, tot);
        if (EPI == GEMV_EPI_ARGMAX) {
            __syncthreads();
            F::argmax(p, tot, row0, tile, tid);
        }
        return;
    }
    // k-split (no RMSNorm, no argmax): partial tile -> workspace; the last block of the tile folds
    float v[NMAT];
    if (tid < 256) {
        F::sum(cpart, tid, v);
#pragma unroll
        for (int m = 0; m < NMAT; m++)
            __hip_atomic_store(p.kpart + ((size_t)blockIdx.x * NMAT + m) * 256 + tid, v[m], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
    __syncthreads();
    if (tid == 0) {
        unsigned* c = p.kcount + tile;
        const unsigned prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == (unsigned)(ks - 1);
        if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_s = last;
    }
    __syncthreads();
    if (!last_s || tid >= 256) return;
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        float t = 0.f;
        for (int j = 0; j < ks; j++)
            t += __hip_atomic_load(p.kpart + ((size_t)(tile * ks + j) * NMAT + m) * 256 + tid, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        v[m] = t;
    }
    F::emit(p, v, row0, tid, tot);
}


template <int EPI>
int launch_epi(const gemv::Params& p, hipStream_t st) {
    constexpr int NMAT = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    const int nsteps = p.cols / 32, tiles = (p.rows + 15) / 16;
    const int kpw_p = (nsteps + kPersistWaves - 1) / kPersistWaves;
    const int persist = ar_device_cus(st);  // one persistent block per CU of the stream's device
    // register budget of the persistent form: planes 8*KS + weights 4*NMAT*KS
    const int ks_max = NMAT == 2 ? 12 : 16;
    // fewer tiles than CUs (the 2560-row projections at C5): one tile per 16-wavefront block spreads
    // the loads over more wavefronts (measured: O 4096 -> 2560 15.5 us streaming vs 23.7 persistent;
    // QKV 2560 -> 6144 20.3 us persistent vs 25.6 streaming)
    if (kpw_p <= ks_max && tiles >= persist) {
        const dim3 grid(std::min(tiles, persist)), block(64 * kPersistWaves);
        if (kpw_p <= 4)
            ar_launch((gemv_mfma_persist_kernel<EPI, 4>), grid, block, 0, st, p, kpw_p, tiles);
        else if (kpw_p <= 8)
            ar_launch((gemv_mfma_persist_kernel<EPI, 8>), grid, block, 0, st, p, kpw_p, tiles);
        else if (kpw_p <= 12)
            ar_launch((gemv_mfma_persist_kernel<EPI, 12>), grid, block, 0, st, p, kpw_p, tiles);
        else
            ar_launch((gemv_mfma_persist_kernel<EPI, (NMAT == 2 ? 12 : 16)>), grid, block, 0, st, p, kpw_p,
                               tiles);
    } else {
        // fewer tiles than CUs and nothing that needs the whole row in one block: split k over
        // ks = 2*CUs / tiles blocks of 8 wavefronts (two per CU), partials folded in order
        int ks = 1;
        if (p.kpart && p.kcount && tiles <= p.kcount_n && !p.norm_w && EPI != GEMV_EPI_ARGMAX &&
            tiles < persist) {
            ks = std::min(kMaxKSplit, std::max(1, 2 * persist / tiles));
            while (ks > 1 && ((long long)tiles * ks * NMAT * 256 > p.kpart_floats || nsteps < ks * 8)) ks--;
        }
        if (ks > 1) {
            const int per = (nsteps + ks - 1) / ks, kpw = (per + 7) / 8;
            ar_launch((gemv_mfma_stream_kernel<EPI, 8>), dim3(tiles * ks), dim3(64 * 8), 0, st, p, kpw, ks);
        } else {
            const int kpw = (nsteps + kStreamWaves - 1) / kStreamWaves;
            ar_launch((gemv_mfma_stream_kernel<EPI, kStreamWaves>), dim3(tiles), dim3(64 * kStreamWaves), 0, st,
                               p, kpw, 1);
        }
    }
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

}  // namespace

int gemv_launch_mfma(const gemv::Params& p, int epi, hipStream_t st) {
    AR_CHECK_ARG(p.batch >= 1 && p.batch <= 16 && p.cols % 32 == 0, "MFMA GEMV: batch %d / cols %d unsupported",
                 p.batch, p.cols);
    switch (epi) {
        case GEMV_EPI_STORE: return launch_epi<GEMV_EPI_STORE>(p, st);
        case GEMV_EPI_RESIDUAL: return launch_epi<GEMV_EPI_RESIDUAL>(p, st);
        case GEMV_EPI_SWIGLU: return launch_epi<GEMV_EPI_SWIGLU>(p, st);
        case GEMV_EPI_ARGMAX: return launch_epi<GEMV_EPI_ARGMAX>(p, st);
        default: ar_set_error("GEMV: unknown epilogue %d", epi); return AR_HIP_ERR_INVALID;
    }
}
