// Multi-token (prefill) contractions on the MFMA units: C[M x N] = A[M x K] . W[N x K]^T with
// 16-bit operands (bf16, or fp16 for the prefill path's higher-precision activations) and fp32
// accumulation.
//
// The reference has no multi-token path: AutoregressiveModel feeds prompt tokens one per step
// through the decode graph (engine/ml/.../AutoregressiveModel.java:295-308), i.e. every projection
// is a GEMV per token.  Stacking the T prompt rows turns each projection (LayerFeatures.dense,
// domain/graph/.../LayerFeatures.java:785-830) into one GEMM; rows are independent, so the result
// per row is the same contraction the GEMV computes.
//
// Both operands are K-contiguous (activations [M][K] row-major, HF weights [N][K] row-major), which
// is exactly the operand layout of v_mfma_f32_32x32x16_bf16: lane l supplies row (l % 32) and the
// 8 consecutive k values (l / 32) * 8 .. +7 of a 16-wide k slice; the 32x32 fp32 result lands in
// 16 registers per lane, register r holding row (r/4)*8 + (l/32)*4 + r%4, column l % 32.
//
// Tiling: 256 x 128 block tile (128 x 128 when that leaves too few blocks), BK = 64,
// wavefronts of 64 x 64 (2 x 2 MFMA tiles each).  Global tiles are loaded 16 bytes per lane into
// registers one k-step ahead and stored into a row-padded LDS tile (row stride 72 bf16 = 144 B, so
// the 16-byte fragment reads of consecutive rows fall in different bank groups).  Blocks take
// output tiles in an XCD-grouped order (tile_of).
// Epilogues: fp32 store (+bias), fp32 residual add, and SwiGLU of two weight matrices written as
// bf16 (the next GEMM's A operand).
#include <atomic>

#include "ar_hip_internal.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 halfx8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // register staging (stays in VGPRs)

// MFMA operand element: bf16 (v_mfma_f32_32x32x16_bf16) or fp16 (v_mfma_f32_32x32x16_f16); both
// take 8 consecutive k values per lane in the same lane layout and accumulate in fp32.
template <bool F16>
struct Mfma;
template <>
struct Mfma<false> {
    using frag = bf16x8;
    __device__ static inline floatx16 mac(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    __device__ static inline uint16_t from_float(float f) {
        unsigned u = __float_as_uint(f);
        if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
        u += 0x7FFFu + ((u >> 16) & 1u);
        return (uint16_t)(u >> 16);
    }
};
template <>
struct Mfma<true> {
    using frag = halfx8;
    __device__ static inline floatx16 mac(frag a, frag b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    __device__ static inline uint16_t from_float(float f) {
        const _Float16 h = (_Float16)f;
        return *reinterpret_cast<const uint16_t*>(&h);
    }
};

constexpr int BN = 128, BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row

struct GemmParams {
    const uint16_t* A;  // [M][lda] bf16
    const uint16_t* W;  // [N][ldw] bf16
    const uint16_t* W2; // second weight (SwiGLU up projection) or null
    int M, N, K, lda, ldw;
    const float* bias;  // [N] or null (STORE)
    float* C;           // fp32 [M][ldc] (STORE, RESIDUAL)
    int ldc;
    uint16_t* O;        // bf16 [M][ldo] (SWIGLU)
    int ldo;
    int ksplit;         // > 1: block (tile, s) multiplies k-slice s and stores into C + s*M*ldc
    int* rf;            // fp16 SwiGLU output overflow flag (f16_range_check), or null
};

template <int NW, int BMT>  // 1 weight matrix, or 2 for SwiGLU; BMT rows of A per block
struct Tiles {
    uint16_t a[1][BMT * LDS_STRIDE];
    uint16_t w[NW][1][BN * LDS_STRIDE];
};

// Block -> output tile.  Blocks are dispatched round-robin over the 8 XCDs; consecutive tile indices
// are given to one XCD, and tile indices walk groups of 8 m-tiles column by column, so the blocks
// an XCD runs together share A row-tiles and W column-tiles in that XCD's L2.
__device__ inline void tile_of(int bid, int mt, int nt, int* mi, int* ni) {
    const int nblk = mt * nt;
    int t = bid;
    if (nblk % 8 == 0) t = (bid & 7) * (nblk >> 3) + (bid >> 3);
    constexpr int G = 8;
    const int per_group = G * nt;
    const int group = t / per_group, first_m = group * G;
    const int gsize = min(mt - first_m, G);
    const int r = t - group * per_group;
    *mi = first_m + r % gsize;
    *ni = r / gsize;
}

// BMT x 128 block tile, (BMT/64) x 2 wavefronts of 64 x 64.
template <bool F16, int EPI, int BMT>
__global__ __launch_bounds__(BMT * 2) void gemm_kernel(GemmParams p, int mt, int nt) {
    using M = Mfma<F16>;
    using frag = typename M::frag;
    constexpr int NW = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    constexpr int NTHR = BMT * 2;
    constexpr int RPP = NTHR / 8;         // tile rows per load pass (8 threads x 16 B per 64-wide row)
    constexpr int AL = BMT / RPP, WL = BN / RPP;
    __shared__ __attribute__((aligned(16))) Tiles<NW, BMT> t;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int mi, ni;
    const int tiles = mt * nt;
    const int ks = blockIdx.x / tiles;  // k-slice (0 unless split)
    tile_of(blockIdx.x - ks * tiles, mt, nt, &mi, &ni);
    const int kbase = ks * (p.K / p.ksplit);
    float* const Cs = p.C ? p.C + (size_t)ks * p.M * p.ldc : nullptr;
    const int m0 = mi * BMT, n0 = ni * BN;

    // global -> register staging per k-step: AL x 16 B of A and WL x 16 B of each W per thread
    // (element row = tid/8 + RPP*i, k chunk = (tid%8)*8)
    const int lrow = tid >> 3, lk = (tid & 7) * 8;
    u32x4 ra[AL], rw[NW][WL];
#define AR_GEMM_LOAD_GLOBAL(k0)                                                                          \
    _Pragma("unroll") for (int i = 0; i < AL; i++) {                                                     \
        const int am = min(m0 + lrow + RPP * i, p.M - 1);                                                \
        ra[i] = *reinterpret_cast<const u32x4*>(p.A + (size_t)am * p.lda + (k0) + lk);                   \
    }                                                                                                    \
    _Pragma("unroll") for (int i = 0; i < WL; i++) {                                                     \
        const int r = lrow + RPP * i;                                                                    \
        rw[0][i] = *reinterpret_cast<const u32x4*>(p.W + (size_t)(n0 + r) * p.ldw + (k0) + lk);          \
        if constexpr (NW == 2)                                                                           \
            rw[NW - 1][i] = *reinterpret_cast<const u32x4*>(p.W2 + (size_t)(n0 + r) * p.ldw + (k0) + lk);\
    }
#define AR_GEMM_STORE_LDS(buf)                                                                           \
    _Pragma("unroll") for (int i = 0; i < AL; i++)                                                       \
        *reinterpret_cast<u32x4*>(&t.a[buf][(lrow + RPP * i) * LDS_STRIDE + lk]) = ra[i];                \
    _Pragma("unroll") for (int i = 0; i < WL; i++)                                                       \
        _Pragma("unroll") for (int w = 0; w < NW; w++)                                                   \
            *reinterpret_cast<u32x4*>(&t.w[w][buf][(lrow + RPP * i) * LDS_STRIDE + lk]) = rw[w][i];

    floatx16 acc[NW][2][2];
#pragma unroll
    for (int w = 0; w < NW; w++)
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[w][i][j][r] = 0.f;

    // One LDS buffer: the next k-tile's global loads are in flight in registers while the current
    // tile is multiplied; then the tile is swapped under two barriers.  (Half the LDS of a double
    // buffer, so two 256-row blocks fit on a CU.)
    const int nk = p.K / p.ksplit / BK;
    AR_GEMM_LOAD_GLOBAL(kbase)
    AR_GEMM_STORE_LDS(0)
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = 0;
        // (the last step reloads its own tile: a cache hit, kept unconditional so the staging stays
        // in registers)
        const int knext = kbase + (kt + 1 < nk ? kt + 1 : kt) * BK;
        AR_GEMM_LOAD_GLOBAL(knext)
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            const int kofs = kk * 16 + (lane >> 5) * 8;
            frag af[2], bfr[NW][2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int r = wm * 64 + i * 32 + (lane & 31);
                af[i] = *reinterpret_cast<const frag*>(&t.a[buf][r * LDS_STRIDE + kofs]);
            }
#pragma unroll
            for (int w = 0; w < NW; w++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int r = wn * 64 + j * 32 + (lane & 31);
                    bfr[w][j] = *reinterpret_cast<const frag*>(&t.w[w][buf][r * LDS_STRIDE + kofs]);
                }
#pragma unroll
            for (int w = 0; w < NW; w++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[w][i][j] = M::mac(af[i], bfr[w][j], acc[w][i][j]);
        }
        __syncthreads();  // every wave is done with the tile
        AR_GEMM_STORE_LDS(0)  // (unconditional: a conditional store spills the staging registers)
        __syncthreads();
    }
#undef AR_GEMM_LOAD_GLOBAL
#undef AR_GEMM_STORE_LDS

    // ---- epilogue ----------------------------------------------------------------------
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (row >= p.M) continue;
                const float v = acc[0][i][j][r];
                if (EPI == GEMV_EPI_STORE) {
                    Cs[(size_t)row * p.ldc + col] = p.bias ? v + p.bias[col] : v;
                } else if (EPI == GEMV_EPI_RESIDUAL) {
                    float* c = Cs + (size_t)row * p.ldc + col;
                    *c = *c + v;
                } else {
                    const float g = v, u = acc[NW - 1][i][j][r];
                    const float sg = 1.0f / (expf(-g) + 1.0f);
                    const float o = u * (g * sg);
                    if (F16) f16_range_check(o, p.rf);
                    p.O[(size_t)row * p.ldo + col] = M::from_float(o);
                }
            }
        }
}

// ---- large-shape kernel: 256 x 256 tiles fed by direct global -> LDS loads -------------------
//
// For products with many tiles (the long prompts of batched prefill) a 4-wavefront block owns a
// BM x 256 tile (BM = 256: 128 x 128 per wavefront, 16 MFMA accumulators; BM = 128 for the last
// partial round of a product whose tile count is not a multiple of the CU count, see launch_t), BK =
// 64, two LDS stages of 64 KB (BM 256) filled by global_load_lds_dwordx4 (each lane's 16 bytes go
// straight to LDS; no staging registers, no LDS store instructions).  Rows are 128 B; the 16-byte chunk c of row r sits in slot
// c ^ ((r >> 1) & 7), so the eight lanes that read one 16-byte piece each per LDS cycle hit eight
// different bank groups.  Per k-tile the block waits once: after the third k-step's MFMAs every
// wavefront waits for its own copies of the next tile (vmcnt) and its own LDS reads (lgkmcnt),
// then a barrier makes both block-wide, the freed stage is refilled with tile kt + 2, and the next
// tile's first fragments are read while the last k-step's MFMAs run.  The refill is issued in two
// halves: the first right after the barrier, the second after the next tile's first k-step of MFMAs
// (a burst of all 64 copy instructions of a block fills the texture units' queue and stalls the
// wavefronts at issue while their MFMAs wait; split in two: 4-10% faster on the prefill shapes).
// Copies address a wavefront-uniform base (SGPRs) plus a 32-bit per-lane offset, and their LDS
// destination is a uniform M0.  Waits are written by hand: a workgroup-scope fence
// (__syncthreads) would also wait for every outstanding LDS copy.
namespace dma {
constexpr int BNW = 256, BK = 64, STAGES = 2, NTHR = 256, KS = BK / 16;
constexpr int ROWB = BK * 2;
constexpr int TILE_W = 256 * ROWB;
template <int BM>
struct Shape {
    static constexpr int TILE_A = BM * ROWB;
    static constexpr int STAGE_B = TILE_A + TILE_W;
    static constexpr int LDS_BYTES = STAGES * STAGE_B;  // 128 KB (BM 256) or 96 KB (BM 128)
    static constexpr int DMA_A = TILE_A / 1024 / 4;      // copy instructions per wavefront per stage: A
    static constexpr int DMA_W = TILE_W / 1024 / 4;      // and W
};
// s_waitcnt immediates (vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14])
constexpr int vm_imm(int v, int lgkm) { return (v & 15) | ((v >> 4) << 14) | (7 << 4) | (lgkm << 8); }
typedef __attribute__((address_space(3))) void lds_void;
__device__ inline int swz(int r, int c) { return c ^ ((r >> 1) & 7); }
}  // namespace dma

template <bool F16, int EPI, int BM>
__global__ __launch_bounds__(dma::NTHR) void gemm_dma_kernel(GemmParams p, int mt, int nt) {
    using Sh = dma::Shape<BM>;
    using Mf = Mfma<F16>;
    using frag = typename Mf::frag;
    extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
    constexpr int NW = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    constexpr int BN = dma::BNW / NW;  // output columns per block (SwiGLU: 128 gate rows + 128 up rows)
    constexpr int WN = BN / 2, FN = WN / 32, FM = BM / 64, WM = BM / 2;  // wavefront tile WM x WN
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int mi, ni;
    tile_of(blockIdx.x, mt, nt, &mi, &ni);
    const int m0 = mi * BM, n0 = ni * BN;
    const int nk = p.K / dma::BK;

    // copy plan: instruction i of wavefront w fills rows 8j .. 8j+7 (j = 4i + w) of a tile; lane l
    // writes slot l % 8 of row 8j + l / 8, i.e. fetches chunk dma::swz(row, l % 8)
    // per-lane byte offsets from wave-uniform bases (the block's first A row, its first W / W2 row),
    // so each copy is a uniform base in SGPRs plus a 32-bit VGPR offset, and the LDS destination a
    // uniform M0: advancing k only moves the bases
    const uint16_t* const baseA = p.A + (size_t)m0 * p.lda;
    const uint16_t* const baseW = p.W + (size_t)n0 * p.ldw;
    const uint16_t* const baseW2 = NW == 2 ? p.W2 + (size_t)n0 * p.ldw : baseW;
    uint32_t offA[Sh::DMA_A], offW[Sh::DMA_W];
#pragma unroll
    for (int i = 0; i < Sh::DMA_A; i++) {
        const int j = 4 * i + wave, r = 8 * j + (lane >> 3), c = dma::swz(r, lane & 7);
        offA[i] = (uint32_t)(((min(m0 + r, p.M - 1) - m0) * p.lda + c * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < Sh::DMA_W; i++) {
        const int j = 4 * i + wave, r = 8 * j + (lane >> 3), c = dma::swz(r, lane & 7);
        offW[i] = (uint32_t)((((NW == 2 && r >= BN) ? r - BN : r) * p.ldw + c * 8) * 2);
    }
    auto issue = [&](int slot, int kt, int i_lo = 0, int i_hi = Sh::DMA_W) {
        const int k0 = kt * dma::BK;
        unsigned char* st = lds + slot * Sh::STAGE_B;
        const char* bA = reinterpret_cast<const char*>(baseA + k0);
        const char* bW = reinterpret_cast<const char*>(baseW + k0);
        const char* bW2 = reinterpret_cast<const char*>(baseW2 + k0);
#pragma unroll
        for (int i = 0; i < Sh::DMA_W; i++) {
            if (i < i_lo || i >= i_hi) continue;
            const int j = 4 * i + wave;
            if (i < Sh::DMA_A)
                __builtin_amdgcn_global_load_lds((const void*)(bA + offA[i]), (dma::lds_void*)(st + j * 1024), 16, 0, 0);
            // W rows past BN belong to W2 (the SwiGLU up projection): copies i >= 4 (rows 32i + ...)
            const char* bw = (NW == 2 && 32 * i >= BN) ? bW2 : bW;
            __builtin_amdgcn_global_load_lds((const void*)(bw + offW[i]), (dma::lds_void*)(st + Sh::TILE_A + j * 1024), 16, 0, 0);
        }
    };

    floatx16 acc[NW][FM][FN];
#pragma unroll
    for (int w = 0; w < NW; w++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[w][i][j][r] = 0.f;

    frag fa[2][FM], fb[2][NW][FN];  // fragments of two k-steps
    auto read = [&](int set, int slot, int kk) {
        const unsigned char* st = lds + slot * Sh::STAGE_B;
        const int c = kk * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const int r = wm * WM + i * 32 + (lane & 31);
            fa[set][i] = *reinterpret_cast<const frag*>(st + r * dma::ROWB + dma::swz(r, c) * 16);
        }
#pragma unroll
        for (int w = 0; w < NW; w++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int r = w * BN + wn * WN + j * 32 + (lane & 31);
                fb[set][w][j] = *reinterpret_cast<const frag*>(st + Sh::TILE_A + r * dma::ROWB + dma::swz(r, c) * 16);
            }
    };
    auto mma = [&](int set) {
#pragma unroll
        for (int w = 0; w < NW; w++)
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) acc[w][i][j] = Mf::mac(fa[set][i], fb[set][w][j], acc[w][i][j]);
    };

#pragma unroll
    for (int s = 0; s < dma::STAGES; s++) issue(s, min(s, nk - 1));
    asm volatile("" ::: "memory");
    // all but stage 0's copies may be in flight
    __builtin_amdgcn_s_waitcnt(dma::vm_imm((Sh::DMA_A + Sh::DMA_W) * (dma::STAGES - 1), 15));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read(0, 0, 0);
    read(1, 0, 1);
    for (int kt = 0; kt < nk; kt++) {
        const int slot = kt % dma::STAGES, nslot = (kt + 1) % dma::STAGES;
#pragma unroll
        for (int kk = 0; kk < dma::KS - 2; kk++) {
            mma(kk & 1);
            __builtin_amdgcn_sched_barrier(0);
            if (kk == 0 && kt >= 1) issue(nslot, min(kt + 1, nk - 1), Sh::DMA_W / 2, Sh::DMA_W);  // second half of tile kt+1
            read(kk & 1, slot, kk + 2);
        }
        mma((dma::KS - 2) & 1);
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(dma::vm_imm((Sh::DMA_A + Sh::DMA_W) * (dma::STAGES - 2), 0));  // tile kt+1 landed, LDS reads done
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // the stage just finished takes tile kt + dma::STAGES (the last tiles reload tile nk - 1, which
        // keeps every wait count static); the reads of the last iteration fetch a stale stage
        issue(slot, min(kt + dma::STAGES, nk - 1), 0, Sh::DMA_W / 2);  // first half of tile kt+2
        read((dma::KS - 2) & 1, nslot, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma((dma::KS - 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
        read((dma::KS - 1) & 1, nslot, 1);
    }
    __builtin_amdgcn_s_waitcnt(0);  // no copy in flight when the block ends

    // epilogue, one 32-row band of the wavefront at a time; the residual's old values are loaded 32
    // at a time (clamped rows, no branches) before the adds and the guarded stores
#pragma unroll
    for (int i = 0; i < FM; i++) {
        const int rbase = m0 + wm * WM + i * 32 + (lane >> 5) * 4;
        if constexpr (EPI == GEMV_EPI_RESIDUAL) {
#pragma unroll
            for (int j0 = 0; j0 < FN; j0 += 2) {
                float old[2][16];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int col = n0 + wn * WN + (j0 + j) * 32 + (lane & 31);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = min(rbase + (r >> 2) * 8 + (r & 3), p.M - 1);
                        old[j][r] = p.C[(size_t)row * p.ldc + col];
                    }
                }
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int col = n0 + wn * WN + (j0 + j) * 32 + (lane & 31);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = rbase + (r >> 2) * 8 + (r & 3);
                        if (row < p.M) p.C[(size_t)row * p.ldc + col] = old[j][r] + acc[0][i][j0 + j][r];
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int col = n0 + wn * WN + j * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + (r >> 2) * 8 + (r & 3);
                    if (row >= p.M) continue;
                    const float v = acc[0][i][j][r];
                    if (EPI == GEMV_EPI_STORE) {
                        p.C[(size_t)row * p.ldc + col] = p.bias ? v + p.bias[col] : v;
                    } else {
                        const float g = v, u = acc[NW - 1][i][j][r];
                        const float sg = 1.0f / (expf(-g) + 1.0f);
                        const float o = u * (g * sg);
                        if (F16) f16_range_check(o, p.rf);
                        p.O[(size_t)row * p.ldo + col] = Mf::from_float(o);
                    }
                }
            }
        }
    }
}

template <bool F16, int EPI, int BM>
int launch_dma(const GemmParams& p, hipStream_t st) {
    constexpr int NW = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    using Sh = dma::Shape<BM>;
    const int mt = (p.M + BM - 1) / BM, nt = p.N / (dma::BNW / NW);
    // more than 64 KB of dynamic LDS needs the per-kernel opt-in, once per device
    static std::atomic<bool> attr_set[kMaxDevices];
    const int slot = ar_device_slot(st);
    if (slot < 0 || !attr_set[slot].load(std::memory_order_relaxed)) {
        AR_HIP_TRY(hipFuncSetAttribute((const void*)gemm_dma_kernel<F16, EPI, BM>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, Sh::LDS_BYTES));
        if (slot >= 0) attr_set[slot].store(true, std::memory_order_relaxed);
    }
    hipLaunchKernelGGL((gemm_dma_kernel<F16, EPI, BM>), dim3(mt * nt), dim3(dma::NTHR), Sh::LDS_BYTES, st, p, mt, nt);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

// The large-tile kernel pays off with at least kDmaMinTiles tiles (measured on the prefill shapes:
// +7-13% at 65,536 rows; at 2,048 rows the SwiGLU product's 384 tiles still gain (C4 prefill
// 11.56 -> 11.14 ms), while 128-tile products leave too many CUs idle).
constexpr long long kDmaMinTiles = 256;

template <int EPI>
bool use_dma(const GemmParams& p) {
    constexpr int NW = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    const int bn = dma::BNW / NW;
    if (p.ksplit != 1 || p.N % bn || p.K % dma::BK) return false;
    return (long long)((p.M + 255) / 256) * (p.N / bn) >= kDmaMinTiles;
}

// The columns [n0, n0 + n) of a product: the same A, the weight rows n0.. and the output columns n0..
GemmParams column_range(const GemmParams& p, int n0, int n) {
    GemmParams q = p;
    q.W = p.W + (size_t)n0 * p.ldw;
    if (p.W2) q.W2 = p.W2 + (size_t)n0 * p.ldw;
    if (p.bias) q.bias = p.bias + n0;
    if (p.C) q.C = p.C + n0;
    if (p.O) q.O = p.O + n0;
    q.N = n;
    return q;
}

// 256 x 256 tiles in whole rounds over the CUs, and the remainder as 128-row tiles.  With one
// 256-row block per CU, a tile count that is not a multiple of the CU count leaves a last round in
// which most CUs idle (C4 gate/up: 384 tiles on 256 CUs = two full-tile times); the columns past the
// whole rounds go instead to half-height tiles, twice as many blocks of half the work (C4: 256 tiles
// of 256 x 256 for the first 4096 outputs, then 256 of 128 x 256: one and a half tile times).
template <bool F16, int EPI>
int launch_dma_rounds(const GemmParams& p, int cus, hipStream_t st) {
    constexpr int NW = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    const int bn = dma::BNW / NW;
    const int mt = (p.M + 255) / 256, nt = p.N / bn;
    const long long tiles = (long long)mt * nt;
    if (cus > 0 && tiles > cus && tiles % cus != 0) {
        const int nt1 = (int)((tiles / cus) * cus / mt);                // columns of whole 256-row rounds
        const long long half = (long long)((p.M + 127) / 128) * (nt - nt1);  // 128-row tiles of the rest
        if (nt1 > 0 && half <= cus) {
            AR_TRY((launch_dma<F16, EPI, 256>(column_range(p, 0, nt1 * bn), st)));
            return launch_dma<F16, EPI, 128>(column_range(p, nt1 * bn, (nt - nt1) * bn), st);
        }
    }
    return launch_dma<F16, EPI, 256>(p, st);
}

template <int EPI, int BMT>
int launch_bm(const GemmParams& p, bool f16, hipStream_t st) {
    const int mt = (p.M + BMT - 1) / BMT, nt = p.N / BN;
    const dim3 grid(mt * nt * p.ksplit), block(BMT * 2);
    if (f16)
        hipLaunchKernelGGL((gemm_kernel<true, EPI, BMT>), grid, block, 0, st, p, mt, nt);
    else
        hipLaunchKernelGGL((gemm_kernel<false, EPI, BMT>), grid, block, 0, st, p, mt, nt);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

// 256-row block tiles halve the A/W tile loads per MFMA (measured: the 128 x 128 tile is bound by
// L2 -> CU operand traffic); they are used while they still give two blocks per CU, or one for
// SwiGLU (two weight tiles per block).  Measured at C4 (2048 rows): QKV 47 us with 128-row tiles vs
// 51 us, gate/up 163 us with 256-row tiles vs 176 us.
template <int EPI>
int launch_t(const GemmParams& p, bool f16, hipStream_t st) {
    if (use_dma<EPI>(p)) {
        const int cus = ar_device_cus(st);
        return f16 ? launch_dma_rounds<true, EPI>(p, cus, st) : launch_dma_rounds<false, EPI>(p, cus, st);
    }
    const long long blocks256 = (long long)((p.M + 255) / 256) * (p.N / BN) * p.ksplit;
    if (blocks256 >= (EPI == GEMV_EPI_SWIGLU ? 256 : 512)) return launch_bm<EPI, 256>(p, f16, st);
    return launch_bm<EPI, 128>(p, f16, st);
}

}  // namespace

int launch_gemm(const GemmLaunch& a, hipStream_t stream) {
    AR_CHECK_ARG(a.A && a.W, "GEMM: null operand");
    AR_CHECK_ARG(a.M > 0 && a.N > 0 && a.K > 0, "GEMM: empty shape");
    AR_CHECK_ARG(a.N % BN == 0, "GEMM: N=%d must be a multiple of %d", a.N, BN);
    AR_CHECK_ARG(a.K % BK == 0, "GEMM: K=%d must be a multiple of %d", a.K, BK);
    AR_CHECK_ARG(a.ksplit >= 1 && a.K % (BK * a.ksplit) == 0 && (a.ksplit == 1 || a.epilogue == GEMV_EPI_STORE),
                 "GEMM: a k-split of %d needs K %% %d == 0 and the store epilogue", a.ksplit, BK * a.ksplit);
    AR_CHECK_ARG(a.lda >= a.K && a.ldw >= a.K && a.lda % 8 == 0 && a.ldw % 8 == 0, "GEMM: bad leading dims");
    AR_CHECK_ARG((reinterpret_cast<uintptr_t>(a.A) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.W) & 15) == 0,
                 "GEMM: operands must be 16-byte aligned");
    GemmParams p;
    p.A = a.A; p.W = a.W; p.W2 = a.W2; p.M = a.M; p.N = a.N; p.K = a.K; p.lda = a.lda; p.ldw = a.ldw;
    p.bias = a.bias; p.C = a.C; p.ldc = a.ldc; p.O = a.O; p.ldo = a.ldo; p.ksplit = a.ksplit; p.rf = a.range_flag;
    switch (a.epilogue) {
        case GEMV_EPI_STORE:
            AR_CHECK_ARG(a.C && a.ldc >= a.N, "GEMM: bad fp32 output");
            return launch_t<GEMV_EPI_STORE>(p, a.f16, stream);
        case GEMV_EPI_RESIDUAL:
            AR_CHECK_ARG(a.C && a.ldc >= a.N, "GEMM: bad fp32 output");
            return launch_t<GEMV_EPI_RESIDUAL>(p, a.f16, stream);
        case GEMV_EPI_SWIGLU:
            AR_CHECK_ARG(a.W2 && (reinterpret_cast<uintptr_t>(a.W2) & 15) == 0, "GEMM: SwiGLU needs an aligned W2");
            AR_CHECK_ARG(a.O && a.ldo >= a.N, "GEMM: bad bf16 output");
            return launch_t<GEMV_EPI_SWIGLU>(p, a.f16, stream);
    }
    ar_set_error("GEMM: unsupported epilogue %d", a.epilogue);
    return AR_HIP_ERR_INVALID;
}
