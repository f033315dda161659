// fp32 multi-token projection on the MFMA units (v_mfma_f32_32x32x2_f32): the prompt rows of an
// fp32-weight model in one product per projection instead of one decode step per token.
//
// C[M x N] = A[M x K] . W[N x K]^T, fp32 operands and accumulation -- the stacked-row form of
// LayerFeatures.dense (domain/graph/.../LayerFeatures.java:785-830) for prompt rows, which the
// reference feeds one per step (engine/ml/.../AutoregressiveModel.java:295-308).
//
// The products are small in rows (a 128-token prompt), so a block of 32 (or 64) rows x 64 columns
// splits its k range over KS groups of wavefronts (two wavefronts per SIMD at KS = 4) and each
// wavefront stages its weight rows through LDS with direct copies one iteration ahead (see the kernel).
// Epilogues: STORE (+ bias), RESIDUAL (C += product), SWIGLU (C = (A.W2^T) * silu(A.W^T)), and
// k-slices stored separately for the consumer to add in a fixed order.
#include <atomic>

#include "ar_hip_internal.h"

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));  // (a native vector: stays in registers)

constexpr int BK = 32;  // k granularity every launch accepts

struct Params {
    const float* A;   // [M][lda]
    const float* W;   // [N][ldw]
    const float* W2;  // SwiGLU up projection, or null
    const float* bias;
    float* C;         // [M][ldc] (ksplit > 1: slice s at C + s*M*ldc)
    int M, N, K, lda, ldw, ldc, ksplit;
};

// Output tile of block `bid`: consecutive blocks (one XCD takes every 8th) walk m fastest within
// groups of 8 n-tiles, so blocks running together on an XCD share W column tiles in its L2.
__device__ inline void tile_of(int bid, int mt, int nt, int* mi, int* ni) {
    const int nblk = mt * nt;
    int t = bid;
    if (nblk % 8 == 0) t = (bid & 7) * (nblk >> 3) + (bid >> 3);
    *mi = t % mt;
    *ni = t / mt;
}

// Block barrier over LDS only: the weight loads of the next iteration stay in flight across it.
__device__ inline void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Block tile (32*WM) x 64: two column wavefronts x KS k-groups.  Wavefront (kg, wn) computes the WM
// 32 x 32 output blocks of rows 0..32*WM-1 and columns wn*32..wn*32+31 over k-group kg's 32 k values
// of every iteration (KS*32 per iteration); the KS partial sums meet in LDS at the end (added in
// group order) and group 0 runs the epilogue.  Operands of one MFMA step: lanes 0-31 supply
// k = 8q + c, lanes 32-63 k = 8q + 4 + c, for component c of the float4 each lane holds of chunk q, so
// the 32x32x2 MFMA pairs equal k values of A and W.
//  * W: every wavefront stages its own 32 rows x 32 k of each weight matrix through LDS with direct
//    global -> LDS copies (`global_load_lds_dwordx4`: 64 lanes x 16 contiguous bytes, so the loads
//    are coalesced; reading the rows straight into registers costs one 16-byte piece of 32 different
//    rows per instruction: 12-20% slower at the 128-row prompt shapes), double-buffered one iteration
//    ahead; the 16-byte chunk c of row r sits in slot c ^ (r & 7), so the eight lanes of one 16-byte
//    read phase hit eight different bank groups.  Only the wavefront that copies a tile reads it: a
//    vmcnt wait, no barrier.
//  * A: the tile (32*WM rows x KS*32 k) is staged row-major in LDS (row stride KS*32 + 4 floats,
//    conflict-free 16-byte reads), its next iteration prefetched in registers, swapped under two
//    block barriers that wait for LDS only.
// s_waitcnt immediates (vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]): vmcnt v only
constexpr int vm_imm(int v) { return (v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8); }
typedef __attribute__((address_space(3))) void lds_void;
constexpr int BKG = 32;  // k values per k-group per iteration

template <int WM, int KS, int EPI>
struct F32Shape {
    static constexpr int NW = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1, WN = 2, NWAVE = WN * KS;
    static constexpr int BKI = BKG * KS, SA = BKI + 4;
    static constexpr int WT = 32 * BKG;                        // floats of one wavefront's tile of one matrix
    static constexpr int W_FLOATS = 2 * NW * NWAVE * WT;       // double-buffered
    static constexpr int RED_FLOATS = (KS - 1) * WN * NW * WM * 1024;
    static constexpr int DYN = W_FLOATS > RED_FLOATS ? W_FLOATS : RED_FLOATS;
    static constexpr int LDS_BYTES = (DYN + 32 * WM * SA) * 4;  // + the A tile
};

template <int WM, int KS, int EPI>
__global__ __launch_bounds__(128 * KS) void gemm_f32_kernel(Params p, int mt, int nt) {
    using Sh = F32Shape<WM, KS, EPI>;
    constexpr int NW = Sh::NW, WN = Sh::WN, NWAVE = Sh::NWAVE;
    constexpr int BM = 32 * WM, NT = 64 * NWAVE;
    constexpr int BKI = Sh::BKI, SA = Sh::SA, WT = Sh::WT;
    constexpr int QG = BKG / 8;            // float4 chunks per lane per iteration
    constexpr int AL = BM * BKI / 4 / NT;  // float4 A loads per thread per iteration
    static_assert(AL >= 1 && (BM * BKI / 4) % NT == 0, "tile / thread shape");
    extern __shared__ __attribute__((aligned(1024))) float dsm[];
    float* const sw = dsm;            // [2][NW][NWAVE][32 rows x BKG]; the k-group reduction after the loop
    float* const sa = dsm + Sh::DYN;  // A tile

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave / WN, wn = wave - kg * WN;
    const int tiles = mt * nt;
    const int ks = blockIdx.x / tiles;
    int mi, ni;
    tile_of(blockIdx.x - ks * tiles, mt, nt, &mi, &ni);
    const int m0 = mi * BM, n0 = ni * 64;
    const int kper = p.K / p.ksplit, kbase = ks * kper, nit = kper / BKI;
    const int h = lane >> 5, l32 = lane & 31;

    f4 ra[AL];
    auto load_a = [&](int it) __attribute__((always_inline)) {
        const int k0 = kbase + it * BKI;
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int e = tid + i * NT, r = e / (BKI / 4), c = e - r * (BKI / 4);
            const int row = min(m0 + r, p.M - 1);  // rows past M re-read the last row (never stored)
            ra[i] = *reinterpret_cast<const f4*>(p.A + (size_t)row * p.lda + k0 + 4 * c);
        }
    };
    auto store_a = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int e = tid + i * NT, r = e / (BKI / 4), c = e - r * (BKI / 4);
            *reinterpret_cast<f4*>(&sa[r * SA + 4 * c]) = ra[i];
        }
    };
    // copy i of matrix x fills rows 8i .. 8i+7 of the wavefront's 32 weight rows: lane l writes slot
    // l % 8 of row 8i + l / 8, i.e. fetches chunk (l % 8) ^ (row & 7); the LDS destination (M0) is
    // uniform over the wavefront
    const float* wsrc[NW];
    const int drow = lane >> 3, dslot = lane & 7;
#pragma unroll
    for (int x = 0; x < NW; x++) wsrc[x] = (x ? p.W2 : p.W) + (size_t)(n0 + wn * 32) * p.ldw + kbase + kg * BKG;
    auto copy_w = [&](int it, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < NW; x++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 8 * i + drow;
                const float* g = wsrc[x] + (size_t)r * p.ldw + it * BKI + 4 * (dslot ^ (r & 7));
                float* d = sw + ((buf * NW + x) * NWAVE + wave) * WT + i * 256;
                __builtin_amdgcn_global_load_lds((const void*)g, (lds_void*)d, 16, 0, 0);
            }
    };
    f4 wr[NW][QG];
    auto read_w = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < NW; x++)
#pragma unroll
            for (int q = 0; q < QG; q++) {
                const int c = 2 * q + h;
                wr[x][q] = *reinterpret_cast<const f4*>(sw + ((buf * NW + x) * NWAVE + wave) * WT + l32 * BKG +
                                                        4 * (c ^ (l32 & 7)));
            }
    };

    floatx16 acc[NW][WM];
#pragma unroll
    for (int x = 0; x < NW; x++)
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[x][i][r] = 0.f;
    auto compute = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < QG; q++)
#pragma unroll
            for (int i = 0; i < WM; i++) {
                const f4 a = *reinterpret_cast<const f4*>(&sa[(i * 32 + l32) * SA + kg * BKG + 8 * q + 4 * h]);
#pragma unroll
                for (int x = 0; x < NW; x++) {
                    acc[x][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, wr[x][q].x, acc[x][i], 0, 0, 0);
                    acc[x][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, wr[x][q].y, acc[x][i], 0, 0, 0);
                    acc[x][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, wr[x][q].z, acc[x][i], 0, 0, 0);
                    acc[x][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, wr[x][q].w, acc[x][i], 0, 0, 0);
                }
            }
    };

    // iteration it: the A tile `it` in LDS, this wavefront's W tile `it` in buffer it & 1; the next
    // iteration's A rows (registers) and W copies (the other buffer, last read by this wavefront in
    // the previous iteration) are issued first (the last iteration re-copies its own tile: the
    // counts of every wait stay static)
    load_a(0);
    copy_w(0, 0);
    __builtin_amdgcn_s_waitcnt(vm_imm(0));
    store_a();
    lds_barrier();
    for (int it = 0; it < nit; it++) {
        load_a(min(it + 1, nit - 1));
        copy_w(min(it + 1, nit - 1), (it + 1) & 1);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(vm_imm(AL + 4 * NW));  // this wavefront's W tile `it` has landed
        asm volatile("" ::: "memory");
        read_w(it & 1);
        compute();
        lds_barrier();
        if (it + 1 >= nit) break;
        __builtin_amdgcn_s_waitcnt(vm_imm(4 * NW));  // the A rows have landed (the W copies may still fly)
        store_a();
        lds_barrier();
    }
    __builtin_amdgcn_s_waitcnt(vm_imm(0));  // no copy in flight when the buffers are reused below
    lds_barrier();

    // k-groups 1..KS-1 hand their sums to group 0, which adds them in group order
    if constexpr (KS > 1) {
        if (kg > 0) {
#pragma unroll
            for (int x = 0; x < NW; x++)
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    float* d = &dsm[((((kg - 1) * WN + wn) * NW + x) * WM + i) * 1024 + lane];
#pragma unroll
                    for (int r = 0; r < 16; r++) d[r * 64] = acc[x][i][r];
                }
        }
        lds_barrier();
        if (kg > 0) return;
#pragma unroll
        for (int g = 1; g < KS; g++)
#pragma unroll
            for (int x = 0; x < NW; x++)
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    const float* s = &dsm[((((g - 1) * WN + wn) * NW + x) * WM + i) * 1024 + lane];
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[x][i][r] += s[r * 64];
                }
    }

    // output block (i) of this wave: lane holds column (lane & 31), rows (r>>2)*8 + (lane>>5)*4 + (r&3)
    const int col = n0 + wn * 32 + l32;
    float* const Cs = p.C + (size_t)ks * p.M * p.ldc;
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
            if (row >= p.M) continue;
            float* c = Cs + (size_t)row * p.ldc + col;
            if (EPI == GEMV_EPI_STORE) {
                *c = p.bias ? acc[0][i][r] + p.bias[col] : acc[0][i][r];
            } else if (EPI == GEMV_EPI_RESIDUAL) {
                *c = *c + acc[0][i][r];
            } else {
                const float g = acc[0][i][r], u = acc[NW - 1][i][r];
                const float sg = 1.0f / (expf(-g) + 1.0f);
                *c = u * (g * sg);
            }
        }
}

template <int WM, int KS, int EPI>
int launch_t(const Params& p, hipStream_t st) {
    using Sh = F32Shape<WM, KS, EPI>;
    static_assert(Sh::LDS_BYTES <= 160 * 1024, "LDS");
    const int mt = (p.M + 32 * WM - 1) / (32 * WM), nt = p.N / 64;
    const long long blocks = (long long)mt * nt * p.ksplit;
    AR_CHECK_ARG(blocks <= 0x7fffffffLL, "GEMM f32: too many blocks");
    auto kern = gemm_f32_kernel<WM, KS, EPI>;
    // more than 64 KB of dynamic LDS needs the per-kernel opt-in, once per device
    static std::atomic<bool> attr_set[kMaxDevices];
    const int slot = ar_device_slot(st);
    if (slot < 0 || !attr_set[slot].load(std::memory_order_relaxed)) {
        AR_HIP_TRY(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Sh::LDS_BYTES));
        if (slot >= 0) attr_set[slot].store(true, std::memory_order_relaxed);
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(128 * KS), Sh::LDS_BYTES, st, p, mt, nt);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

// 64-row tiles once there are enough rows to fill the CUs with them (the W registers then feed two
// output blocks), else 32-row tiles; as many k-groups as the k-slice divides into
template <int EPI>
int launch_epi(const Params& p, hipStream_t st) {
    const int kper = p.K / p.ksplit;
    if (p.M >= 512) {
        if (kper % 64 == 0) return launch_t<2, 2, EPI>(p, st);
        return launch_t<2, 1, EPI>(p, st);
    }
    if (kper % 128 == 0) return launch_t<1, 4, EPI>(p, st);
    if (kper % 64 == 0) return launch_t<1, 2, EPI>(p, st);
    return launch_t<1, 1, EPI>(p, st);
}

}  // namespace

int gemm_f32_ksplit(int M, int N, int K, int cus) {
    const int bm = M >= 512 ? 64 : 32;
    const long long tiles = (long long)((M + bm - 1) / bm) * (N / 64);
    int s = 1;
    while (s < 8 && tiles * s * 2 <= cus && K % (256 * s * 2) == 0) s *= 2;
    return s;
}

int launch_gemm_f32(const GemmF32Launch& a, hipStream_t stream) {
    AR_CHECK_ARG(a.A && a.W && a.C, "GEMM f32: null operand");
    AR_CHECK_ARG(a.M > 0 && a.N > 0 && a.K > 0, "GEMM f32: empty shape");
    AR_CHECK_ARG(a.N % 64 == 0, "GEMM f32: N=%d must be a multiple of 64", a.N);
    AR_CHECK_ARG(a.ksplit >= 1 && a.K % (BK * a.ksplit) == 0, "GEMM f32: K=%d must be a multiple of %d", a.K,
                 BK * a.ksplit);
    AR_CHECK_ARG(a.ksplit == 1 || a.epilogue == GEMV_EPI_STORE, "GEMM f32: k-slices need the store epilogue");
    AR_CHECK_ARG(a.lda >= a.K && a.ldw >= a.K && a.ldc >= a.N && a.lda % 4 == 0 && a.ldw % 4 == 0,
                 "GEMM f32: bad leading dims");
    AR_CHECK_ARG((reinterpret_cast<uintptr_t>(a.A) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.W) & 15) == 0 &&
                     (!a.W2 || (reinterpret_cast<uintptr_t>(a.W2) & 15) == 0),
                 "GEMM f32: operands must be 16-byte aligned");
    Params p;
    p.A = a.A; p.W = a.W; p.W2 = a.W2; p.bias = a.bias; p.C = a.C;
    p.M = a.M; p.N = a.N; p.K = a.K; p.lda = a.lda; p.ldw = a.ldw; p.ldc = a.ldc; p.ksplit = a.ksplit;
    switch (a.epilogue) {
        case GEMV_EPI_STORE: return launch_epi<GEMV_EPI_STORE>(p, stream);
        case GEMV_EPI_RESIDUAL: return launch_epi<GEMV_EPI_RESIDUAL>(p, stream);
        case GEMV_EPI_SWIGLU:
            AR_CHECK_ARG(a.W2, "GEMM f32: SwiGLU needs W2");
            return launch_epi<GEMV_EPI_SWIGLU>(p, stream);
    }
    ar_set_error("GEMM f32: unsupported epilogue %d", a.epilogue);
    return AR_HIP_ERR_INVALID;
}
