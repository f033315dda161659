// fp32 multi-token projection on the MFMA units (v_mfma_f32_32x32x2_f32): the prompt rows of an
// fp32-weight model in one product per projection instead of one decode step per token.
//
// C[M x N] = A[M x K] . W[N x K]^T, fp32 operands and accumulation -- the stacked-row form of
// LayerFeatures.dense (domain/graph/.../LayerFeatures.java:785-830) for prompt rows, which the
// reference feeds one per step (engine/ml/.../AutoregressiveModel.java:295-308).
//
// Block tile (32*WM) x (32*WN), one 32 x 32 output block per wavefront, k in tiles of 32 staged
// k-major in LDS (row k holds the tile's rows / columns contiguously, so lanes 0-31 read 32
// consecutive floats of row k and lanes 32-63 of row k+1 -- the two k values of one MFMA -- without
// bank conflicts), the next k tile loaded into registers during the current tile's MFMAs.
// Epilogues: STORE (+ bias), RESIDUAL (C += product), SWIGLU (C = (A.W2^T) * silu(A.W^T)), and
// k-slices stored separately for the consumer to add in a fixed order.
#include "ar_hip_internal.h"

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 32;

struct Params {
    const float* A;   // [M][lda]
    const float* W;   // [N][ldw]
    const float* W2;  // SwiGLU up projection, or null
    const float* bias;
    float* C;         // [M][ldc] (ksplit > 1: slice s at C + s*M*ldc)
    int M, N, K, lda, ldw, ldc, ksplit;
};

// LDS row stride (floats) of a k-major tile of `cols` columns: 32 columns pad to 32 (the two lane
// halves read rows k and k+1, 32 banks apart), multiples of 64 pad by 32 for the same reason.
constexpr int lds_stride(int cols) { return cols % 64 == 0 ? cols + 32 : cols; }

// Output tile of block `bid`: consecutive blocks (one XCD takes every 8th) walk m fastest within
// groups of 8 n-tiles, so blocks running together on an XCD share W column tiles in its L2.
__device__ inline void tile_of(int bid, int mt, int nt, int* mi, int* ni) {
    const int nblk = mt * nt;
    int t = bid;
    if (nblk % 8 == 0) t = (bid & 7) * (nblk >> 3) + (bid >> 3);
    *mi = t % mt;
    *ni = t / mt;
}

template <int WM, int WN, int EPI>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f32_kernel(Params p, int mt, int nt) {
    constexpr int NW = (EPI == GEMV_EPI_SWIGLU) ? 2 : 1;
    constexpr int BM = 32 * WM, BN = 32 * WN, NT = 64 * WM * WN;
    constexpr int SA = lds_stride(BM), SW = lds_stride(BN);
    // global -> register staging: thread t loads float4 j = t / rows of row t % rows of a tile
    constexpr int AL = BM * (BK / 4) / NT, WL = BN * (BK / 4) / NT;  // float4 loads per thread
    static_assert(AL >= 1 && WL >= 1 && BM * (BK / 4) % NT == 0 && BN * (BK / 4) % NT == 0, "tile / thread shape");
    __shared__ float As[2][BK * SA];
    __shared__ float Ws[NW][2][BK * SW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int tiles = mt * nt;
    const int ks = blockIdx.x / tiles;
    int mi, ni;
    tile_of(blockIdx.x - ks * tiles, mt, nt, &mi, &ni);
    const int m0 = mi * BM, n0 = ni * BN;
    const int kper = p.K / p.ksplit, kbase = ks * kper, nkt = kper / BK;

    float4 ra[AL], rw[NW][WL];
    auto load_tile = [&](int kt) {
        const int k0 = kbase + kt * BK;
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int e = tid + i * NT, r = e % BM, j = e / BM;
            const int row = min(m0 + r, p.M - 1);  // rows past M re-read the last row (never stored)
            ra[i] = *reinterpret_cast<const float4*>(p.A + (size_t)row * p.lda + k0 + 4 * j);
        }
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float* Wm = w ? p.W2 : p.W;
#pragma unroll
            for (int i = 0; i < WL; i++) {
                const int e = tid + i * NT, c = e % BN, j = e / BN;
                rw[w][i] = *reinterpret_cast<const float4*>(Wm + (size_t)(n0 + c) * p.ldw + k0 + 4 * j);
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AL; i++) {
            const int e = tid + i * NT, r = e % BM, j = e / BM;
            float* d = &As[buf][(4 * j) * SA + r];
            d[0] = ra[i].x; d[SA] = ra[i].y; d[2 * SA] = ra[i].z; d[3 * SA] = ra[i].w;
        }
#pragma unroll
        for (int w = 0; w < NW; w++)
#pragma unroll
            for (int i = 0; i < WL; i++) {
                const int e = tid + i * NT, c = e % BN, j = e / BN;
                float* d = &Ws[w][buf][(4 * j) * SW + c];
                d[0] = rw[w][i].x; d[SW] = rw[w][i].y; d[2 * SW] = rw[w][i].z; d[3 * SW] = rw[w][i].w;
            }
    };

    floatx16 acc[NW];
#pragma unroll
    for (int w = 0; w < NW; w++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[w][r] = 0.f;

    load_tile(0);
    store_tile(0);
    __syncthreads();
    const int am = wm * 32 + (lane & 31), bn = wn * 32 + (lane & 31), kh = lane >> 5;
    for (int kt = 0; kt < nkt; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nkt) load_tile(kt + 1);
        const float* as = &As[buf][kh * SA + am];
#pragma unroll
        for (int kp = 0; kp < BK / 2; kp++) {
            const float a = as[2 * kp * SA];
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float b = Ws[w][buf][(2 * kp + kh) * SW + bn];
                acc[w] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[w], 0, 0, 0);
            }
        }
        if (kt + 1 < nkt) store_tile(buf ^ 1);
        __syncthreads();
    }

    // output block of this wave: lane holds column (lane & 31), rows (r>>2)*8 + (lane>>5)*4 + (r&3)
    const int col = n0 + wn * 32 + (lane & 31);
    float* const Cs = p.C + (size_t)ks * p.M * p.ldc;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (row >= p.M) continue;
        float* c = Cs + (size_t)row * p.ldc + col;
        if (EPI == GEMV_EPI_STORE) {
            *c = p.bias ? acc[0][r] + p.bias[col] : acc[0][r];
        } else if (EPI == GEMV_EPI_RESIDUAL) {
            *c = *c + acc[0][r];
        } else {
            const float g = acc[0][r], u = acc[NW - 1][r];
            const float sg = 1.0f / (expf(-g) + 1.0f);
            *c = u * (g * sg);
        }
    }
}

template <int WM, int WN, int EPI>
int launch_t(const Params& p, hipStream_t st) {
    const int mt = (p.M + 32 * WM - 1) / (32 * WM), nt = p.N / (32 * WN);
    const long long blocks = (long long)mt * nt * p.ksplit;
    AR_CHECK_ARG(blocks <= 0x7fffffffLL, "GEMM f32: too many blocks");
    hipLaunchKernelGGL((gemm_f32_kernel<WM, WN, EPI>), dim3((unsigned)blocks), dim3(64 * WM * WN), 0, st, p, mt, nt);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

template <int EPI>
int launch_epi(const Params& p, hipStream_t st) {
    // 64-row tiles once there are enough rows to fill the CUs with them, else 32-row tiles
    if (p.M >= 512) return launch_t<2, 2, EPI>(p, st);
    return launch_t<1, 2, EPI>(p, st);
}

}  // namespace

int gemm_f32_ksplit(int M, int N, int K, int cus) {
    const long long tiles = (long long)((M + 31) / 32) * (N / 64);
    int s = 1;
    while (s < 8 && tiles * s < 2LL * cus && K % (BK * s * 2) == 0 && K / (s * 2) >= 256) s *= 2;
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
