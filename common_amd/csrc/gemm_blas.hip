// Prefill products on rocBLAS: the same C[M x N] = A[M x K] . W[N x K]^T contractions as gemm.hip
// (fp16 operands, fp32 accumulation) for the batched prompt pass, through rocblas_gemm_ex.
//
// Each of the prefill's projections is a plain product once its epilogue is expressed in BLAS
// terms: the QKV store is beta = 0 into fp32 C, the O and down residual adds are beta = 1 on the
// fp32 residual rows (C += A W^T, the order gemm.hip's residual epilogue adds in), and the gate/up
// pair is one product over the stacked [W; W2] rows (the model's arena keeps the up matrix right
// after the gate matrix) into fp16 [M][2N] rows, followed by swiglu_rows_kernel.  The operand
// layouts map onto column-major BLAS without copies: row-major C = A W^T is column-major
// C^T = W^T' A^T', i.e. gemm(op(W) = T, op(A) = N, m = N, n = M, k = K) with W and A both read as
// K-major columns.
//
// Atomics are disabled on the handle (no split-k solutions that add partial tiles in a varying
// order), so a product is bit-identical from run to run.
#include <rocblas/rocblas.h>

#include "ar_hip_internal.h"

namespace {

const char* blas_status(rocblas_status s) { return rocblas_status_to_string(s); }

#define AR_BLAS_TRY(expr)                                                                          \
    do {                                                                                           \
        rocblas_status _s = (expr);                                                                \
        if (_s != rocblas_status_success) {                                                        \
            ar_set_error("%s failed: %s (%s:%d)", #expr, blas_status(_s), __FILE__, __LINE__);     \
            return AR_HIP_ERR_HIP;                                                                 \
        }                                                                                          \
    } while (0)

int handle_of(ar_hip_ctx* ctx, hipStream_t st, rocblas_handle* out) {
    if (!ctx->blas) {
        AR_HIP_TRY(hipSetDevice(ctx->device));
        rocblas_handle h = nullptr;
        AR_BLAS_TRY(rocblas_create_handle(&h));
        rocblas_status s = rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed);
        if (s != rocblas_status_success) {
            rocblas_destroy_handle(h);
            ar_set_error("rocblas_set_atomics_mode failed: %s", blas_status(s));
            return AR_HIP_ERR_HIP;
        }
        ctx->blas = h;
    }
    rocblas_handle h = static_cast<rocblas_handle>(ctx->blas);
    AR_BLAS_TRY(rocblas_set_stream(h, st));
    *out = h;
    return AR_HIP_OK;
}

// C (ldc) = beta C + A W^T over rows [M], outputs [N], depth K; out16: C is fp16, else fp32.
int gemm_ex(rocblas_handle h, const uint16_t* A, int lda, const uint16_t* W, int ldw, void* C, int ldc, int M,
            int N, int K, float beta, bool out16) {
    const float alpha = 1.0f;
    const rocblas_datatype ct = out16 ? rocblas_datatype_f16_r : rocblas_datatype_f32_r;
    AR_BLAS_TRY(rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &alpha, W,
                                rocblas_datatype_f16_r, ldw, A, rocblas_datatype_f16_r, lda, &beta, C, ct, ldc, C, ct,
                                ldc, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0));
    return AR_HIP_OK;
}

// act[r][c] = up * silu(gate) with gate = G[r][c], up = G[r][N + c] (fp16 [M][2N] rows), written as
// fp16 at O[r * ldo + c]; the value formula of gemm.hip's SwiGLU epilogue, in fp32.  A gate or up
// value rounded to fp16 infinity, a NaN, or an output past the fp16 range sets *rf (the caller then
// discards the batched pass).  8 columns per thread.
__global__ void __launch_bounds__(256) swiglu_rows_kernel(const _Float16* __restrict__ G, int M, int N,
                                                          _Float16* __restrict__ O, int ldo, int* rf) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const int groups = N / 8;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * groups) return;
    const int r = (int)(i / groups), c = (int)(i - (size_t)r * groups) * 8;
    const h8 g = *reinterpret_cast<const h8*>(G + (size_t)r * 2 * N + c);
    const h8 u = *reinterpret_cast<const h8*>(G + (size_t)r * 2 * N + N + c);
    h8 o;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float gv = (float)g[k], uv = (float)u[k];
        const float sg = 1.0f / (expf(-gv) + 1.0f);
        const float v = uv * (gv * sg);
        bad |= !(fabsf(gv) < kF16Overflow) || !(fabsf(uv) < kF16Overflow) || !(fabsf(v) < kF16Overflow);
        o[k] = (_Float16)v;
    }
    *reinterpret_cast<h8*>(O + (size_t)r * ldo + c) = o;
    if (__builtin_expect(bad, 0) && rf) *rf = 1;
}

}  // namespace

void gemm_blas_release(ar_hip_ctx* ctx) {
    if (ctx->blas) {
        rocblas_destroy_handle(static_cast<rocblas_handle>(ctx->blas));
        ctx->blas = nullptr;
    }
}

int launch_gemm_blas(ar_hip_ctx* ctx, const GemmLaunch& a, uint16_t* gu, size_t gu_elems, hipStream_t st) {
    AR_CHECK_ARG(a.f16, "rocBLAS GEMM: fp16 operands only");
    AR_CHECK_ARG(a.A && a.W, "rocBLAS GEMM: null operand");
    AR_CHECK_ARG(a.M > 0 && a.N > 0 && a.K > 0, "rocBLAS GEMM: empty shape");
    AR_CHECK_ARG(a.lda >= a.K && a.ldw >= a.K, "rocBLAS GEMM: bad leading dims");
    AR_CHECK_ARG(a.ksplit == 1 && !a.bias, "rocBLAS GEMM: no k-split or bias");
    rocblas_handle h;
    AR_TRY(handle_of(ctx, st, &h));
    switch (a.epilogue) {
        case GEMV_EPI_STORE:
        case GEMV_EPI_RESIDUAL:
            AR_CHECK_ARG(a.C && a.ldc >= a.N, "rocBLAS GEMM: bad fp32 output");
            AR_TRY(ar_check_range(a.C, ((size_t)(a.M - 1) * a.ldc + a.N) * 4, "rocblas_gemm_ex", "C"));
            return gemm_ex(h, a.A, a.lda, a.W, a.ldw, a.C, a.ldc, a.M, a.N, a.K,
                           a.epilogue == GEMV_EPI_RESIDUAL ? 1.0f : 0.0f, false);
        case GEMV_EPI_SWIGLU: {
            AR_CHECK_ARG(a.W2 && a.O && a.ldo >= a.N && a.N % 8 == 0 && a.ldo % 8 == 0,
                         "rocBLAS GEMM: bad SwiGLU operands");
            AR_CHECK_ARG(gu && gu_elems >= (size_t)a.M * 2 * a.N, "rocBLAS GEMM: SwiGLU scratch too small");
            AR_TRY(ar_check_range(gu, (size_t)a.M * 2 * a.N * 2, "rocblas_gemm_ex", "gate/up rows"));
            AR_TRY(ar_check_range(a.O, ((size_t)(a.M - 1) * a.ldo + a.N) * 2, "swiglu_rows_kernel", "O"));
            if (a.W2 == a.W + (size_t)a.N * a.ldw) {  // [W; W2] stacked: one product of 2N outputs
                AR_TRY(gemm_ex(h, a.A, a.lda, a.W, a.ldw, gu, 2 * a.N, a.M, 2 * a.N, a.K, 0.0f, true));
            } else {
                AR_TRY(gemm_ex(h, a.A, a.lda, a.W, a.ldw, gu, 2 * a.N, a.M, a.N, a.K, 0.0f, true));
                AR_TRY(gemm_ex(h, a.A, a.lda, a.W2, a.ldw, gu + a.N, 2 * a.N, a.M, a.N, a.K, 0.0f, true));
            }
            const size_t n = (size_t)a.M * (a.N / 8);
            swiglu_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(
                reinterpret_cast<const _Float16*>(gu), a.M, a.N, reinterpret_cast<_Float16*>(a.O), a.ldo,
                a.range_flag);
            AR_LAUNCH_CHECK();
            return AR_HIP_OK;
        }
    }
    ar_set_error("rocBLAS GEMM: unsupported epilogue %d", a.epilogue);
    return AR_HIP_ERR_INVALID;
}
