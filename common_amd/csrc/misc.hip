// Small kernels of the decode path and the stand-alone operators.
#include "ar_hip_internal.h"

namespace {

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ inline bool better(float v1, int i1, float v2, int i2) {
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

// Start of a decode step, one block: picks the token fed at position p for every sequence (the
// prompt token, or the greedy choice of the previous step decoded from the packed argmax keys),
// clears the keys, copies the embedding row and publishes p as the step's position.
// AutoregressiveModel.next + embedding copy (engine/ml/.../AutoregressiveModel.java:295-308,430).
template <typename WT>
__global__ __launch_bounds__(1024) void step_begin_kernel(const WT* table, int dim, int vocab, int* tokens,
                                                         int token_stride, unsigned long long* keys, int* state,
                                                         int batch, float* x, int x_stride, uint16_t* x_hi,
                                                         uint16_t* x_lo, const float* x_gain, float* ss_out) {
    __shared__ int tok_s[8];
    __shared__ unsigned long long red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int p = state[2];
    const int plen = state[1];
    for (int b = 0; b < batch; b++) {
        if (p > 0 && p >= plen) {
            unsigned long long k = (tid < kArgmaxSlots) ? keys[(size_t)b * kArgmaxSlots + tid] : 0ull;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const unsigned long long o = __shfl_xor(k, off, 64);
                k = o > k ? o : k;
            }
            if (lane == 0) red[wave] = k;
            __syncthreads();
            if (tid == 0) {
                unsigned long long m = red[0];
                for (int w = 1; w < (int)(blockDim.x >> 6); w++) m = red[w] > m ? red[w] : m;
                int t = m ? (int)(0xFFFFFFFFu - (unsigned)(m & 0xFFFFFFFFull)) : 0;
                if (t < 0 || t >= vocab) t = 0;
                tokens[(size_t)b * token_stride + p] = t;
                tok_s[b] = t;
            }
            __syncthreads();
        } else if (tid == 0) {
            tok_s[b] = tokens[(size_t)b * token_stride + p];
        }
    }
    __syncthreads();
    for (int i = tid; i < batch * kArgmaxSlots; i += blockDim.x) keys[i] = 0ull;
    for (int b = 0; b < batch; b++) {
        const WT* row = table + (size_t)tok_s[b] * dim;
        // every lane takes part in each pass (16-lane groups hold 16 consecutive entries: the
        // per-16-row sums of squares for the fragment-ordered GEMVs' RMSNorm)
        for (int i0 = 0; i0 < dim; i0 += blockDim.x) {
            const int i = i0 + tid;
            float v = 0.f;
            if (i < dim) {
                if constexpr (sizeof(WT) == 2) v = __uint_as_float((unsigned)row[i] << 16);
                else v = row[i];
                x[(size_t)b * x_stride + i] = v;
                if (x_hi)
                    bf16_planes(x_gain ? v * x_gain[i] : v, x_hi + (size_t)b * x_stride + i, x_lo + (size_t)b * x_stride + i);
            }
            if (ss_out) {
                float s2 = v * v;
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) s2 += __shfl_xor(s2, off, 64);
                if ((tid & 15) == 0 && i < dim) ss_out[(size_t)(i / 16) * 16 + b] = s2;
            }
        }
    }
    if (tid == 0) {
        state[0] = p;
        state[2] = p + 1;
    }
}

// rmsnorm, one block per row (NormalizationLayerFeatures.java:584-595)
__global__ void rmsnorm_kernel(const float* x, const float* w, float* y, int n, float eps) {
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += xr[i] * xr[i];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += red[i];
    const float r = 1.0f / sqrtf(t / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) yr[i] = (w[i] * xr[i]) * r;
}

// split-half RoPE on flat (heads*hd) rows (AttentionFeatures.java:195-237, RotationFeatures.java:124-208)
__global__ void rope_kernel(float* x, int heads, int hd, int pos, double c, int row_stride) {
    const int fd = hd / 2;
    float* xr = x + (size_t)blockIdx.y * row_stride;
    for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < heads * fd; idx += gridDim.x * blockDim.x) {
        const int h = idx / fd, f = idx - h * fd;
        const double ang = (double)pos * exp((double)f * c);
        const float cs = (float)cos(ang), sn = (float)sin(ang);
        const float x1 = xr[(size_t)h * hd + f], x2 = xr[(size_t)h * hd + f + fd];
        xr[(size_t)h * hd + f] = x1 * cs - x2 * sn;
        xr[(size_t)h * hd + f + fd] = x2 * cs + x1 * sn;
    }
}

// first index of the maximum, one block per row (AggregationFeatures.java:111-121)
__global__ void index_of_max_kernel(const float* x, int n, int* out) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        if (better(xr[i], i, bv, bi)) { bv = xr[i]; bi = i; }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        bv = sv[0]; bi = si[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++)
            if (better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
        out[blockIdx.x] = (bi == 0x7FFFFFFF) ? 0 : bi;
    }
}

// float32 -> bfloat16 bits, round to nearest even (NaN kept quiet)
__global__ void f32_to_bf16_kernel(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        unsigned u = __float_as_uint(src[i]);
        if ((u & 0x7F800000u) == 0x7F800000u) {
            dst[i] = (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
        } else {
            u += 0x7FFFu + ((u >> 16) & 1u);
            dst[i] = (uint16_t)(u >> 16);
        }
    }
}

__global__ void bf16_to_f16_kernel(const uint16_t* src, uint16_t* dst, size_t n, int* rf) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float f = __uint_as_float((unsigned)src[i] << 16);
        f16_range_check(f, rf);
        const _Float16 h = (_Float16)f;
        dst[i] = *reinterpret_cast<const uint16_t*>(&h);
    }
}

__global__ void fill_i32_kernel(int* dst, int value, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = value;
}

int grid_for(size_t n, int threads, int cap = 4096) {
    size_t g = (n + threads - 1) / threads;
    if (g < 1) g = 1;
    if (g > (size_t)cap) g = cap;
    return (int)g;
}

}  // namespace

int launch_step_begin(const void* table, int wdtype, int dim, int vocab, int* tokens, int token_stride,
                      unsigned long long* keys, int* state, int batch, float* x, int x_stride, uint16_t* x_hi,
                      uint16_t* x_lo, const float* x_gain, float* ss_out, hipStream_t stream) {
    AR_CHECK_ARG(table && tokens && keys && state && x && dim > 0, "step begin: bad arguments");
    AR_CHECK_ARG(!ss_out || dim % 16 == 0, "step begin: sums of squares need dim %% 16 == 0");
    AR_CHECK_ARG(!x_hi == !x_lo, "step begin: operand planes come in hi/lo pairs");
    AR_CHECK_ARG(batch >= 1 && batch <= 8, "step begin: batch %d outside 1..8", batch);
    if (ar_check_ptrs_enabled()) {
        const char* k = "step begin";
        const size_t wb = wdtype == AR_DTYPE_BF16 ? 2 : 4, B1 = batch - 1;
        AR_TRY(ar_check_range(table, (size_t)vocab * dim * wb, k, "embedding table"));
        AR_TRY(ar_check_range(tokens, (size_t)batch * token_stride * 4, k, "token rows"));
        AR_TRY(ar_check_range(keys, (size_t)batch * kArgmaxSlots * 8, k, "argmax keys"));
        AR_TRY(ar_check_range(state, 3 * sizeof(int), k, "loop state"));
        AR_TRY(ar_check_range(x, (B1 * x_stride + dim) * 4, k, "residual rows"));
        AR_TRY(ar_check_range(x_hi, (B1 * x_stride + dim) * 2, k, "hi plane"));
        AR_TRY(ar_check_range(x_lo, (B1 * x_stride + dim) * 2, k, "lo plane"));
        AR_TRY(ar_check_range(x_gain, (size_t)dim * 4, k, "plane gain"));
        AR_TRY(ar_check_range(ss_out, (size_t)(dim / 16) * 16 * 4, k, "sums of squares"));
    }
    if (wdtype == AR_DTYPE_BF16)
        hipLaunchKernelGGL(step_begin_kernel<uint16_t>, dim3(1), dim3(1024), 0, stream, (const uint16_t*)table, dim,
                           vocab, tokens, token_stride, keys, state, batch, x, x_stride, x_hi, x_lo, x_gain, ss_out);
    else
        hipLaunchKernelGGL(step_begin_kernel<float>, dim3(1), dim3(1024), 0, stream, (const float*)table, dim, vocab,
                           tokens, token_stride, keys, state, batch, x, x_stride, x_hi, x_lo, x_gain, ss_out);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_rmsnorm(const float* x, const float* w, float* y, int rows, int n, float eps, hipStream_t stream) {
    AR_CHECK_ARG(x && w && y && rows > 0 && n > 0, "rmsnorm: bad arguments");
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, stream, x, w, y, n, eps);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_rope(float* x, int heads, int hd, int pos, double theta, int rows, int row_stride, hipStream_t stream) {
    AR_CHECK_ARG(x && heads > 0 && hd > 0 && hd % 2 == 0 && rows > 0 && pos >= 0, "rope: bad arguments");
    const double c = -2.0 * log(theta) / (double)hd;
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for((size_t)heads * hd / 2, 256, 64), rows), dim3(256), 0, stream, x,
                       heads, hd, pos, c, row_stride);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_index_of_max(const float* x, int rows, int n, int* out, hipStream_t stream) {
    AR_CHECK_ARG(x && out && rows > 0 && n > 0, "indexOfMax: bad arguments");
    hipLaunchKernelGGL(index_of_max_kernel, dim3(rows), dim3(256), 0, stream, x, n, out);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_f32_to_bf16(const float* src, uint16_t* dst, size_t n, hipStream_t stream) {
    if (!n) return AR_HIP_OK;
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, src, dst, n);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_bf16_to_f16(const uint16_t* src, uint16_t* dst, size_t n, int* range_flag, hipStream_t stream) {
    if (!n) return AR_HIP_OK;
    hipLaunchKernelGGL(bf16_to_f16_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, src, dst, n, range_flag);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_fill_i32(int* dst, int value, size_t n, hipStream_t stream) {
    if (!n) return AR_HIP_OK;
    hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, dst, value, n);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}
