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

// x[b] = E[tokens[b][pos]]: the embedding lookup AutoregressiveModel does with a host copy
// (engine/ml/.../AutoregressiveModel.java:430), done on the device so the token never leaves it.
template <typename WT>
__global__ void embed_kernel(const WT* table, int dim, const int* tokens, int token_stride, const int* pos,
                             float* x, int x_stride) {
    const int b = blockIdx.y;
    const int p = pos ? *pos : 0;
    const int tok = tokens[(size_t)b * token_stride + p];
    const WT* row = table + (size_t)tok * dim;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x) {
        float v;
        if constexpr (sizeof(WT) == 2) v = __uint_as_float((unsigned)row[i] << 16);
        else v = row[i];
        x[(size_t)b * x_stride + i] = v;
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

int launch_embed(const void* table, int wdtype, int dim, const int* tokens, int token_stride, const int* pos,
                 int batch, float* x, int x_stride, hipStream_t stream) {
    AR_CHECK_ARG(table && tokens && x && dim > 0 && batch >= 1, "embed: bad arguments");
    dim3 grid(grid_for(dim, 256, 64), batch);
    if (wdtype == AR_DTYPE_BF16)
        hipLaunchKernelGGL(embed_kernel<uint16_t>, grid, dim3(256), 0, stream, (const uint16_t*)table, dim, tokens,
                           token_stride, pos, x, x_stride);
    else
        hipLaunchKernelGGL(embed_kernel<float>, grid, dim3(256), 0, stream, (const float*)table, dim, tokens,
                           token_stride, pos, x, x_stride);
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

int launch_fill_i32(int* dst, int value, size_t n, hipStream_t stream) {
    if (!n) return AR_HIP_OK;
    hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, dst, value, n);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}
