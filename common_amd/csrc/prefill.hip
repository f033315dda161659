// Multi-token prefill kernels: the T prompt rows of a sequence processed together.
//
// The reference feeds prompt tokens one per step through the decode graph
// (engine/ml/.../AutoregressiveModel.java:295-308).  Row t of a prefill is exactly step t of that
// loop: same RMSNorm (NormalizationLayerFeatures.java:584-595), QK-norm (AttentionFeatures.java:
// 840-845, 886-891), split-half RoPE at position p0 + t (RotationFeatures.java:124-208), cache
// write of row p0 + t (AttentionFeatures.java:858-877) and causal attention over rows 0..p0 + t
// (AttentionFeatures.java:901-921, ActivationFeatures.java:135-143).  The projections run as MFMA
// GEMMs (gemm.hip) on fp16 activations (10-bit mantissa: the bf16 weights convert to fp16 exactly
// for |w| >= 2^-17, and activation rounding error stays ~8x below bf16's); everything here keeps
// fp32 arithmetic except the MFMA operands of the attention products.
#include "ar_hip_internal.h"

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 halfx8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// fp32 -> fp16 bits (round to nearest even); a value that overflows marks *rf (f16_range_check)
__device__ inline uint16_t f2h(float f, int* rf = nullptr) {
    f16_range_check(f, rf);
    const _Float16 h = (_Float16)f;
    return *reinterpret_cast<const uint16_t*>(&h);
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ inline float block_sum(float v, float* scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += scratch[w];
    return t;
}

// x[r] = E[tokens[b][t]] for r = b*T + t (row r of sequence b holds prompt token t).
template <typename WT>
__global__ void embed_rows_kernel(const WT* table, int dim, const int* tokens, int token_stride, int T, float* x) {
    const int r = blockIdx.x, b = r / T, t = r - b * T;
    const WT* row = table + (size_t)tokens[(size_t)b * token_stride + t] * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        float v;
        if constexpr (sizeof(WT) == 2) v = __uint_as_float((unsigned)row[i] << 16);
        else v = row[i];
        x[(size_t)r * dim + i] = v;
    }
}

// out[r] = fp16((w * x[r]) * 1/sqrt(mean(x[r]^2) + eps)), one block per row.
__global__ __launch_bounds__(256) void rmsnorm_rows_f16_kernel(const float* x, const float* w, uint16_t* out,
                                                                int n, float eps, int* rf) {
    __shared__ float scratch[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += xr[i] * xr[i];
    ss = block_sum(ss, scratch);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[(size_t)blockIdx.x * n + i] = f2h((w[i] * xr[i]) * r, rf);
}

// Residual fold of a split-k projection followed by the row RMSNorm: x[r] += sum_s parts[s][r] (in
// slice order), written back, then out[r] = fp16((w * x[r]) * 1/sqrt(mean(x[r]^2) + eps)).
__global__ __launch_bounds__(256) void fold_rmsnorm_rows_f16_kernel(float* x, const float* parts, int nparts,
                                                                     size_t part_stride, const float* w,
                                                                     uint16_t* out, int n, float eps, int* rf) {
    __shared__ float scratch[4];
    float* xr = x + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = xr[i];
        for (int s = 0; s < nparts; s++) v += parts[s * part_stride + (size_t)blockIdx.x * n + i];
        if (nparts) xr[i] = v;
        ss += v * v;
    }
    ss = block_sum(ss, scratch);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[(size_t)blockIdx.x * n + i] = f2h((w[i] * xr[i]) * r, rf);
}

// The fold + row RMSNorm above with an fp32 output row (the fp32-weight prefill's GEMM input).
__global__ __launch_bounds__(256) void fold_rmsnorm_rows_f32_kernel(float* x, const float* parts, int nparts,
                                                                     size_t part_stride, const float* w, float* out,
                                                                     int n, float eps) {
    __shared__ float scratch[4];
    float* xr = x + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = xr[i];
        for (int s = 0; s < nparts; s++) v += parts[s * part_stride + (size_t)blockIdx.x * n + i];
        if (nparts) xr[i] = v;
        ss += v * v;
    }
    ss = block_sum(ss, scratch);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[(size_t)blockIdx.x * n + i] = (w[i] * xr[i]) * r;
}

// dst[b] = src[first + b*step] + sum_s parts[s][first + b*step], rows of n floats.
__global__ __launch_bounds__(256) void fold_rows_kernel(const float* src, const float* parts, int nparts,
                                                        size_t part_stride, int first, int step, int n, float* dst) {
    const size_t row = (size_t)first + (size_t)blockIdx.x * step;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = src[row * n + i];
        for (int s = 0; s < nparts; s++) v += parts[s * part_stride + row * n + i];
        dst[(size_t)blockIdx.x * n + i] = v;
    }
}

struct PrepParams {
    const float* qkv;       // [R][qkv_stride] raw projections
    int qkv_stride;
    const float* q_norm;
    const float* k_norm;
    float eps;
    int per_head;
    const float2* rope_tab; // [S][hd/2]
    void* kcache;           // [B][KV][S][hd], fp32 or fp16 (kv16)
    void* vcache;
    int kv16;
    int S, T, p0, heads, kv_heads, hd;
    uint16_t* qb;           // [R][heads*hd] fp16 normalised, rotated queries
    uint16_t* k16;          // [B][KV][Tp][hd] fp16 keys of the prompt rows (for the attention MFMAs)
    int Tp;
    int* rf;                // overflow flag of the fp16 stores (f16_range_check)
    float* q32;             // fp32-weight prefill: fp32 queries [R][heads*hd], no fp16 q / k16 copies
};

// One block per prompt row: QK-norm (whole vector or per head), RoPE at position p0 + t, k and v
// into the cache row, the query to an fp16 row for the attention kernel.
__global__ __launch_bounds__(256) void qk_prep_kernel(PrepParams p) {
    __shared__ float scratch[4];
    __shared__ float rh[64];  // per-head factors (per-head mode): heads + kv_heads <= 64
    const int r = blockIdx.x, b = r / p.T, t = r - b * p.T, pos = p.p0 + t;
    const int hd = p.hd, fd = hd / 2, q_dim = p.heads * hd, kv_dim = p.kv_heads * hd;
    const float* q = p.qkv + (size_t)r * p.qkv_stride;
    const float* k = q + q_dim;
    const float* v = k + kv_dim;
    float rq = 1.f, rk = 1.f;
    if (!p.per_head) {
        float sq = 0.f, sk = 0.f;
        for (int i = threadIdx.x; i < q_dim; i += blockDim.x) sq += q[i] * q[i];
        for (int i = threadIdx.x; i < kv_dim; i += blockDim.x) sk += k[i] * k[i];
        sq = block_sum(sq, scratch);
        sk = block_sum(sk, scratch);
        rq = 1.0f / sqrtf(sq / (float)q_dim + p.eps);
        rk = 1.0f / sqrtf(sk / (float)kv_dim + p.eps);
    } else {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        for (int h = wave; h < p.heads + p.kv_heads; h += blockDim.x >> 6) {
            const float* src = h < p.heads ? q + (size_t)h * hd : k + (size_t)(h - p.heads) * hd;
            float s = 0.f;
            for (int i = lane; i < hd; i += 64) s += src[i] * src[i];
            s = wave_sum(s);
            if (lane == 0) rh[h] = 1.0f / sqrtf(s / (float)hd + p.eps);
        }
        __syncthreads();
    }
    const float2* rope = p.rope_tab + (size_t)pos * fd;
    for (int idx = threadIdx.x; idx < p.heads * fd; idx += blockDim.x) {
        const int h = idx / fd, f = idx - h * fd;
        const float s = p.per_head ? rh[h] : rq;
        float x1 = q[(size_t)h * hd + f], x2 = q[(size_t)h * hd + f + fd];
        if (p.q_norm) {
            x1 = (p.q_norm[(size_t)h * hd + f] * x1) * s;
            x2 = (p.q_norm[(size_t)h * hd + f + fd] * x2) * s;
        }
        const float2 cs = rope[f];
        if (p.q32) {
            float* qo = p.q32 + (size_t)r * q_dim + (size_t)h * hd;
            qo[f] = x1 * cs.x - x2 * cs.y;
            qo[f + fd] = x2 * cs.x + x1 * cs.y;
        } else {
            uint16_t* qo = p.qb + (size_t)r * q_dim + (size_t)h * hd;
            qo[f] = f2h(x1 * cs.x - x2 * cs.y, p.rf);
            qo[f + fd] = f2h(x2 * cs.x + x1 * cs.y, p.rf);
        }
    }
    for (int idx = threadIdx.x; idx < p.kv_heads * fd; idx += blockDim.x) {
        const int g = idx / fd, f = idx - g * fd;
        const float s = p.per_head ? rh[p.heads + g] : rk;
        float x1 = k[(size_t)g * hd + f], x2 = k[(size_t)g * hd + f + fd];
        if (p.k_norm) {
            x1 = (p.k_norm[(size_t)g * hd + f] * x1) * s;
            x2 = (p.k_norm[(size_t)g * hd + f + fd] * x2) * s;
        }
        const float2 cs = rope[f];
        const size_t kofs = (((size_t)b * p.kv_heads + g) * p.S + pos) * hd;
        const float o1 = x1 * cs.x - x2 * cs.y, o2 = x2 * cs.x + x1 * cs.y;
        if (p.kv16) {
            reinterpret_cast<uint16_t*>(p.kcache)[kofs + f] = f2h(o1, p.rf);
            reinterpret_cast<uint16_t*>(p.kcache)[kofs + f + fd] = f2h(o2, p.rf);
        } else {
            reinterpret_cast<float*>(p.kcache)[kofs + f] = o1;
            reinterpret_cast<float*>(p.kcache)[kofs + f + fd] = o2;
        }
        if (!p.q32) {
            uint16_t* k16 = p.k16 + (((size_t)b * p.kv_heads + g) * p.Tp + t) * hd;
            k16[f] = f2h(o1, p.rf);
            k16[f + fd] = f2h(o2, p.rf);
        }
    }
    for (int idx = threadIdx.x; idx < kv_dim; idx += blockDim.x) {
        const int g = idx / hd, i = idx - g * hd;
        const size_t vofs = (((size_t)b * p.kv_heads + g) * p.S + pos) * hd + i;
        if (p.kv16)
            reinterpret_cast<uint16_t*>(p.vcache)[vofs] = f2h(v[idx], p.rf);
        else
            reinterpret_cast<float*>(p.vcache)[vofs] = v[idx];
    }
}

// Four fp32 values -> four fp16 (8 bytes, one store).
__device__ inline uint2 pack4h(float a, float b, float c, float d, int* rf) {
    return make_uint2((unsigned)f2h(a, rf) | ((unsigned)f2h(b, rf) << 16),
                      (unsigned)f2h(c, rf) | ((unsigned)f2h(d, rf) << 16));
}

__device__ inline float2 block_sum2(float2 v, float2* scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v.x = wave_sum(v.x);
    v.y = wave_sum(v.y);
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float2 t = make_float2(0.f, 0.f);
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) {
        t.x += scratch[w].x;
        t.y += scratch[w].y;
    }
    return t;
}

// fp32 output form of the fold + row RMSNorm (the fp32-weight prefill's GEMM input): 16-byte
// accesses, the row in registers, every part of a value loaded before the adds (x, then the parts
// in slice order, nparts <= 4); n % 4 == 0, n <= NV * 1024.
template <int NV>
__global__ __launch_bounds__(256) void fold_rmsnorm_rows_f32_v4_kernel(float* x, const float* parts, int nparts,
                                                                        size_t part_stride, const float* w, float* out,
                                                                        int n, float eps) {
    __shared__ float scratch[4];
    const int n4 = n >> 2;
    const size_t row = (size_t)blockIdx.x * n;
    float4* xr = reinterpret_cast<float4*>(x + row);
    float4 v[NV];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            float4 q[4];
#pragma unroll
            for (int s = 0; s < 4; s++)
                if (s < nparts) q[s] = reinterpret_cast<const float4*>(parts + s * part_stride + row)[i];
            float4 a = xr[i];
#pragma unroll
            for (int s = 0; s < 4; s++)
                if (s < nparts) {
                    a.x += q[s].x; a.y += q[s].y; a.z += q[s].z; a.w += q[s].w;
                }
            if (nparts) xr[i] = a;
            v[j] = a;
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
    }
    ss = block_sum(ss, scratch);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    float4* orow = reinterpret_cast<float4*>(out + row);
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            const float4 g = reinterpret_cast<const float4*>(w)[i];
            orow[i] = make_float4((g.x * v[j].x) * r, (g.y * v[j].y) * r, (g.z * v[j].z) * r, (g.w * v[j].w) * r);
        }
    }
}

// The fold + row RMSNorm above with 16-byte accesses and the row held in registers (one read of x
// and of each part, one write of x and of the fp16 row): n % 4 == 0, n <= NV * 1024, nparts <= 4.
// Each value is folded in the same order (x, then parts in slice order), its parts loaded together.
template <int NV>
__global__ __launch_bounds__(256) void fold_rmsnorm_rows_f16_v4_kernel(float* x, const float* parts, int nparts,
                                                                        size_t part_stride, const float* w,
                                                                        uint16_t* out, int n, float eps, int* rf) {
    __shared__ float scratch[4];
    const int n4 = n >> 2;
    const size_t row = (size_t)blockIdx.x * n;
    float4* xr = reinterpret_cast<float4*>(x + row);
    float4 v[NV];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            float4 q[4];  // every part loaded before the adds (nparts <= 4)
#pragma unroll
            for (int s = 0; s < 4; s++)
                if (s < nparts) q[s] = reinterpret_cast<const float4*>(parts + s * part_stride + row)[i];
            float4 a = xr[i];
#pragma unroll
            for (int s = 0; s < 4; s++)
                if (s < nparts) {
                    a.x += q[s].x; a.y += q[s].y; a.z += q[s].z; a.w += q[s].w;
                }
            if (nparts) xr[i] = a;
            v[j] = a;
            ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
    }
    ss = block_sum(ss, scratch);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    uint2* orow = reinterpret_cast<uint2*>(out + row);
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            const float4 g = reinterpret_cast<const float4*>(w)[i];
            orow[i] = pack4h((g.x * v[j].x) * r, (g.y * v[j].y) * r, (g.z * v[j].z) * r, (g.w * v[j].w) * r, rf);
        }
    }
}

// qk_prep_kernel for the whole-vector QK-norm (the reference's) or no QK-norm, with 16-byte accesses
// and the row's q / k held in registers: thread i takes rotation pairs (f .. f+3, f+hd/2 .. +3) of
// query pair-group i (and of key pair-group i), so the norm sums, the rotation and the fp16 / cache
// stores use the values loaded once.  hd % 8 == 0, heads*hd/8 <= QP*256, kv_heads*hd/8 <= 256.
template <int QP>
__global__ __launch_bounds__(256) void qk_prep_v4_kernel(PrepParams p) {
    __shared__ float2 scratch[4];
    const int tid = threadIdx.x;
    const int r = blockIdx.x, b = r / p.T, t = r - b * p.T, pos = p.p0 + t;
    const int hd = p.hd, fd = hd / 2, fd4 = fd / 4, q_dim = p.heads * hd, kv_dim = p.kv_heads * hd;
    const float* q = p.qkv + (size_t)r * p.qkv_stride;
    const float* k = q + q_dim;
    const float* v = k + kv_dim;
    const int nq = p.heads * fd4, nk = p.kv_heads * fd4;
    float4 q1[QP], q2[QP], k1 = make_float4(0.f, 0.f, 0.f, 0.f), k2 = k1;
    float2 ss = make_float2(0.f, 0.f);
    // this thread's first v slice, loaded with q and k so its latency overlaps the norms and rotations
    const float4 v0 = tid < kv_dim / 4 ? reinterpret_cast<const float4*>(v)[tid] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < QP; j++) {
        const int idx = tid + 256 * j;
        if (idx < nq) {
            const int h = idx / fd4, f = (idx - h * fd4) * 4;
            q1[j] = *reinterpret_cast<const float4*>(q + (size_t)h * hd + f);
            q2[j] = *reinterpret_cast<const float4*>(q + (size_t)h * hd + fd + f);
            ss.x += q1[j].x * q1[j].x + q1[j].y * q1[j].y + q1[j].z * q1[j].z + q1[j].w * q1[j].w +
                    q2[j].x * q2[j].x + q2[j].y * q2[j].y + q2[j].z * q2[j].z + q2[j].w * q2[j].w;
        }
    }
    if (tid < nk) {
        const int g = tid / fd4, f = (tid - g * fd4) * 4;
        k1 = *reinterpret_cast<const float4*>(k + (size_t)g * hd + f);
        k2 = *reinterpret_cast<const float4*>(k + (size_t)g * hd + fd + f);
        ss.y = k1.x * k1.x + k1.y * k1.y + k1.z * k1.z + k1.w * k1.w + k2.x * k2.x + k2.y * k2.y + k2.z * k2.z +
               k2.w * k2.w;
    }
    float rq = 1.f, rk = 1.f;
    if (p.q_norm || p.k_norm) {
        ss = block_sum2(ss, scratch);
        rq = 1.0f / sqrtf(ss.x / (float)q_dim + p.eps);
        rk = 1.0f / sqrtf(ss.y / (float)kv_dim + p.eps);
    }
    const float4* rope = reinterpret_cast<const float4*>(p.rope_tab + (size_t)pos * fd);  // (c, s) pairs
    // normalise (g * x) * r and rotate four pairs: out1 = x1 c - x2 s, out2 = x2 c + x1 s
    auto rotate = [&](float4 a, float4 c, const float* gain, size_t goff, float rn, int f, float* o1, float* o2) {
        if (gain) {
            const float4 g1 = *reinterpret_cast<const float4*>(gain + goff + f);
            const float4 g2 = *reinterpret_cast<const float4*>(gain + goff + fd + f);
            a.x = (g1.x * a.x) * rn; a.y = (g1.y * a.y) * rn; a.z = (g1.z * a.z) * rn; a.w = (g1.w * a.w) * rn;
            c.x = (g2.x * c.x) * rn; c.y = (g2.y * c.y) * rn; c.z = (g2.z * c.z) * rn; c.w = (g2.w * c.w) * rn;
        }
        const float4 t0 = rope[f / 2], t1 = rope[f / 2 + 1];  // (c_f, s_f, c_f+1, s_f+1), (c_f+2, ...)
        const float x1[4] = {a.x, a.y, a.z, a.w}, x2[4] = {c.x, c.y, c.z, c.w};
        const float cs[4] = {t0.x, t0.z, t1.x, t1.z}, sn[4] = {t0.y, t0.w, t1.y, t1.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            o1[e] = x1[e] * cs[e] - x2[e] * sn[e];
            o2[e] = x2[e] * cs[e] + x1[e] * sn[e];
        }
    };
#pragma unroll
    for (int j = 0; j < QP; j++) {
        const int idx = tid + 256 * j;
        if (idx < nq) {
            const int h = idx / fd4, f = (idx - h * fd4) * 4;
            float o1[4], o2[4];
            rotate(q1[j], q2[j], p.q_norm, (size_t)h * hd, rq, f, o1, o2);
            if (p.q32) {
                float* qo = p.q32 + (size_t)r * q_dim + (size_t)h * hd;
                *reinterpret_cast<float4*>(qo + f) = make_float4(o1[0], o1[1], o1[2], o1[3]);
                *reinterpret_cast<float4*>(qo + fd + f) = make_float4(o2[0], o2[1], o2[2], o2[3]);
            } else {
                uint16_t* qo = p.qb + (size_t)r * q_dim + (size_t)h * hd;
                *reinterpret_cast<uint2*>(qo + f) = pack4h(o1[0], o1[1], o1[2], o1[3], p.rf);
                *reinterpret_cast<uint2*>(qo + fd + f) = pack4h(o2[0], o2[1], o2[2], o2[3], p.rf);
            }
        }
    }
    if (tid < nk) {
        const int g = tid / fd4, f = (tid - g * fd4) * 4;
        float o1[4], o2[4];
        rotate(k1, k2, p.k_norm, (size_t)g * hd, rk, f, o1, o2);
        const size_t kofs = (((size_t)b * p.kv_heads + g) * p.S + pos) * hd;
        if (p.kv16) {
            uint16_t* kc = reinterpret_cast<uint16_t*>(p.kcache) + kofs;
            *reinterpret_cast<uint2*>(kc + f) = pack4h(o1[0], o1[1], o1[2], o1[3], p.rf);
            *reinterpret_cast<uint2*>(kc + fd + f) = pack4h(o2[0], o2[1], o2[2], o2[3], p.rf);
        } else {
            float* kc = reinterpret_cast<float*>(p.kcache) + kofs;
            *reinterpret_cast<float4*>(kc + f) = make_float4(o1[0], o1[1], o1[2], o1[3]);
            *reinterpret_cast<float4*>(kc + fd + f) = make_float4(o2[0], o2[1], o2[2], o2[3]);
        }
        if (!p.q32) {
            uint16_t* k16 = p.k16 + (((size_t)b * p.kv_heads + g) * p.Tp + t) * hd;
            *reinterpret_cast<uint2*>(k16 + f) = pack4h(o1[0], o1[1], o1[2], o1[3], p.rf);
            *reinterpret_cast<uint2*>(k16 + fd + f) = pack4h(o2[0], o2[1], o2[2], o2[3], p.rf);
        }
    }
    for (int i4 = tid; i4 < kv_dim / 4; i4 += 256) {
        const int g = (4 * i4) / hd, i = 4 * i4 - g * hd;
        const float4 vv = i4 == tid ? v0 : reinterpret_cast<const float4*>(v)[i4];
        const size_t vofs = (((size_t)b * p.kv_heads + g) * p.S + pos) * hd + i;
        if (p.kv16)
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.vcache) + vofs) = pack4h(vv.x, vv.y, vv.z, vv.w, p.rf);
        else
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.vcache) + vofs) = vv;
    }
}

// fp16 Vᵀ tiles of the prompt rows from the V cache: block (tile of 64 rows, KV head, sequence)
// reads 64 contiguous cache rows (16-byte loads) into LDS and writes, per hd row, the 64 keys as
// eight 16-byte chunks of fp16 (rows past the prompt, up to the grid's last tile, are written as 0).
template <int HD, typename KVT>
__global__ __launch_bounds__(256) void vt16_kernel(const KVT* vcache, int S, int p0, int T, int kv_heads,
                                                   uint16_t* vt16, int Tp, int* rf) {
    constexpr int VEC = 16 / sizeof(KVT);  // cache elements per 16-byte load
    __shared__ float tile[64][HD + 1];
    const int t0 = blockIdx.x * 64, g = blockIdx.y, b = blockIdx.z;
    const size_t head = (size_t)b * kv_heads + g;
    const KVT* src = vcache + (head * S + p0) * HD;
    for (int idx = threadIdx.x; idx < 64 * HD / VEC; idx += 256) {
        const int r = idx / (HD / VEC), i = (idx - r * (HD / VEC)) * VEC;
        if (t0 + r < T) {
            typedef KVT vec_t __attribute__((ext_vector_type(VEC)));
            const vec_t v = *reinterpret_cast<const vec_t*>(src + (size_t)(t0 + r) * HD + i);
#pragma unroll
            for (int e = 0; e < VEC; e++) tile[r][i + e] = (float)v[e];
        } else {
#pragma unroll
            for (int e = 0; e < VEC; e++) tile[r][i + e] = 0.f;
        }
    }
    __syncthreads();
    uint16_t* dst = vt16 + head * HD * Tp + t0;
    for (int idx = threadIdx.x; idx < HD * 8; idx += 256) {  // (hd row, chunk of 8 keys)
        const int i = idx >> 3, c = (idx & 7) * 8;
        const uint2 lo = pack4h(tile[c][i], tile[c + 1][i], tile[c + 2][i], tile[c + 3][i], rf);
        const uint2 hi = pack4h(tile[c + 4][i], tile[c + 5][i], tile[c + 6][i], tile[c + 7][i], rf);
        *reinterpret_cast<uint4*>(dst + (size_t)i * Tp + c) = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
}

struct FlashParams {
    const uint16_t* qb;   // [B*T][heads*hd] fp16 queries
    const uint16_t* k16;  // [B][KV][Tp][hd] fp16 keys (prompt rows)
    const uint16_t* vt16; // [B][KV][hd][Tp] fp16 values, transposed
    uint16_t* out;        // [B*T][heads*hd] fp16
    int T, Tp, heads, kv_heads;
    int gsub;   // query heads of one KV group per block (divides heads/kv_heads and 4)
    int nsub;   // (heads/kv_heads) / gsub
    int pairs;  // B * kv_heads
    int nq;     // query blocks of 32 * (4/gsub) rows
};

// Causal attention over the prompt, one 8-wavefront block per (sequence, KV head, query block).
// The 8 wavefronts are NG = 8/KS query groups x KS key slices: a query group is `gsub` query heads
// of the KV group x (NG/gsub) query tiles of 32 rows, and keys advance in super-tiles of SK = 32*KS,
// staged once per block in double-buffered LDS (the next super-tile's global loads are in flight
// while the current one is used); key slice j of a group takes keys 32j .. 32j+31 of each super-tile,
// and the KS partial softmax states are merged through LDS at the end.  KS = 4 (32-row query blocks,
// 128-key super-tiles) when the KV group's heads fit in two groups: causal blocks carry work
// proportional to their last row, so many small blocks dispatched heaviest first balance the CUs
// (a 2048-row prompt of 8 KV pairs makes 512 blocks instead of 256, one per CU, each waiting on the
// longest); KS = 2 (64-key super-tiles) for four heads per group.  Blocks of one (sequence, KV head)
// are placed on one XCD when the pair count allows, so that pair's K/V stays in that XCD's L2.
// Per wave the product is computed transposed so every lane owns one query:
//   S^T (32 keys x 32 queries) = K . Q^T   A = K rows (LDS), B = Q (registers)
//   O^T (hd x 32 queries)     += V^T . P^T A = V^T rows (LDS), B = P^T straight from registers
// In the result layout lane l holds query l%32 and keys (r/4)*8 + (l/32)*4 + r%4 (r = 0..15), so a
// query's 32 scores sit in lanes l and l^32: its max and sum need one shuffle.  The P.V contraction
// runs over keys in that same register order (any order of a sum's terms gives the same sum up to
// rounding), so P^T registers are the B operand as they are, and V^T is read in the matching order.
// Softmax runs in base 2 on scores pre-multiplied by log2(e)/sqrt(hd); the running maximum is only
// raised (and O, l rescaled) when a tile's maximum exceeds it by more than 8, so P <= 2^8 in fp16.
constexpr int kFlashWaves = 8;   // per block: NG query groups x KS key slices

template <int HD, int SK>
struct FlashLds {
    static constexpr int KROW = HD + 8;  // K tile row stride (halves): 16-byte rows, conflict-free b128 reads
    static constexpr int VS = SK + 4;    // V^T tile row stride (halves): conflict-free b64 reads
    static constexpr int K_HALVES = SK * KROW;
    static constexpr int V_HALVES = HD * VS;
    static constexpr int TILE_BYTES = 2 * 2 * (K_HALVES + V_HALVES);  // two buffers of K and V^T
    static constexpr int WRITERS = 8 - 8 / (SK / 32);                 // waves of key slices 1 .. KS-1
    static constexpr int MERGE_BYTES = WRITERS * (HD / 2 + 2) * 64 * 4;  // (O^T + m + l) x 64 lanes each
    static constexpr int BYTES = TILE_BYTES > MERGE_BYTES ? TILE_BYTES : MERGE_BYTES;
};

template <int HD, int KS>
__global__ __launch_bounds__(512) void flash_prefill_kernel(FlashParams p) {
    constexpr int SK = 32 * KS;           // keys per super-tile
    constexpr int NG = 8 / KS;            // query groups
    using L = FlashLds<HD, SK>;
    constexpr int NT = HD / 32;           // 32-row hd tiles of O^T
    constexpr int CPT = HD * SK / 8 / 512;  // 16-byte chunks per thread per super-tile (K and V^T alike)
    __shared__ __attribute__((aligned(16))) unsigned char lds[L::BYTES];
    uint16_t* const ks = reinterpret_cast<uint16_t*>(lds);              // [2][SK][KROW]
    uint16_t* const vs = ks + 2 * L::K_HALVES;                          // [2][HD][VS]

    // (w through readfirstlane: the compiler then treats everything derived from the wavefront index
    // — the key slice, the query rows, the diagonal-tile test — as uniform and branches on it)
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, h2 = lane >> 5,
              lq = lane & 31;
    const int slice = w / NG, wq = w % NG;
    // block -> (unit, query block); unit -> (pair = sequence*KV + g, head subset)
    const int units = p.pairs * p.nsub;
    int unit, qrank;
    if (units % 8 == 0) {
        const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, per = units >> 3;
        unit = xcd + 8 * (slot % per);
        qrank = slot / per;
    } else {
        unit = blockIdx.x % units;
        qrank = blockIdx.x / units;
    }
    const int pair = unit % p.pairs, sub = unit / p.pairs;
    const int b = pair / p.kv_heads, g = pair % p.kv_heads;
    const int qblk = p.nq - 1 - qrank;
    const int rows_blk = 32 * (NG / p.gsub);
    const int h = g * (p.heads / p.kv_heads) + sub * p.gsub + wq % p.gsub;
    const int row0 = qblk * rows_blk + (wq / p.gsub) * 32;
    const int myq = row0 + lq;  // this lane's query row (may be >= T: computed, not stored)
    const int q_dim = p.heads * HD;
    const uint16_t* kb = p.k16 + (size_t)pair * p.Tp * HD;
    const uint16_t* vb = p.vt16 + (size_t)pair * HD * p.Tp;
    const int kend = min(qblk * rows_blk + rows_blk, p.T);  // keys the block needs: 0 .. kend-1
    const int ntiles = (kend + SK - 1) / SK;

    halfx8 qf[HD / 16];  // B operand: query lq, hd (l/32)*8 + 16*kk .. +7
    {
        const int t = min(myq, p.T - 1);
        const uint16_t* qrow = p.qb + ((size_t)b * p.T + t) * q_dim + (size_t)h * HD + h2 * 8;
#pragma unroll
        for (int kk = 0; kk < HD / 16; kk++) qf[kk] = *reinterpret_cast<const halfx8*>(qrow + kk * 16);
    }
    floatx16 o[NT];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[j][r] = 0.f;
    float m = -INFINITY, l = 0.f;
    const float c2 = 1.4426950408889634f / sqrtf((float)HD);

    // super-tile staging: chunk c of K is key row c/(HD/8), halves (c%(HD/8))*8; of V^T, hd row
    // c/(SK/8), keys (c%(SK/8))*8.  Rows k0..k0+SK-1 < Tp always (k0 < T, Tp a multiple of SK).
    // Two register sets alternate, so a super-tile's global loads are issued two iterations
    // before the iteration that stores them into LDS.
    u32x4 kreg[2][CPT], vreg[2][CPT];
    auto load_k = [&](int set, int k0) {
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = tid + 512 * i;
            kreg[set][i] = *reinterpret_cast<const u32x4*>(kb + (size_t)(k0 + c / (HD / 8)) * HD + (c % (HD / 8)) * 8);
        }
    };
    auto load_v = [&](int set, int k0) {
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = tid + 512 * i;
            vreg[set][i] = *reinterpret_cast<const u32x4*>(vb + (size_t)(c / (SK / 8)) * p.Tp + k0 + (c % (SK / 8)) * 8);
        }
    };
    auto load_tile = [&](int set, int k0) { load_k(set, k0); load_v(set, k0); };
    auto store_tile = [&](int set, int buf) {
#pragma unroll
        for (int i = 0; i < CPT; i++) {
            const int c = tid + 512 * i;
            *reinterpret_cast<u32x4*>(ks + buf * L::K_HALVES + (c / (HD / 8)) * L::KROW + (c % (HD / 8)) * 8) =
                kreg[set][i];
            uint2* vd = reinterpret_cast<uint2*>(vs + buf * L::V_HALVES + (c / (SK / 8)) * L::VS + (c % (SK / 8)) * 8);
            vd[0] = make_uint2(vreg[set][i].x, vreg[set][i].y);
            vd[1] = make_uint2(vreg[set][i].z, vreg[set][i].w);
        }
    };
    // block barrier that waits for this wavefront's LDS accesses only: the global loads into the
    // staging registers stay in flight across it (__syncthreads would also wait for them)
    auto lds_barrier = [] {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt not waited on
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // one super-tile for this wavefront's 32 keys kh .. kh+31 (skipped when all are masked)
    auto tile = [&](int t) {
        const int buf = t & 1, kh = t * SK + 32 * slice;
        if (!(kh <= row0 + 31 && kh < p.T)) return;  // every key of the slice is masked for this wave
        const uint16_t* kt = ks + buf * L::K_HALVES + (32 * slice + lq) * L::KROW + h2 * 8;
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; r++) s[r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < HD / 16; kk++)
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const halfx8*>(kt + kk * 16), qf[kk], s, 0, 0,
                                                       0);
        // The causal mask only on the tiles that cross the diagonal or the prompt's end (a uniform
        // branch); the scale c2 > 0 is applied to the maximum and inside the exponent's FMA, so the
        // other tiles spend four vector operations and one exp2 per score.
        const bool edge = (kh + 31 > row0) || (kh + 31 >= p.T);
        if (edge) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = kh + (r >> 2) * 8 + h2 * 4 + (r & 3);
                if (key > myq || key >= p.T) s[r] = -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; r++) mx = fmaxf(mx, s[r]);
        mx = max_xor32(mx) * c2;
        if (__ballot(mx > m + 8.0f)) {
            const float m_new = fmaxf(m, mx);
            const float alpha = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - m_new);
            l *= alpha;
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[j][r] *= alpha;
            m = m_new;
        }
        // a query whose keys so far are all masked keeps m = -inf: its weights are exp2(-inf) = 0
        const float mu = (m == -INFINITY) ? 0.f : m;
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const float e = __builtin_amdgcn_exp2f(fmaf(s[r], c2, -mu));
            s[r] = e;
            sum += e;
        }
        l += sum_xor32(sum);
        // O^T += V^T P^T over the 32 keys, in register order: k-step kk, slot i <-> register 8kk+i
        // <-> key kh + 16kk + 8*(i/4) + (l/32)*4 + i%4
        const uint16_t* vt0 = vs + buf * L::V_HALVES + lq * L::VS + 32 * slice + h2 * 4;
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            halfx8 pf;
#pragma unroll
            for (int i = 0; i < 8; i++) pf[i] = (_Float16)s[8 * kk + i];
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const uint16_t* vt = vt0 + j * 32 * L::VS + 16 * kk;
                const uint2 lo = *reinterpret_cast<const uint2*>(vt);
                const uint2 hi = *reinterpret_cast<const uint2*>(vt + 8);
                const halfx8 vf = __builtin_bit_cast(halfx8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[j], 0, 0, 0);
            }
        }
    };
    // iteration t: LDS buffer t&1 holds tile t; register set (t+1)&1 holds tile t+1 (loaded two
    // iterations ago), which goes into buffer (t+1)&1 (last read in iteration t-1), and then takes
    // the loads of tile t+3; set t&1 holds tile t+2, in flight
    load_tile(0, 0);
    if (ntiles > 1) load_tile(1, SK);
    store_tile(0, 0);
    if (ntiles > 2) load_tile(0, 2 * SK);
    lds_barrier();
    for (int t = 0; t < ntiles; t += 2) {
        // (the register set is a compile-time index in each half of the unrolled pair)
        if (t + 1 < ntiles) store_tile(1, 1);
        if (t + 3 < ntiles) load_k(1, (t + 3) * SK);
        tile(t);
        if (t + 3 < ntiles) load_v(1, (t + 3) * SK);
        lds_barrier();
        if (t + 1 >= ntiles) break;
        if (t + 2 < ntiles) store_tile(0, 0);
        if (t + 4 < ntiles) load_k(0, (t + 4) * SK);
        tile(t + 1);
        if (t + 4 < ntiles) load_v(0, (t + 4) * SK);
        lds_barrier();
    }
    // merge key slices 1 .. KS-1 into slice 0 (the tile buffers are free after the last barrier)
    float* const mg0 = reinterpret_cast<float*>(lds) + lane;  // [writer][value][lane], writer = (slice-1)*NG + wq
    if (slice > 0) {
        float* mg = mg0 + ((slice - 1) * NG + wq) * (HD / 2 + 2) * 64;
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) mg[(j * 16 + r) * 64] = o[j][r];
        mg[(HD / 2) * 64] = m;
        mg[(HD / 2 + 1) * 64] = l;
    }
    __syncthreads();
    if (slice > 0 || myq >= p.T) return;
    // m is finite: key 0 is in slice 0's first super-tile; slices whose keys were all masked keep -inf
    float m_all = m;
#pragma unroll
    for (int j = 1; j < KS; j++) m_all = fmaxf(m_all, mg0[(((j - 1) * NG + wq) * (HD / 2 + 2) + HD / 2) * 64]);
    float wgt[KS], den;
    wgt[0] = __builtin_amdgcn_exp2f(m - m_all);
    den = l * wgt[0];
#pragma unroll
    for (int j = 1; j < KS; j++) {
        const float* mg = mg0 + ((j - 1) * NG + wq) * (HD / 2 + 2) * 64;
        const float ms = mg[(HD / 2) * 64];
        wgt[j] = (ms == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms - m_all);
        den = fmaf(mg[(HD / 2 + 1) * 64], wgt[j], den);
    }
    const float inv = 1.0f / den;
    uint16_t* orow = p.out + ((size_t)b * p.T + myq) * q_dim + (size_t)h * HD;
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float v = o[j][r] * wgt[0];
#pragma unroll
            for (int k = 1; k < KS; k++) v = fmaf(mg0[(((k - 1) * NG + wq) * (HD / 2 + 2) + j * 16 + r) * 64], wgt[k], v);
            orow[j * 32 + (r >> 2) * 8 + h2 * 4 + (r & 3)] = f2h(v * inv);
        }
}

}  // namespace

int launch_embed_rows(const void* table, int wdtype, int dim, const int* tokens, int token_stride, int T, int rows,
                      float* x, hipStream_t stream) {
    AR_CHECK_ARG(table && tokens && x && rows > 0 && dim > 0 && T > 0, "embed rows: bad arguments");
    if (wdtype == AR_DTYPE_BF16)
        hipLaunchKernelGGL(embed_rows_kernel<uint16_t>, dim3(rows), dim3(256), 0, stream, (const uint16_t*)table, dim,
                           tokens, token_stride, T, x);
    else
        hipLaunchKernelGGL(embed_rows_kernel<float>, dim3(rows), dim3(256), 0, stream, (const float*)table, dim,
                           tokens, token_stride, T, x);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_rmsnorm_rows_f16(const float* x, const float* w, uint16_t* out, int rows, int n, float eps,
                            int* range_flag, hipStream_t stream) {
    AR_CHECK_ARG(x && w && out && rows > 0 && n > 0, "rmsnorm rows: bad arguments");
    hipLaunchKernelGGL(rmsnorm_rows_f16_kernel, dim3(rows), dim3(256), 0, stream, x, w, out, n, eps, range_flag);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_fold_rmsnorm_rows_f16(float* x, const float* parts, int nparts, const float* w, uint16_t* out, int rows,
                                 int n, float eps, int* range_flag, hipStream_t stream) {
    AR_CHECK_ARG(x && w && out && rows > 0 && n > 0 && nparts >= 0 && (parts || nparts == 0),
                 "fold rmsnorm rows: bad arguments");
    const bool v4 = n % 4 == 0 && n <= 4096 && nparts <= 4 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(w) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0 &&
                    (nparts == 0 || (reinterpret_cast<uintptr_t>(parts) & 15) == 0);
    if (v4 && n <= 1024)
        hipLaunchKernelGGL(fold_rmsnorm_rows_f16_v4_kernel<1>, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps, range_flag);
    else if (v4 && n <= 2048)
        hipLaunchKernelGGL(fold_rmsnorm_rows_f16_v4_kernel<2>, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps, range_flag);
    else if (v4)
        hipLaunchKernelGGL(fold_rmsnorm_rows_f16_v4_kernel<4>, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps, range_flag);
    else
        hipLaunchKernelGGL(fold_rmsnorm_rows_f16_kernel, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps, range_flag);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_fold_rmsnorm_rows_f32(float* x, const float* parts, int nparts, const float* w, float* out, int rows,
                                 int n, float eps, hipStream_t stream) {
    AR_CHECK_ARG(x && w && out && rows > 0 && n > 0 && nparts >= 0 && (parts || nparts == 0),
                 "fold rmsnorm rows: bad arguments");
    const bool v4 = n % 4 == 0 && n <= 4096 && nparts <= 4 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(w) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                    (nparts == 0 || (reinterpret_cast<uintptr_t>(parts) & 15) == 0);
    if (v4 && n <= 1024)
        hipLaunchKernelGGL(fold_rmsnorm_rows_f32_v4_kernel<1>, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps);
    else if (v4 && n <= 2048)
        hipLaunchKernelGGL(fold_rmsnorm_rows_f32_v4_kernel<2>, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps);
    else if (v4)
        hipLaunchKernelGGL(fold_rmsnorm_rows_f32_v4_kernel<4>, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps);
    else
        hipLaunchKernelGGL(fold_rmsnorm_rows_f32_kernel, dim3(rows), dim3(256), 0, stream, x, parts, nparts,
                           (size_t)rows * n, w, out, n, eps);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_fold_rows(const float* src, const float* parts, int nparts, size_t part_rows, int first, int step,
                     int count, int n, float* dst, hipStream_t stream) {
    AR_CHECK_ARG(src && dst && count > 0 && n > 0 && nparts >= 0 && (parts || nparts == 0), "fold rows: bad arguments");
    hipLaunchKernelGGL(fold_rows_kernel, dim3(count), dim3(256), 0, stream, src, parts, nparts, part_rows * n, first,
                       step, n, dst);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_qk_prep(const PrefillPrep& a, hipStream_t stream) {
    AR_CHECK_ARG(a.qkv && a.rope_tab && a.kcache && a.vcache && (a.q32 || (a.qb && a.k16 && a.vt16)),
                 "qk prep: null pointer");
    AR_CHECK_ARG(a.q32 || a.Tp >= a.T, "qk prep: fp16 copies hold %d rows, %d needed", a.Tp, a.T);
    AR_CHECK_ARG(!a.q32 || !a.kv16, "qk prep: the fp32 path keeps an fp32 cache");
    AR_CHECK_ARG(a.heads + a.kv_heads <= 64, "qk prep: too many heads");
    AR_CHECK_ARG(a.p0 >= 0 && a.p0 + a.T <= a.S, "qk prep: rows %d..%d outside the %d-row cache", a.p0, a.p0 + a.T,
                 a.S);
    PrepParams p;
    p.qkv = a.qkv; p.qkv_stride = a.qkv_stride; p.q_norm = a.q_norm; p.k_norm = a.k_norm; p.eps = a.eps;
    p.per_head = a.per_head; p.rope_tab = a.rope_tab; p.kcache = a.kcache; p.vcache = a.vcache; p.S = a.S;
    p.kv16 = a.kv16;
    p.T = a.T; p.p0 = a.p0; p.heads = a.heads; p.kv_heads = a.kv_heads; p.hd = a.hd; p.qb = a.qb;
    p.k16 = a.k16; p.Tp = a.Tp; p.rf = a.range_flag; p.q32 = a.q32;
    const int nq = a.heads * a.hd / 8, nk = a.kv_heads * a.hd / 8;
    const bool v4 = !a.per_head && a.hd % 8 == 0 && a.qkv_stride % 4 == 0 && nk <= 256 && nq <= 4 * 256 &&
                    (reinterpret_cast<uintptr_t>(a.qkv) & 15) == 0 &&
                    (!a.q_norm || (reinterpret_cast<uintptr_t>(a.q_norm) & 15) == 0) &&
                    (!a.k_norm || (reinterpret_cast<uintptr_t>(a.k_norm) & 15) == 0) &&
                    (reinterpret_cast<uintptr_t>(a.rope_tab) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.qb) & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(a.k16) & 7) == 0 && (reinterpret_cast<uintptr_t>(a.q32) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(a.kcache) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(a.vcache) & 15) == 0;
    if (v4 && nq <= 256)
        hipLaunchKernelGGL(qk_prep_v4_kernel<1>, dim3(a.B * a.T), dim3(256), 0, stream, p);
    else if (v4 && nq <= 512)
        hipLaunchKernelGGL(qk_prep_v4_kernel<2>, dim3(a.B * a.T), dim3(256), 0, stream, p);
    else if (v4)
        hipLaunchKernelGGL(qk_prep_v4_kernel<4>, dim3(a.B * a.T), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(qk_prep_kernel, dim3(a.B * a.T), dim3(256), 0, stream, p);
    AR_LAUNCH_CHECK();
    if (a.q32) return AR_HIP_OK;  // fp32 path: attention reads the fp32 cache rows directly
    AR_CHECK_ARG(a.Tp % 128 == 0 && a.Tp >= a.T, "qk prep: Vᵀ rows %d not a multiple of 128 covering %d", a.Tp, a.T);
    // whole 128-key super-tiles of the flash pass: rows T .. up to the next multiple of 128 are written
    // as 0, so a masked key (weight 0) never meets a stale infinity of an earlier, longer prompt
    const dim3 vgrid((a.T + 127) / 128 * 2, a.kv_heads, a.B);
#define AR_VT16(HDV, T_)                                                                                     \
    hipLaunchKernelGGL((vt16_kernel<HDV, T_>), vgrid, dim3(256), 0, stream, reinterpret_cast<const T_*>(a.vcache), \
                       a.S, a.p0, a.T, a.kv_heads, a.vt16, a.Tp, a.range_flag)
    if (a.hd != 128 && a.hd != 64) {
        ar_set_error("qk prep: head_dim %d not supported (64, 128)", a.hd);
        return AR_HIP_ERR_INVALID;
    }
    if (a.hd == 128 && a.kv16)
        AR_VT16(128, _Float16);
    else if (a.hd == 128)
        AR_VT16(128, float);
    else if (a.kv16)
        AR_VT16(64, _Float16);
    else
        AR_VT16(64, float);
#undef AR_VT16
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_flash_prefill(const uint16_t* qb, const uint16_t* k16, const uint16_t* vt16, uint16_t* out, int B, int T,
                         int Tp, int heads, int kv_heads, int hd, hipStream_t stream) {
    AR_CHECK_ARG(qb && k16 && vt16 && out && T > 0 && B > 0, "flash prefill: bad arguments");
    AR_CHECK_ARG(heads % kv_heads == 0 && Tp >= T, "flash prefill: bad shape");
    FlashParams p;
    p.qb = qb; p.k16 = k16; p.vt16 = vt16; p.out = out; p.T = T; p.Tp = Tp; p.heads = heads; p.kv_heads = kv_heads;
    const int G = heads / kv_heads;
    p.gsub = (G % 4 == 0) ? 4 : (G % 2 == 0) ? 2 : 1;
    p.nsub = G / p.gsub;
    p.pairs = B * kv_heads;
    // four key slices (two query groups of 32 rows) unless the group holds four heads
    const int KS = p.gsub == 4 ? 2 : 4;
    AR_CHECK_ARG(Tp % (32 * KS) == 0, "flash prefill: Tp=%d not a multiple of the %d-key super-tile", Tp, 32 * KS);
    const int rows_blk = 32 * ((8 / KS) / p.gsub);
    p.nq = (T + rows_blk - 1) / rows_blk;
    const long long blocks = (long long)p.nq * p.pairs * p.nsub;
    AR_CHECK_ARG(blocks <= 0x7fffffff, "flash prefill: too many blocks");
    dim3 grid((unsigned)blocks);
#define AR_FLASH(HDV, KSV) hipLaunchKernelGGL((flash_prefill_kernel<HDV, KSV>), grid, dim3(512), 0, stream, p)
    if (hd == 128 && KS == 4)
        AR_FLASH(128, 4);
    else if (hd == 128)
        AR_FLASH(128, 2);
    else if (hd == 64 && KS == 4)
        AR_FLASH(64, 4);
    else if (hd == 64)
        AR_FLASH(64, 2);
    else {
        ar_set_error("flash prefill: head_dim %d not supported", hd);
        return AR_HIP_ERR_INVALID;
    }
#undef AR_FLASH
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}
