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

// fp32 -> fp16 bits (round to nearest even)
__device__ inline uint16_t f2h(float f) {
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
                                                                int n, float eps) {
    __shared__ float scratch[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += xr[i] * xr[i];
    ss = block_sum(ss, scratch);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[(size_t)blockIdx.x * n + i] = f2h((w[i] * xr[i]) * r);
}

struct PrepParams {
    const float* qkv;       // [R][qkv_stride] raw projections
    int qkv_stride;
    const float* q_norm;
    const float* k_norm;
    float eps;
    int per_head;
    const float2* rope_tab; // [S][hd/2]
    float* kcache;          // [B][KV][S][hd]
    float* vcache;
    int S, T, p0, heads, kv_heads, hd;
    uint16_t* qb;           // [R][heads*hd] fp16 normalised, rotated queries
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
        uint16_t* qo = p.qb + (size_t)r * q_dim + (size_t)h * hd;
        qo[f] = f2h(x1 * cs.x - x2 * cs.y);
        qo[f + fd] = f2h(x2 * cs.x + x1 * cs.y);
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
        float* kc = p.kcache + (((size_t)b * p.kv_heads + g) * p.S + pos) * hd;
        kc[f] = x1 * cs.x - x2 * cs.y;
        kc[f + fd] = x2 * cs.x + x1 * cs.y;
    }
    for (int idx = threadIdx.x; idx < kv_dim; idx += blockDim.x) {
        const int g = idx / hd, i = idx - g * hd;
        p.vcache[(((size_t)b * p.kv_heads + g) * p.S + pos) * hd + i] = v[idx];
    }
}

struct FlashParams {
    const uint16_t* qb;   // [B*T][heads*hd] fp16
    const float* kcache;  // [B][KV][S][hd]
    const float* vcache;
    uint16_t* out;        // [B*T][heads*hd] fp16
    int S, T, p0, heads, kv_heads;
};

// Causal attention for a tile of 128 query rows (4 wavefronts x 32 rows) of one head, over key
// tiles of 32 rows with an online softmax.  S = Q K^T and O += P V run on
// v_mfma_f32_32x32x16_f16; K and V tiles are converted to fp16 in LDS (V transposed, so a lane
// can read 8 consecutive keys of one column); P goes through LDS to change from the result layout
// (column = key) to the operand layout (row = query, 8 consecutive keys).
template <int HD>
__global__ __launch_bounds__(256) void flash_prefill_kernel(FlashParams p) {
    constexpr int BQ = 128, BKV = 32;
    constexpr int KS = HD + 8;   // LDS row stride of the K tile (fp16)
    constexpr int VS = BKV + 8;  // LDS row stride of the transposed V tile (fp16)
    constexpr int PS = BKV + 8;  // LDS row stride of a wave's P tile
    constexpr int NT = HD / 32;  // 32-column output tiles
    __shared__ __attribute__((aligned(16))) uint16_t ks[BKV * KS];
    __shared__ __attribute__((aligned(16))) uint16_t vt[HD * VS];
    __shared__ __attribute__((aligned(16))) uint16_t ps[4][32 * PS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int g = h / (p.heads / p.kv_heads);
    const int q_dim = p.heads * HD;
    const int row0 = qt * BQ + wave * 32;  // first query row (within the sequence) of this wave
    const float* kc = p.kcache + ((size_t)b * p.kv_heads + g) * (size_t)p.S * HD;
    const float* vc = p.vcache + ((size_t)b * p.kv_heads + g) * (size_t)p.S * HD;

    // this wave's queries in operand layout: row l%32, hd (l/32)*8 + 16*kk .. +7
    halfx8 qf[HD / 16];
    {
        const int t = min(row0 + (lane & 31), p.T - 1);
        const uint16_t* qrow = p.qb + ((size_t)b * p.T + t) * q_dim + (size_t)h * HD + (lane >> 5) * 8;
#pragma unroll
        for (int kk = 0; kk < HD / 16; kk++) qf[kk] = *reinterpret_cast<const halfx8*>(qrow + kk * 16);
    }
    floatx16 o[NT];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[j][r] = 0.f;
    float m_r[16], l_r[16];
#pragma unroll
    for (int r = 0; r < 16; r++) { m_r[r] = -INFINITY; l_r[r] = 0.f; }
    const float scale = sqrtf((float)HD);

    // keys 0 .. p0 + (last query row of the block)
    const int qlast = min(qt * BQ + BQ, p.T) - 1;
    const int kend = p.p0 + qlast + 1;
    for (int k0 = 0; k0 < kend; k0 += BKV) {
        __syncthreads();  // previous tile's LDS reads are done
        // K tile -> ks[key][hd], V tile -> vt[hd][key], as fp16 (rows past kend are clamped;
        // the causal mask drops them)
        for (int e = tid * 4; e < BKV * HD; e += 256 * 4) {
            const int kr = e / HD, c = e - kr * HD;
            const int key = min(k0 + kr, kend - 1);
            const float4 kv4 = *reinterpret_cast<const float4*>(kc + (size_t)key * HD + c);
            const float4 vv4 = *reinterpret_cast<const float4*>(vc + (size_t)key * HD + c);
            uint16_t* kd = &ks[kr * KS + c];
            kd[0] = f2h(kv4.x); kd[1] = f2h(kv4.y); kd[2] = f2h(kv4.z); kd[3] = f2h(kv4.w);
            vt[(c + 0) * VS + kr] = f2h(vv4.x);
            vt[(c + 1) * VS + kr] = f2h(vv4.y);
            vt[(c + 2) * VS + kr] = f2h(vv4.z);
            vt[(c + 3) * VS + kr] = f2h(vv4.w);
        }
        __syncthreads();
        if (k0 > p.p0 + row0 + 31) continue;  // every key of this tile is after this wave's rows

        // S = Q K^T for 32 rows x 32 keys
        floatx16 s;
#pragma unroll
        for (int r = 0; r < 16; r++) s[r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < HD / 16; kk++) {
            const halfx8 kf = *reinterpret_cast<const halfx8*>(&ks[(lane & 31) * KS + kk * 16 + (lane >> 5) * 8]);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(qf[kk], kf, s, 0, 0, 0);
        }
        // mask, online softmax; lane holds key k0 + lane%32 for rows (r/4)*8 + (lane/32)*4 + r%4
        const int key = k0 + (lane & 31);
        float alpha[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int qrow = row0 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            float v = s[r] / scale;
            if (key > p.p0 + qrow) v = -INFINITY;
            float mx = v;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            const float m_new = fmaxf(m_r[r], mx);
            const float e = (v == -INFINITY) ? 0.f : expf(v - m_new);
            float sum = e;
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) sum += __shfl_xor(sum, off, 64);
            alpha[r] = (m_r[r] == -INFINITY) ? 0.f : expf(m_r[r] - m_new);
            l_r[r] = l_r[r] * alpha[r] + sum;
            m_r[r] = m_new;
            s[r] = e;
        }
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[j][r] *= alpha[r];
        // P (result layout) -> LDS -> operand layout
        uint16_t* pw = ps[wave];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int prow = (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            pw[prow * PS + (lane & 31)] = f2h(s[r]);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's P writes are in LDS
#pragma unroll
        for (int kk = 0; kk < BKV / 16; kk++) {
            const halfx8 pf = *reinterpret_cast<const halfx8*>(&pw[(lane & 31) * PS + kk * 16 + (lane >> 5) * 8]);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const halfx8 vf =
                    *reinterpret_cast<const halfx8*>(&vt[(j * 32 + (lane & 31)) * VS + kk * 16 + (lane >> 5) * 8]);
                o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pf, vf, o[j], 0, 0, 0);
            }
        }
    }
    // normalise and store
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int qrow = row0 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (qrow >= p.T) continue;
        const float inv = 1.0f / l_r[r];
        uint16_t* orow = p.out + ((size_t)b * p.T + qrow) * q_dim + (size_t)h * HD;
#pragma unroll
        for (int j = 0; j < NT; j++) orow[j * 32 + (lane & 31)] = f2h(o[j][r] * inv);
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
                            hipStream_t stream) {
    AR_CHECK_ARG(x && w && out && rows > 0 && n > 0, "rmsnorm rows: bad arguments");
    hipLaunchKernelGGL(rmsnorm_rows_f16_kernel, dim3(rows), dim3(256), 0, stream, x, w, out, n, eps);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_qk_prep(const PrefillPrep& a, hipStream_t stream) {
    AR_CHECK_ARG(a.qkv && a.rope_tab && a.kcache && a.vcache && a.qb, "qk prep: null pointer");
    AR_CHECK_ARG(a.heads + a.kv_heads <= 64, "qk prep: too many heads");
    AR_CHECK_ARG(a.p0 >= 0 && a.p0 + a.T <= a.S, "qk prep: rows %d..%d outside the %d-row cache", a.p0, a.p0 + a.T,
                 a.S);
    PrepParams p;
    p.qkv = a.qkv; p.qkv_stride = a.qkv_stride; p.q_norm = a.q_norm; p.k_norm = a.k_norm; p.eps = a.eps;
    p.per_head = a.per_head; p.rope_tab = a.rope_tab; p.kcache = a.kcache; p.vcache = a.vcache; p.S = a.S;
    p.T = a.T; p.p0 = a.p0; p.heads = a.heads; p.kv_heads = a.kv_heads; p.hd = a.hd; p.qb = a.qb;
    hipLaunchKernelGGL(qk_prep_kernel, dim3(a.B * a.T), dim3(256), 0, stream, p);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

int launch_flash_prefill(const uint16_t* qb, const float* kcache, const float* vcache, uint16_t* out, int B, int S,
                         int T, int p0, int heads, int kv_heads, int hd, hipStream_t stream) {
    AR_CHECK_ARG(qb && kcache && vcache && out && T > 0 && B > 0, "flash prefill: bad arguments");
    AR_CHECK_ARG(heads % kv_heads == 0 && p0 >= 0 && p0 + T <= S, "flash prefill: bad shape");
    FlashParams p;
    p.qb = qb; p.kcache = kcache; p.vcache = vcache; p.out = out; p.S = S; p.T = T; p.p0 = p0; p.heads = heads;
    p.kv_heads = kv_heads;
    dim3 grid((T + 127) / 128, heads, B);
    if (hd == 128)
        hipLaunchKernelGGL(flash_prefill_kernel<128>, grid, dim3(256), 0, stream, p);
    else if (hd == 64)
        hipLaunchKernelGGL(flash_prefill_kernel<64>, grid, dim3(256), 0, stream, p);
    else {
        ar_set_error("flash prefill: head_dim %d not supported", hd);
        return AR_HIP_ERR_INVALID;
    }
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}
