// Decode-step grouped-query attention with the QK-norm / RoPE / KV-cache-write prologue fused in.
//
// One launch covers what the reference builds as a chain of graph ops per layer
// (engine/ml/.../AttentionFeatures.java:785-929):
//   QK-norm        rmsnorm over the whole q / k vector (:840-845, :886-891) or per head
//   split-half RoPE reshapeToSplitHalfRope + ropeRotation + reshapeFromSplitHalfRope
//                  (:195-237; RotationFeatures.java:124-208), angles pos * exp(f * -2 ln(theta)/hd)
//                  evaluated in double
//   cache write    k, v at row pos (:858-864, :871-877; CollectionReceptor.java:95-105)
//   scores         q . K[t] / sqrt(hd) (attentionKeysStandard :531-559)
//   causal mask    rows t > pos are never visited; the reference adds -10000 there (:906-917),
//                  whose exp underflows to exactly 0, so skipping them is identical
//   softmax        max-subtracted (ActivationFeatures.java:135-143), computed online per split
//   values         sum_t a[t] V[t] (attentionValuesStandard :572-616)
//
// Layout: caches are compact and head-major, (batch, kv_heads, max_seq, hd) fp32; query head h
// reads KV head h / (heads / kv_heads), which holds exactly what the reference's GQA-expanded
// cache copy (:823-826) holds.
//
// Grid (max_splits, kv_heads, batch), 256 threads.  The live context [0, pos] is cut into
// nsplit contiguous splits of >= 16 rows (at most max_splits); block (s, g, b) handles split s
// for the heads/kv_heads query heads sharing KV head g:
//   phase 1: 16-lane groups compute one row's scores for all heads of the group (K row read once)
//   phase 2: each wavefront accumulates a[t] * V[t] for every fourth row (V row read once)
// Both phases walk the split in passes of 64 rows with the next pass's loads in flight.
// With one split the block writes the normalised output; otherwise it writes unnormalised
// partials (o, max, sum) that attn_combine_kernel merges in the next launch (the kernel boundary
// makes them visible, so no block needs a device-wide fence).
#include "ar_hip_internal.h"

namespace {

constexpr int kThreads = 256;   // threads of the split (multi-block) form
constexpr int kMaxTile = 256;   // rows per split in that form
constexpr int kShortMax = 256;  // caches up to this many rows: one block per (sequence, KV head)
constexpr int kMaxSplits = 1024;

struct AttnParams {
    const float* qkv;
    int qkv_stride;
    const float* q_norm;
    const float* k_norm;
    float qk_eps;
    int per_head_norm;
    float* kcache;
    float* vcache;
    int max_seq;
    const int* pos;
    int heads, kv_heads;
    double rope_c;  // -2 ln(theta) / hd
    const float2* rope_tab;  // [max_seq][hd/2] (cos, sin) or null
    int max_splits;
    float* part_o;
    float* part_ml;
    float* out;
    int out_stride;
};

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Block-wide sum of per-thread values; every thread gets the result.
template <int NT>
__device__ inline float block_sum(float v, float* scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) t += scratch[w];
    return t;
}

// Split plan for a live context of n rows: nsplit splits of `tile` rows (the last may be short).
__device__ inline void split_plan(int n, int max_splits, int* nsplit, int* tile) {
    int ns = min(max_splits, (n + 15) / 16);
    if (ns < 1) ns = 1;
    const int t = (n + ns - 1) / ns;
    *tile = t;
    *nsplit = (n + t - 1) / t;
}

// (cos, sin) of pos * exp(f * -2 ln(theta) / hd): from the table the model precomputes in
// double on the host, or evaluated here in double when no table is given.
__device__ inline void rope_cs(const float2* row, int pos, int f, double c, float* cs, float* sn) {
    if (row) {
        const float2 t = row[f];
        *cs = t.x;
        *sn = t.y;
        return;
    }
    const double invf = exp((double)f * c);
    const double ang = (double)pos * invf;
    *cs = (float)cos(ang);
    *sn = (float)sin(ang);
}

// NT threads: 256 when the context is cut into splits across blocks, 512 / 1024 for a context of
// at most kShortMax rows handled by one block per (sequence, KV head) with no combine launch.
template <int HD, int G, int NT>
__global__ __launch_bounds__(NT) void attn_decode_kernel(AttnParams p) {
    constexpr int FD = HD / 2;
    constexpr int EPL = HD / 16;     // elements per lane in a 16-lane row group (phase 1)
    constexpr int VPL = HD / 64;     // value columns per lane (phase 2)
    constexpr int NG = NT / 16;                // 16-lane row groups (phase 1)
    constexpr int NWV = NT / 64;               // wavefronts (phase 2)
    constexpr int KU = NT == 1024 ? 2 : 4;     // K rows per group per pass
    constexpr int VU = NT == 1024 ? 8 : 16;    // V rows per wavefront per pass
    constexpr int PASS1 = NG * KU, PASS2 = NWV * VU;
    constexpr int TILE = NT == 256 ? kMaxTile : kShortMax;
    __shared__ __attribute__((aligned(16))) float q_s[G][HD];
    __shared__ __attribute__((aligned(16))) float k_new[HD];
    __shared__ __attribute__((aligned(16))) float v_new[HD];
    __shared__ float s_s[G][TILE];
    __shared__ __attribute__((aligned(16))) float red_s[NWV][G][HD];
    __shared__ float m_s[G], l_s[G];
    __shared__ float scratch[NWV];
    __shared__ float rq_s[G], rk_s;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid >> 4, gl = tid & 15;
    const int b = blockIdx.z, kvh = blockIdx.y, split = blockIdx.x;
    const int heads = p.heads, kvH = p.kv_heads;
    const int q_dim = heads * HD, kv_dim = kvH * HD;
    const float* q_raw = p.qkv + (size_t)b * p.qkv_stride;
    const float* k_raw = q_raw + q_dim;
    const float* v_raw = k_raw + kv_dim;
    const bool whole_norm = (p.q_norm || p.k_norm) && !p.per_head_norm;

    // ---- every load that does not depend on the position, issued together with it ----------
    const int pos = *p.pos;
    constexpr int QPT = (G * FD + NT - 1) / NT;  // query (f, f+hd/2) pairs per thread
    float qx1[QPT], qx2[QPT], qg1[QPT], qg2[QPT];
#pragma unroll
    for (int j = 0; j < QPT; j++) {
        const int idx = min(tid + j * NT, G * FD - 1);
        const int g = idx / FD, f = idx - g * FD;
        const size_t off = (size_t)(kvh * G + g) * HD + f;
        qx1[j] = q_raw[off];
        qx2[j] = q_raw[off + FD];
        qg1[j] = p.q_norm ? p.q_norm[off] : 1.f;
        qg2[j] = p.q_norm ? p.q_norm[off + FD] : 1.f;
    }
    const int kf = min(tid, FD - 1);
    const float kx1 = k_raw[(size_t)kvh * HD + kf], kx2 = k_raw[(size_t)kvh * HD + kf + FD];
    const float kg1 = p.k_norm ? p.k_norm[(size_t)kvh * HD + kf] : 1.f;
    const float kg2 = p.k_norm ? p.k_norm[(size_t)kvh * HD + kf + FD] : 1.f;
    const float vnew = v_raw[(size_t)kvh * HD + min(tid, HD - 1)];
    float sq = 0.f, sk = 0.f;  // this thread's share of sum(q^2), sum(k^2) over the whole vectors
    if (whole_norm) {
#pragma unroll 4
        for (int i = tid * 4; i < q_dim; i += NT * 4) {
            const float4 v = *reinterpret_cast<const float4*>(q_raw + i);
            sq += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
#pragma unroll 2
        for (int i = tid * 4; i < kv_dim; i += NT * 4) {
            const float4 v = *reinterpret_cast<const float4*>(k_raw + i);
            sk += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    }

    if (pos < 0 || pos >= p.max_seq) return;
    const int n = pos + 1;
    int nsplit, tile;
    split_plan(n, p.max_splits, &nsplit, &tile);
    if (split >= nsplit) return;
    const int t0 = split * tile;
    const int t1 = min(t0 + tile, n);
    const size_t head_base = ((size_t)b * kvH + kvh) * (size_t)p.max_seq * HD;
    float* kc = p.kcache + head_base;
    float* vc = p.vcache + head_base;

    // ---- first pass of K and V rows, issued before anything that depends on the QKV kernel.
    // Rows are clamped to the split (duplicates are dropped below); row `pos` is stale in the
    // cache until this block writes it, so that row is taken from LDS instead.
    float kr[KU][EPL];
    float vr[VU][VPL];
    auto load_k = [&](float (&dst)[KU][EPL], int base) {
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int t = min(base + grp + NG * u, t1 - 1);
#pragma unroll
            for (int j = 0; j < EPL / 4; j++) {
                const float4 v = *reinterpret_cast<const float4*>(kc + (size_t)t * HD + j * 64 + gl * 4);
                dst[u][j * 4] = v.x; dst[u][j * 4 + 1] = v.y; dst[u][j * 4 + 2] = v.z; dst[u][j * 4 + 3] = v.w;
            }
        }
    };
    auto load_v = [&](float (&dst)[VU][VPL], int base) {
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = min(base + wave + NWV * u, t1 - 1);
            if constexpr (VPL == 2) {
                const float2 v = *reinterpret_cast<const float2*>(vc + (size_t)t * HD + lane * 2);
                dst[u][0] = v.x; dst[u][1] = v.y;
            } else {
                dst[u][0] = vc[(size_t)t * HD + lane];
            }
        }
    };
    load_k(kr, t0);
    load_v(vr, t0);
    const float2* rope_row = p.rope_tab ? p.rope_tab + (size_t)pos * FD : nullptr;
    float2 qcs[QPT], kcs;
#pragma unroll
    for (int j = 0; j < QPT; j++) {
        const int idx = min(tid + j * NT, G * FD - 1);
        rope_cs(rope_row, pos, idx % FD, p.rope_c, &qcs[j].x, &qcs[j].y);
    }
    rope_cs(rope_row, pos, kf, p.rope_c, &kcs.x, &kcs.y);

    // ---- QK-norm factors ----------------------------------------------------------
    if (p.q_norm || p.k_norm) {
        if (whole_norm) {
            sq = block_sum<NT>(sq, scratch);
            sk = block_sum<NT>(sk, scratch);
            if (tid == 0) {
                const float rq = 1.0f / sqrtf(sq / (float)q_dim + p.qk_eps);
                for (int g = 0; g < G; g++) rq_s[g] = rq;
                rk_s = 1.0f / sqrtf(sk / (float)kv_dim + p.qk_eps);
            }
        } else {
            // wave w reduces heads w, w+4, ...; the k head goes to the last slot
            for (int j = wave; j < G + 1; j += NWV) {
                const float* src = (j < G) ? q_raw + (size_t)(kvh * G + j) * HD : k_raw + (size_t)kvh * HD;
                float s = 0.f;
                for (int i = lane; i < HD; i += 64) s += src[i] * src[i];
                s = wave_sum(s);
                if (lane == 0) {
                    const float r = 1.0f / sqrtf(s / (float)HD + p.qk_eps);
                    if (j < G) rq_s[j] = r; else rk_s = r;
                }
            }
        }
        __syncthreads();
    }

    // ---- normalised, rotated queries of this group -> LDS ---------------------------
#pragma unroll
    for (int j = 0; j < QPT; j++) {
        const int idx = tid + j * NT;
        if (idx < G * FD) {
            const int g = idx / FD, f = idx - g * FD;
            float x1 = qx1[j], x2 = qx2[j];
            if (p.q_norm) {
                x1 = (qg1[j] * x1) * rq_s[g];
                x2 = (qg2[j] * x2) * rq_s[g];
            }
            q_s[g][f] = x1 * qcs[j].x - x2 * qcs[j].y;
            q_s[g][f + FD] = x2 * qcs[j].x + x1 * qcs[j].y;
        }
    }
    // ---- the split holding `pos` writes this step's k and v rows (cache + LDS) ---------
    const bool has_pos = pos >= t0 && pos < t1;
    if (has_pos) {
        if (tid < FD) {
            float x1 = kx1, x2 = kx2;
            if (p.k_norm) {
                x1 = (kg1 * x1) * rk_s;
                x2 = (kg2 * x2) * rk_s;
            }
            const float o1 = x1 * kcs.x - x2 * kcs.y, o2 = x2 * kcs.x + x1 * kcs.y;
            k_new[tid] = o1;
            k_new[tid + FD] = o2;
            kc[(size_t)pos * HD + tid] = o1;
            kc[(size_t)pos * HD + tid + FD] = o2;
        }
        if (tid < HD) {
            v_new[tid] = vnew;
            vc[(size_t)pos * HD + tid] = vnew;
        }
    }
    __syncthreads();

    // ---- phase 1: scores -----------------------------------------------------------
    {
        float qr[G][EPL];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int j = 0; j < EPL / 4; j++) {
                const float4 t = *reinterpret_cast<const float4*>(&q_s[g][j * 64 + gl * 4]);
                qr[g][j * 4] = t.x; qr[g][j * 4 + 1] = t.y; qr[g][j * 4 + 2] = t.z; qr[g][j * 4 + 3] = t.w;
            }
        const float scale = sqrtf((float)HD);
        for (int base = t0; base < t1; base += PASS1) {
            // the next pass's rows are in flight while this pass is scored
            float kn[KU][EPL];
            const bool more = base + PASS1 < t1;
            if (more) load_k(kn, base + PASS1);
#pragma unroll
            for (int u = 0; u < KU; u++) {
                const int t = base + grp + NG * u;
                if (has_pos && t == pos) {
#pragma unroll
                    for (int j = 0; j < EPL / 4; j++) {
                        const float4 v = *reinterpret_cast<const float4*>(&k_new[j * 64 + gl * 4]);
                        kr[u][j * 4] = v.x; kr[u][j * 4 + 1] = v.y; kr[u][j * 4 + 2] = v.z; kr[u][j * 4 + 3] = v.w;
                    }
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    float d = 0.f;
#pragma unroll
                    for (int e = 0; e < EPL; e++) d = fmaf(qr[g][e], kr[u][e], d);
#pragma unroll
                    for (int off = 8; off > 0; off >>= 1) d += __shfl_xor(d, off, 16);
                    if (gl == 0 && t < t1) s_s[g][t - t0] = d / scale;
                }
            }
            if (more)
#pragma unroll
                for (int u = 0; u < KU; u++)
#pragma unroll
                    for (int e = 0; e < EPL; e++) kr[u][e] = kn[u][e];
        }
    }
    __syncthreads();

    // ---- split-local softmax statistics --------------------------------------------
    const int len = t1 - t0;
    for (int g = wave; g < G; g += NWV) {
        float m = -INFINITY;
        for (int i = lane; i < len; i += 64) m = fmaxf(m, s_s[g][i]);
        m = wave_max(m);
        float l = 0.f;
        for (int i = lane; i < len; i += 64) {
            const float e = expf(s_s[g][i] - m);
            s_s[g][i] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) { m_s[g] = m; l_s[g] = l; }
    }
    __syncthreads();

    // ---- phase 2: values -------------------------------------------------------------
    {
        float acc[G][VPL];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int j = 0; j < VPL; j++) acc[g][j] = 0.f;
        for (int base = t0; base < t1; base += PASS2) {
            float vn[VU][VPL];
            const bool more = base + PASS2 < t1;
            if (more) load_v(vn, base + PASS2);
#pragma unroll
            for (int u = 0; u < VU; u++) {
                const int t = base + wave + NWV * u;
                if (t < t1) {
                    if (has_pos && t == pos) {
#pragma unroll
                        for (int j = 0; j < VPL; j++) vr[u][j] = v_new[lane * VPL + j];
                    }
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        const float a = s_s[g][t - t0];
#pragma unroll
                        for (int j = 0; j < VPL; j++) acc[g][j] = fmaf(a, vr[u][j], acc[g][j]);
                    }
                }
            }
            if (more)
#pragma unroll
                for (int u = 0; u < VU; u++)
#pragma unroll
                    for (int j = 0; j < VPL; j++) vr[u][j] = vn[u][j];
        }
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int j = 0; j < VPL; j++) red_s[wave][g][lane * VPL + j] = acc[g][j];
    }
    __syncthreads();

    const int hbase = kvh * G;
    for (int idx = tid; idx < G * HD; idx += NT) {
        const int g = idx / HD, i = idx - g * HD;
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < NWV; w++) o += red_s[w][g][i];
        if (nsplit == 1) {
            p.out[(size_t)b * p.out_stride + (size_t)(hbase + g) * HD + i] = o / l_s[g];
        } else {
            const size_t slot = ((size_t)b * heads + hbase + g) * p.max_splits + split;
            p.part_o[slot * HD + i] = o;
            if (i == 0) {
                p.part_ml[slot * 2] = m_s[g];
                p.part_ml[slot * 2 + 1] = l_s[g];
            }
        }
    }
}

// Merges the split partials of every query head: o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.
// The (m, l) pairs are loaded in parallel into LDS, the weights e^(m_s - M) computed once per
// split, then every thread sums its column over the splits eight loads at a time.
template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(AttnParams p) {
    __shared__ float w_s[kMaxSplits];
    __shared__ float red[HD / 64];
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const int lane = i & 63, wave = i >> 6;
    const int pos = *p.pos;
    if (pos < 0 || pos >= p.max_seq) return;
    int nsplit, tile;
    split_plan(pos + 1, p.max_splits, &nsplit, &tile);
    if (nsplit == 1) return;  // the attention kernel wrote the output itself
    const size_t slot0 = ((size_t)b * p.heads + h) * p.max_splits;
    float m_loc = -INFINITY;
    for (int s = i; s < nsplit; s += HD) {
        const float m = p.part_ml[(slot0 + s) * 2];
        w_s[s] = m;
        m_loc = fmaxf(m_loc, m);
    }
    m_loc = wave_max(m_loc);
    if (lane == 0) red[wave] = m_loc;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < HD / 64; w++) M = fmaxf(M, red[w]);
    float l_loc = 0.f;
    for (int s = i; s < nsplit; s += HD) {
        const float w = expf(w_s[s] - M);
        w_s[s] = w;
        l_loc = fmaf(p.part_ml[(slot0 + s) * 2 + 1], w, l_loc);
    }
    l_loc = wave_sum(l_loc);
    __syncthreads();
    if (lane == 0) red[wave] = l_loc;
    __syncthreads();
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < HD / 64; w++) L += red[w];
    float O = 0.f;
    int s = 0;
    for (; s + 8 <= nsplit; s += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = p.part_o[(slot0 + s + u) * HD + i];
#pragma unroll
        for (int u = 0; u < 8; u++) O = fmaf(v[u], w_s[s + u], O);
    }
    for (; s < nsplit; s++) O = fmaf(p.part_o[(slot0 + s) * HD + i], w_s[s], O);
    p.out[(size_t)b * p.out_stride + (size_t)h * HD + i] = O / L;
}

template <int HD, int G>
int launch_t(const AttnLaunch& a, hipStream_t stream) {
    AttnParams p;
    p.qkv = a.qkv; p.qkv_stride = a.qkv_stride; p.q_norm = a.q_norm; p.k_norm = a.k_norm;
    p.qk_eps = a.qk_eps; p.per_head_norm = a.per_head_norm; p.kcache = a.kcache; p.vcache = a.vcache;
    p.max_seq = a.max_seq; p.pos = a.pos; p.heads = a.heads; p.kv_heads = a.kv_heads;
    p.rope_c = -2.0 * log(a.rope_theta) / (double)HD;
    p.rope_tab = a.rope_tab;
    p.max_splits = a.max_splits; p.part_o = a.part_o; p.part_ml = a.part_ml;
    p.out = a.out; p.out_stride = a.out_stride;
    if (a.max_splits == 1 && a.max_seq <= kShortMax) {
        // whole context in one block: 1024 threads (512 when 8 query heads share a KV head, for registers)
        constexpr int NT = G <= 4 ? 1024 : 512;
        hipLaunchKernelGGL((attn_decode_kernel<HD, G, NT>), dim3(1, a.kv_heads, a.batch), dim3(NT), 0, stream, p);
        AR_LAUNCH_CHECK();
        return AR_HIP_OK;
    }
    hipLaunchKernelGGL((attn_decode_kernel<HD, G, kThreads>), dim3(a.max_splits, a.kv_heads, a.batch),
                       dim3(kThreads), 0, stream, p);
    AR_LAUNCH_CHECK();
    if (a.max_splits > 1) {
        hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(a.heads, a.batch), dim3(HD), 0, stream, p);
        AR_LAUNCH_CHECK();
    }
    return AR_HIP_OK;
}

template <int HD>
int pick_g(const AttnLaunch& a, hipStream_t s) {
    switch (a.heads / a.kv_heads) {
        case 1: return launch_t<HD, 1>(a, s);
        case 2: return launch_t<HD, 2>(a, s);
        case 4: return launch_t<HD, 4>(a, s);
        case 8: return launch_t<HD, 8>(a, s);
    }
    ar_set_error("attention: heads/kv_heads = %d not in {1,2,4,8}", a.heads / a.kv_heads);
    return AR_HIP_ERR_INVALID;
}

}  // namespace

size_t attention_partial_floats(int batch, int heads, int max_splits, int hd) {
    return (size_t)batch * heads * max_splits * (size_t)hd;
}

int attention_max_splits(int max_seq, int kv_heads, int batch) {
    if (max_seq <= kShortMax) return 1;  // one block per (sequence, KV head), no combine launch
    const int need = (max_seq + kMaxTile - 1) / kMaxTile;      // rows per split <= kMaxTile
    const int want = (1024 + kv_heads * batch - 1) / (kv_heads * batch);  // ~4 blocks per CU
    const int cap = (max_seq + 15) / 16;                       // splits of >= 16 rows
    int s = want < cap ? want : cap;
    if (s < need) s = need;
    return s < 1 ? 1 : s;
}

int launch_attention_decode(const AttnLaunch& a, hipStream_t stream) {
    AR_CHECK_ARG(a.qkv && a.kcache && a.vcache && a.pos && a.out, "attention: null pointer");
    AR_CHECK_ARG(a.heads > 0 && a.kv_heads > 0 && a.heads % a.kv_heads == 0, "attention: bad head counts %d/%d",
                 a.heads, a.kv_heads);
    AR_CHECK_ARG(a.max_splits <= kMaxSplits, "attention: %d splits exceed %d", a.max_splits, kMaxSplits);
    AR_CHECK_ARG(a.max_splits >= 1 && ((long long)a.max_splits * kMaxTile >= a.max_seq ||
                                       (a.max_splits == 1 && a.max_seq <= kShortMax)),
                 "attention: %d splits of at most %d rows do not cover %d rows", a.max_splits, kMaxTile, a.max_seq);
    AR_CHECK_ARG(a.max_splits == 1 || (a.part_o && a.part_ml), "attention: missing split buffers");
    AR_CHECK_ARG(a.batch >= 1 && a.batch <= 65535, "attention: bad batch %d", a.batch);
    AR_CHECK_ARG((reinterpret_cast<uintptr_t>(a.kcache) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.vcache) & 15) == 0,
                 "attention: caches must be 16-byte aligned");
    if (a.head_dim == 128) return pick_g<128>(a, stream);
    if (a.head_dim == 64) return pick_g<64>(a, stream);
    ar_set_error("attention: head_dim %d not supported (64, 128)", a.head_dim);
    return AR_HIP_ERR_INVALID;
}
