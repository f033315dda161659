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
// Each 16-lane group streams its own rows of the split (K and V row read once, for all heads of
// the group) in chunks of 4 rows with an online softmax, the next chunk's loads in flight while the
// current one is used; the groups' (max, sum, accumulator) states are merged by shuffles within a
// wavefront and through LDS across wavefronts.
// With one split the block writes the normalised output; otherwise it writes unnormalised
// partials (o, max, sum) that attn_combine_kernel merges in the next launch (the kernel boundary
// makes them visible, so no block needs a device-wide fence).
#include <type_traits>

#include "ar_hip_internal.h"

namespace {

constexpr int kThreads = 256;   // threads of the split (multi-block) form
constexpr int kMaxTile = 348;   // rows per split in that form (fp32 cache; C5, 8 x 8 KV heads x 8256
                                // rows: 24 splits of 344 rows 106.8 us/layer vs 33 of 251 rows 110.6,
                                // 20 of 413 rows 109.7, 16 of 516 rows 118.3)
constexpr int kMaxTile16 = 1040; // fp16 cache: the per-row work (fp16 -> fp32 conversions) makes
                                 // longer splits pay (C5, 8 x 8 KV heads x 8256 rows: 8 splits of
                                 // 1032 rows 5.55 ms/step vs 33 of 251 rows 6.32)
constexpr int kShortMax = 256;  // caches up to this many rows: one block per (sequence, KV head)
constexpr int kMaxSplits = 1024;

struct AttnParams {
    const float* q;        // [batch][stride]: this step's raw q, k, v (k and v may live elsewhere)
    const float* k;
    const float* v;
    int qkv_stride;
    const float* q_norm;
    const float* k_norm;
    float qk_eps;
    int per_head_norm;
    void* kcache;          // fp32, or fp16 for the KV16 instantiation
    void* vcache;
    int max_seq;
    const int* pos;        // device position, or null: pos_value
    int pos_value;
    int heads, kv_heads;
    double rope_c;  // -2 ln(theta) / hd
    const float2* rope_tab;  // [max_seq][hd/2] (cos, sin) or null
    int max_splits;
    float* part_o;
    float* part_ml;
    float* out;
    int out_stride;
    uint16_t* out_hi;  // bf16 operand planes of out for the next GEMV, or null
    uint16_t* out_lo;
};


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

// NT threads: 256 when the context is cut into splits across blocks, 512 for a context of at most
// kShortMax rows handled by one block per (sequence, KV head) with no combine launch.  KV16: the
// cache holds fp16 rows (the new row is rounded before it is used, so every step sees exactly the
// values the cache holds).  TAB: the rotation angles come from the (cos, sin) table, else they
// are evaluated in double.  RU0: K/V rows per 16-lane group per chunk.
template <int HD, int G, int NT, bool KV16, bool TAB, int RU0>
__global__ __launch_bounds__(NT) void attn_decode_kernel(AttnParams p) {
    using KVT = typename std::conditional<KV16, _Float16, float>::type;
    constexpr int FD = HD / 2;
    constexpr int EPL = HD / 16;     // dims per lane: a 16-lane group holds one row; fp32 rows: lane gl
                                     // holds dims 64*(e/4) + 4*gl + e%4 (each 16-byte load of the group
                                     // covers 256 contiguous bytes); fp16 rows: dims EPL*gl + e (one
                                     // load per row)
    constexpr int NGR = NT / 16;     // 16-lane row groups
    constexpr int NWV = NT / 64;     // wavefronts
    // rows per group per chunk: RU0, chosen from the longest split (a chunk of NGR * RU rows covers
    // it; 16-row splits take one row per group, no clamped duplicate loads); at most 2 for G >= 8,
    // and for G >= 4 with fp32 rows (registers: G query fragments; the G = 4 fp32 instance holds 192
    // VGPRs at RU 4, two wavefronts per SIMD, and 136 at RU 2, three)
    constexpr int RU = ((G >= 8 || (G >= 4 && !KV16)) && RU0 > 2) ? 2 : RU0;
    __shared__ __attribute__((aligned(16))) float q_s[G][HD];
    __shared__ __attribute__((aligned(16))) float k_new[HD];
    __shared__ __attribute__((aligned(16))) float v_new[HD];
    __shared__ __attribute__((aligned(16))) float red_acc[NWV][G][HD];
    __shared__ float red_m[NWV][G], red_l[NWV][G];
    __shared__ float2 sq_s[NWV];
    __shared__ float rq_s[G], rk_s;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = tid >> 4, gl = tid & 15;
    const int b = blockIdx.z, kvh = blockIdx.y, split = blockIdx.x;
    const int heads = p.heads, kvH = p.kv_heads;
    const int q_dim = heads * HD, kv_dim = kvH * HD;
    const float* q_raw = p.q + (size_t)b * p.qkv_stride;
    const float* k_raw = p.k + (size_t)b * p.qkv_stride;
    const float* v_raw = p.v + (size_t)b * p.qkv_stride;
    const bool whole_norm = (p.q_norm || p.k_norm) && !p.per_head_norm;

    // ---- every load that does not depend on the position, issued together with it ----------
    const int pos = p.pos ? *p.pos : p.pos_value;
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
    // whole-vector QK-norm: this thread's float4 slices of q and k, held in registers (straight-line
    // loads, so no wait is needed before the position-dependent loads below are issued); vectors
    // longer than the register slices are finished by a loop after those loads
    constexpr int SQQ = (8192 / (NT * 4)) > 0 ? 8192 / (NT * 4) : 1;
    constexpr int SQK = (2048 / (NT * 4)) > 0 ? 2048 / (NT * 4) : 1;
    float4 wq[SQQ], wk[SQK];
    if (whole_norm) {
#pragma unroll
        for (int j = 0; j < SQQ; j++) {
            const int i = (tid + j * NT) * 4;
            wq[j] = i < q_dim ? *reinterpret_cast<const float4*>(q_raw + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < SQK; j++) {
            const int i = (tid + j * NT) * 4;
            wk[j] = i < kv_dim ? *reinterpret_cast<const float4*>(k_raw + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }

    if (pos < 0 || pos >= p.max_seq) return;
    const int n = pos + 1;
    int nsplit, tile;
    attn_split_plan(n, p.max_splits, &nsplit, &tile);
    if (split >= nsplit) return;
    const int t0 = split * tile;
    const int t1 = min(t0 + tile, n);
    const size_t head_base = ((size_t)b * kvH + kvh) * (size_t)p.max_seq * HD;
    KVT* kc = reinterpret_cast<KVT*>(p.kcache) + head_base;
    KVT* vc = reinterpret_cast<KVT*>(p.vcache) + head_base;
    auto dim_of = [&](int e) { return KV16 ? EPL * gl + e : 16 * (e & ~3) + gl * 4 + (e & 3); };

    // ---- rows of the split: group `grp` takes rows t0 + grp + NGR*i (neighbouring groups read
    // neighbouring rows), chunk c = rows i in [c*RU, c*RU + RU).  The rotation row and the first
    // chunk's K and V rows are issued as soon as the position is known, before anything waits for
    // the loads above (loads complete in issue order: the rotation is needed first).  Rows are clamped to the split (their scores are masked below); row `pos` is
    // stale in the cache until this block writes it, so that row is taken from LDS instead.
    float kr[RU][EPL], vr[RU][EPL];
    auto load_rows = [&](float (&dst)[RU][EPL], const KVT* src, int c) {
#pragma unroll
        for (int j = 0; j < RU; j++) {
            const int t = min(t0 + grp + NGR * (c * RU + j), t1 - 1);
            if constexpr (KV16) {
                typedef _Float16 halfv __attribute__((ext_vector_type(EPL)));
                const halfv v = *reinterpret_cast<const halfv*>(src + (size_t)t * HD + EPL * gl);
#pragma unroll
                for (int e = 0; e < EPL; e++) dst[j][e] = (float)v[e];
            } else {
#pragma unroll
                for (int e = 0; e < EPL; e += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(src + (size_t)t * HD + 16 * e + gl * 4);
                    dst[j][e] = v.x; dst[j][e + 1] = v.y; dst[j][e + 2] = v.z; dst[j][e + 3] = v.w;
                }
            }
        }
    };
    float2 qcs[QPT], kcs;
    if constexpr (TAB) {  // (cos, sin) row of the position from the table, ahead of the K/V rows
        const float2* rope_row = p.rope_tab + (size_t)pos * FD;
#pragma unroll
        for (int j = 0; j < QPT; j++) qcs[j] = rope_row[min(tid + j * NT, G * FD - 1) % FD];
        kcs = rope_row[kf];
    }
    load_rows(kr, kc, 0);
    load_rows(vr, vc, 0);
    if constexpr (!TAB) {
#pragma unroll
        for (int j = 0; j < QPT; j++) {
            const int idx = min(tid + j * NT, G * FD - 1);
            rope_cs(nullptr, pos, idx % FD, p.rope_c, &qcs[j].x, &qcs[j].y);
        }
        rope_cs(nullptr, pos, kf, p.rope_c, &kcs.x, &kcs.y);
    }

    // ---- QK-norm factors ----------------------------------------------------------
    float rq_w = 1.f, rk_w = 1.f;  // whole-vector factors (per-head factors go through LDS)
    if (p.q_norm || p.k_norm) {
        if (whole_norm) {
            float sq = 0.f, sk = 0.f;  // this thread's share of sum(q^2), sum(k^2), in index order
#pragma unroll
            for (int j = 0; j < SQQ; j++) sq += wq[j].x * wq[j].x + wq[j].y * wq[j].y + wq[j].z * wq[j].z + wq[j].w * wq[j].w;
            for (int i = (tid + SQQ * NT) * 4; i < q_dim; i += NT * 4) {
                const float4 v = *reinterpret_cast<const float4*>(q_raw + i);
                sq += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
#pragma unroll
            for (int j = 0; j < SQK; j++) sk += wk[j].x * wk[j].x + wk[j].y * wk[j].y + wk[j].z * wk[j].z + wk[j].w * wk[j].w;
            for (int i = (tid + SQK * NT) * 4; i < kv_dim; i += NT * 4) {
                const float4 v = *reinterpret_cast<const float4*>(k_raw + i);
                sk += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
            sq = wave_sum_lane63(sq);
            sk = wave_sum_lane63(sk);
            if (lane == 63) sq_s[wave] = make_float2(sq, sk);
            __syncthreads();
            float tq = 0.f, tk = 0.f;
#pragma unroll
            for (int w = 0; w < NWV; w++) {
                tq += sq_s[w].x;
                tk += sq_s[w].y;
            }
            rq_w = 1.0f / sqrtf(tq / (float)q_dim + p.qk_eps);
            rk_w = 1.0f / sqrtf(tk / (float)kv_dim + p.qk_eps);
        } else {
            // wave w reduces heads w, w+4, ...; the k head goes to the last slot
            for (int j = wave; j < G + 1; j += NWV) {
                const float* src = (j < G) ? q_raw + (size_t)(kvh * G + j) * HD : k_raw + (size_t)kvh * HD;
                float s = 0.f;
                for (int i = lane; i < HD; i += 64) s += src[i] * src[i];
                s = wave_sum_lane63(s);
                if (lane == 63) {
                    const float r = 1.0f / sqrtf(s / (float)HD + p.qk_eps);
                    if (j < G) rq_s[j] = r; else rk_s = r;
                }
            }
            __syncthreads();
        }
    }

    // ---- normalised, rotated queries of this group -> LDS ---------------------------
#pragma unroll
    for (int j = 0; j < QPT; j++) {
        const int idx = tid + j * NT;
        if (idx < G * FD) {
            const int g = idx / FD, f = idx - g * FD;
            float x1 = qx1[j], x2 = qx2[j];
            if (p.q_norm) {
                const float r = whole_norm ? rq_w : rq_s[g];
                x1 = (qg1[j] * x1) * r;
                x2 = (qg2[j] * x2) * r;
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
                const float r = whole_norm ? rk_w : rk_s;
                x1 = (kg1 * x1) * r;
                x2 = (kg2 * x2) * r;
            }
            const KVT o1 = (KVT)(x1 * kcs.x - x2 * kcs.y), o2 = (KVT)(x2 * kcs.x + x1 * kcs.y);
            k_new[tid] = (float)o1;
            k_new[tid + FD] = (float)o2;
            kc[(size_t)pos * HD + tid] = o1;
            kc[(size_t)pos * HD + tid + FD] = o2;
        }
        if (tid < HD) {
            const KVT vv = (KVT)vnew;
            v_new[tid] = (float)vv;
            vc[(size_t)pos * HD + tid] = vv;
        }
    }
    __syncthreads();

    // ---- one pass over K and V: online softmax per group, chunk by chunk ---------------
    // Scores are kept in base 2: the query fragment is pre-multiplied by log2(e)/sqrt(hd), so
    // exp(s - m) = exp2(s2 - m2) and the hardware exp2 serves every weight; m2 converts back to
    // natural-log units for the split partials.
    const float c2 = 1.4426950408889634f / sqrtf((float)HD);
    float qf[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            const float4 t = *reinterpret_cast<const float4*>(&q_s[g][dim_of(e)]);
            qf[g][e] = t.x * c2; qf[g][e + 1] = t.y * c2; qf[g][e + 2] = t.z * c2; qf[g][e + 3] = t.w * c2;
        }
    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[g][e] = 0.f;
    }
    const int nch = (t1 - t0 + NGR * RU - 1) / (NGR * RU);
    for (int c = 0; c < nch; c++) {
        if (has_pos) {
            // row pos (and every clamped duplicate of it: pos is the split's last row) was loaded
            // stale from the cache; it takes this step's k and v, so a masked duplicate adds 0 * v
            // of a finite row even when the stale row holds an infinity or NaN
#pragma unroll
            for (int j = 0; j < RU; j++)
                if (min(t0 + grp + NGR * (c * RU + j), t1 - 1) == pos)
#pragma unroll
                    for (int e = 0; e < EPL; e++) {
                        kr[j][e] = k_new[dim_of(e)];
                        vr[j][e] = v_new[dim_of(e)];
                    }
        }
        // scores q . K[t] / sqrt(hd) of the chunk's rows (rows past the split: -inf)
        float sc[G][RU];
#pragma unroll
        for (int j = 0; j < RU; j++) {
            const bool valid = t0 + grp + NGR * (c * RU + j) < t1;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < EPL; e++) d = fmaf(qf[g][e], kr[j][e], d);
                d = row16_sum(d);
                sc[g][j] = valid ? d : -INFINITY;
            }
        }
        if (c + 1 < nch) load_rows(kr, kc, c + 1);  // K of the next chunk, in flight from here
#pragma unroll
        for (int g = 0; g < G; g++) {
            float mc = sc[g][0];
#pragma unroll
            for (int j = 1; j < RU; j++) mc = fmaxf(mc, sc[g][j]);
            const float mn = fmaxf(m[g], mc);
            if (mn == -INFINITY) continue;  // nothing valid yet for this group
            const float alpha = (m[g] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[g] - mn);
            l[g] *= alpha;
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[g][e] *= alpha;
#pragma unroll
            for (int j = 0; j < RU; j++) {
                const float pj = __builtin_amdgcn_exp2f(sc[g][j] - mn);  // masked: exp2(-inf) = 0
                l[g] += pj;
#pragma unroll
                for (int e = 0; e < EPL; e++) acc[g][e] = fmaf(pj, vr[j][e], acc[g][e]);
            }
            m[g] = mn;
        }
        if (c + 1 < nch) load_rows(vr, vc, c + 1);  // V of the next chunk
    }

    // ---- merge the groups: the four of a wavefront by lane swaps, the wavefronts through LDS ---
    auto merge_with = [&](auto partner) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float mo = partner(m[g]), lo = partner(l[g]);
            const float mn = fmaxf(m[g], mo);
            const float a = (m[g] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[g] - mn);
            const float bo = (mo == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mo - mn);
            l[g] = l[g] * a + lo * bo;
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                const float ao = partner(acc[g][e]);
                acc[g][e] = acc[g][e] * a + ao * bo;
            }
            m[g] = mn;
        }
    };
    merge_with([&](float v) { return xor16(v, lane); });
    merge_with([&](float v) { return xor32(v, lane); });
    if (lane < 16) {
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int e = 0; e < EPL; e++) red_acc[wave][g][dim_of(e)] = acc[g][e];
            if (lane == 0) {
                red_m[wave][g] = m[g];
                red_l[wave][g] = l[g];
            }
        }
    }
    __syncthreads();

    const int hbase = kvh * G;
    for (int idx = tid; idx < G * HD; idx += NT) {
        const int g = idx / HD, i = idx - g * HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWV; w++) M = fmaxf(M, red_m[w][g]);
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < NWV; w++) {
            const float wt = (red_m[w][g] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(red_m[w][g] - M);
            L = fmaf(red_l[w][g], wt, L);
            o = fmaf(red_acc[w][g][i], wt, o);
        }
        if (nsplit == 1) {
            const size_t oi = (size_t)b * p.out_stride + (size_t)(hbase + g) * HD + i;
            p.out[oi] = o / L;
            if (p.out_hi) bf16_planes(o / L, p.out_hi + oi, p.out_lo + oi);
        } else {
            const size_t slot = ((size_t)b * heads + hbase + g) * p.max_splits + split;
            p.part_o[slot * HD + i] = o;
            if (i == 0) {
                p.part_ml[slot * 2] = M * 0.6931471805599453f;  // back to natural-log units
                p.part_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// Merges the split partials of every query head: o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.
// Every load that does not depend on the position (the partial outputs of the first kMergeRegs
// splits and this thread's (m, l) pair) is issued together with the position load, so the merge
// costs one memory round trip; splits past kMergeRegs (long contexts) are read afterwards.
template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(AttnParams p) {
    constexpr int kMergeRegs = 32;
    __shared__ float w_s[kMaxSplits];
    __shared__ float red[HD / 64];
    const int h = blockIdx.x, b = blockIdx.y, i = threadIdx.x;
    const int lane = i & 63, wave = i >> 6;
    const size_t slot0 = ((size_t)b * p.heads + h) * p.max_splits;
    float ov[kMergeRegs];
#pragma unroll
    for (int s = 0; s < kMergeRegs; s++) ov[s] = s < p.max_splits ? p.part_o[(slot0 + s) * HD + i] : 0.f;
    const float2 ml = i < p.max_splits ? reinterpret_cast<const float2*>(p.part_ml)[slot0 + i]
                                       : make_float2(-INFINITY, 0.f);
    const int pos = p.pos ? *p.pos : p.pos_value;
    if (pos < 0 || pos >= p.max_seq) return;
    int nsplit, tile;
    attn_split_plan(pos + 1, p.max_splits, &nsplit, &tile);
    if (nsplit == 1) return;  // the attention kernel wrote the output itself
    float m_loc = i < nsplit ? ml.x : -INFINITY;
    for (int s = i + HD; s < nsplit; s += HD) m_loc = fmaxf(m_loc, p.part_ml[(slot0 + s) * 2]);
    m_loc = wave_max_lane63(m_loc);
    if (lane == 63) red[wave] = m_loc;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < HD / 64; w++) M = fmaxf(M, red[w]);
    float l_loc = 0.f;
    if (i < nsplit) {
        const float w = expf(ml.x - M);
        w_s[i] = w;
        l_loc = fmaf(ml.y, w, l_loc);
    }
    for (int s = i + HD; s < nsplit; s += HD) {
        const float w = expf(p.part_ml[(slot0 + s) * 2] - M);
        w_s[s] = w;
        l_loc = fmaf(p.part_ml[(slot0 + s) * 2 + 1], w, l_loc);
    }
    l_loc = wave_sum_lane63(l_loc);
    __syncthreads();
    if (lane == 63) red[wave] = l_loc;
    __syncthreads();
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < HD / 64; w++) L += red[w];
    float O = 0.f;
#pragma unroll
    for (int s = 0; s < kMergeRegs; s++)
        if (s < nsplit) O = fmaf(ov[s], w_s[s], O);
    for (int s = kMergeRegs; s < nsplit; s++) O = fmaf(p.part_o[(slot0 + s) * HD + i], w_s[s], O);
    const size_t oi = (size_t)b * p.out_stride + (size_t)h * HD + i;
    p.out[oi] = O / L;
    if (p.out_hi) bf16_planes(O / L, p.out_hi + oi, p.out_lo + oi);
}

template <int HD, int G, bool KV16>
int launch_t(const AttnLaunch& a, hipStream_t stream) {
    AttnParams p;
    p.q = a.qkv ? a.qkv : a.q;
    p.k = a.qkv ? a.qkv + (size_t)a.heads * a.head_dim : a.k;
    p.v = a.qkv ? a.qkv + (size_t)(a.heads + a.kv_heads) * a.head_dim : a.v;
    p.qkv_stride = a.qkv_stride; p.q_norm = a.q_norm; p.k_norm = a.k_norm;
    p.qk_eps = a.qk_eps; p.per_head_norm = a.per_head_norm; p.kcache = a.kcache; p.vcache = a.vcache;
    p.max_seq = a.max_seq; p.pos = a.pos; p.pos_value = a.pos_value; p.heads = a.heads; p.kv_heads = a.kv_heads;
    p.rope_c = -2.0 * log(a.rope_theta) / (double)HD;
    p.rope_tab = a.rope_tab;
    p.max_splits = a.max_splits; p.part_o = a.part_o; p.part_ml = a.part_ml;
    p.out = a.out; p.out_stride = a.out_stride; p.out_hi = a.out_hi; p.out_lo = a.out_lo;
    if (a.max_splits == 1 && a.max_seq <= kShortMax) {
        // whole context in one block
        constexpr int NT = 512;
        const dim3 grid(1, a.kv_heads, a.batch);
        if (p.rope_tab) ar_launch((attn_decode_kernel<HD, G, NT, KV16, true, 4>), grid, dim3(NT), 0, stream, p);
        else ar_launch((attn_decode_kernel<HD, G, NT, KV16, false, 4>), grid, dim3(NT), 0, stream, p);
        AR_LAUNCH_CHECK();
        return AR_HIP_OK;
    }
    const dim3 grid(a.max_splits, a.kv_heads, a.batch);
    // longest split of this launch: of the live context when the position is given, else of any
    // position the cache holds (attn_split_plan: splits of <= 16 rows until max_splits are in use)
    int longest;
    if (a.pos) {
        longest = (a.max_seq + a.max_splits - 1) / a.max_splits;
        if (longest < kAttnMinTile) longest = kAttnMinTile;
    } else {
        int ns;
        attn_split_plan(a.pos_value + 1, a.max_splits, &ns, &longest);
    }
    constexpr int NGR = kThreads / 16;
    if (p.rope_tab && longest <= NGR)
        ar_launch((attn_decode_kernel<HD, G, kThreads, KV16, true, 1>), grid, dim3(kThreads), 0, stream, p);
    else if (p.rope_tab && longest <= 2 * NGR)
        ar_launch((attn_decode_kernel<HD, G, kThreads, KV16, true, 2>), grid, dim3(kThreads), 0, stream, p);
    else if (p.rope_tab)
        ar_launch((attn_decode_kernel<HD, G, kThreads, KV16, true, 4>), grid, dim3(kThreads), 0, stream, p);
    else
        ar_launch((attn_decode_kernel<HD, G, kThreads, KV16, false, 4>), grid, dim3(kThreads), 0, stream, p);
    AR_LAUNCH_CHECK();
    if (a.max_splits > 1) {
        ar_launch((attn_combine_kernel<HD>), dim3(a.heads, a.batch), dim3(HD), 0, stream, p);
        AR_LAUNCH_CHECK();
    }
    return AR_HIP_OK;
}

template <int HD, bool KV16>
int pick_g(const AttnLaunch& a, hipStream_t s) {
    switch (a.heads / a.kv_heads) {
        case 1: return launch_t<HD, 1, KV16>(a, s);
        case 2: return launch_t<HD, 2, KV16>(a, s);
        case 4: return launch_t<HD, 4, KV16>(a, s);
        case 8: return launch_t<HD, 8, KV16>(a, s);
    }
    ar_set_error("attention: heads/kv_heads = %d not in {1,2,4,8}", a.heads / a.kv_heads);
    return AR_HIP_ERR_INVALID;
}

// Causal attention of prompt rows in fp32, the attention of the fp32-weight prefill: row t of
// sequence b (block (b*T + t, g)) attends cache rows 0..p0+t of KV head g for the G query heads of
// the group, with the decode kernel's arithmetic (queries pre-scaled by log2(e)/sqrt(hd), online
// softmax in base 2, 16-lane groups each streaming every 16th row in chunks of RU rows loaded
// together, group states merged by lane swaps and through LDS).  The cache rows of the prompt are written beforehand (qk_prep), so every row
// reads finished rows only.  q32: [B*T][heads*hd] normalised, rotated queries; caches fp32
// [B][KV][S][hd]; out: [B*T][heads*hd].
template <int HD, int G>
__global__ __launch_bounds__(256) void attn_prefill_f32_kernel(const float* q32, const float* kcache,
                                                                const float* vcache, float* out, int T, int p0,
                                                                int S, int heads, int kv_heads) {
    constexpr int EPL = HD / 16, NGR = 16, NWV = 4, RU = 4;
    __shared__ __attribute__((aligned(16))) float red_acc[NWV][G][HD];
    __shared__ float red_m[NWV][G], red_l[NWV][G];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = tid >> 4, gl = tid & 15;
    const int r = blockIdx.x, g = blockIdx.y, b = r / T, t = r - b * T, n = p0 + t + 1;
    const size_t head = ((size_t)b * kv_heads + g) * (size_t)S * HD;
    const float* kc = kcache + head;
    const float* vc = vcache + head;
    auto dim_of = [&](int e) { return 16 * (e & ~3) + gl * 4 + (e & 3); };
    const float c2 = 1.4426950408889634f / sqrtf((float)HD);
    float qf[G][EPL];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(q32 + (size_t)r * heads * HD + (size_t)(g * G + h) * HD +
                                                              16 * e + gl * 4);
            qf[h][e] = v.x * c2; qf[h][e + 1] = v.y * c2; qf[h][e + 2] = v.z * c2; qf[h][e + 3] = v.w * c2;
        }
    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = -INFINITY;
        l[h] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) acc[h][e] = 0.f;
    }
    auto load_row = [&](float (&dst)[EPL], const float* src, int row) {
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(src + (size_t)row * HD + 16 * e + gl * 4);
            dst[e] = v.x; dst[e + 1] = v.y; dst[e + 2] = v.z; dst[e + 3] = v.w;
        }
    };
    // chunk c: rows c*NGR*RU + grp + NGR*j (j < RU) of each 16-lane group, loaded together (rows past
    // n re-read row n-1 and score -inf); the next chunk is in flight while one is used
    float ka[RU][EPL], va[RU][EPL], kb[RU][EPL], vb[RU][EPL];
    auto load_chunk = [&](float (&kd)[RU][EPL], float (&vd)[RU][EPL], int c) {
#pragma unroll
        for (int j = 0; j < RU; j++) {
            const int row = min(c * NGR * RU + grp + NGR * j, n - 1);
            load_row(kd[j], kc, row);
            load_row(vd[j], vc, row);
        }
    };
    auto use_chunk = [&](const float (&kd)[RU][EPL], const float (&vd)[RU][EPL], int c) {
        float sc[G][RU];
#pragma unroll
        for (int j = 0; j < RU; j++) {
            const bool valid = c * NGR * RU + grp + NGR * j < n;
#pragma unroll
            for (int h = 0; h < G; h++) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < EPL; e++) d = fmaf(qf[h][e], kd[j][e], d);
                d = row16_sum(d);
                sc[h][j] = valid ? d : -INFINITY;
            }
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
            float mc = sc[h][0];
#pragma unroll
            for (int j = 1; j < RU; j++) mc = fmaxf(mc, sc[h][j]);
            const float mn = fmaxf(m[h], mc);
            if (mn == -INFINITY) continue;
            const float alpha = (m[h] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[h] - mn);
            l[h] *= alpha;
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[h][e] *= alpha;
#pragma unroll
            for (int j = 0; j < RU; j++) {
                const float pj = __builtin_amdgcn_exp2f(sc[h][j] - mn);
                l[h] += pj;
#pragma unroll
                for (int e = 0; e < EPL; e++) acc[h][e] = fmaf(pj, vd[j][e], acc[h][e]);
            }
            m[h] = mn;
        }
    };
    const int nch = (n + NGR * RU - 1) / (NGR * RU);
    load_chunk(ka, va, 0);
    for (int c = 0; c < nch; c += 2) {
        if (c + 1 < nch) load_chunk(kb, vb, c + 1);
        use_chunk(ka, va, c);
        if (c + 1 >= nch) break;
        if (c + 2 < nch) load_chunk(ka, va, c + 2);
        use_chunk(kb, vb, c + 1);
    }
    auto merge_with = [&](auto partner) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float mo = partner(m[h]), lo = partner(l[h]);
            const float mn = fmaxf(m[h], mo);
            const float a = (m[h] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[h] - mn);
            const float bo = (mo == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mo - mn);
            l[h] = l[h] * a + lo * bo;
#pragma unroll
            for (int e = 0; e < EPL; e++) acc[h][e] = acc[h][e] * a + partner(acc[h][e]) * bo;
            m[h] = mn;
        }
    };
    merge_with([&](float v) { return xor16(v, lane); });
    merge_with([&](float v) { return xor32(v, lane); });
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < G; h++) {
#pragma unroll
            for (int e = 0; e < EPL; e++) red_acc[wave][h][dim_of(e)] = acc[h][e];
            if (lane == 0) {
                red_m[wave][h] = m[h];
                red_l[wave][h] = l[h];
            }
        }
    }
    __syncthreads();
    for (int idx = tid; idx < G * HD; idx += 256) {
        const int h = idx / HD, i = idx - h * HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWV; w++) M = fmaxf(M, red_m[w][h]);
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < NWV; w++) {
            const float wt = (red_m[w][h] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(red_m[w][h] - M);
            L = fmaf(red_l[w][h], wt, L);
            o = fmaf(red_acc[w][h][i], wt, o);
        }
        out[(size_t)r * heads * HD + (size_t)(g * G + h) * HD + i] = o / L;
    }
}

template <int HD>
int launch_prefill_f32_hd(const float* q32, const float* kc, const float* vc, float* out, int B, int T, int p0, int S,
                          int heads, int kv_heads, hipStream_t st) {
    const dim3 grid(B * T, kv_heads);
    switch (heads / kv_heads) {
        case 1: hipLaunchKernelGGL((attn_prefill_f32_kernel<HD, 1>), grid, dim3(256), 0, st, q32, kc, vc, out, T, p0, S, heads, kv_heads); break;
        case 2: hipLaunchKernelGGL((attn_prefill_f32_kernel<HD, 2>), grid, dim3(256), 0, st, q32, kc, vc, out, T, p0, S, heads, kv_heads); break;
        case 4: hipLaunchKernelGGL((attn_prefill_f32_kernel<HD, 4>), grid, dim3(256), 0, st, q32, kc, vc, out, T, p0, S, heads, kv_heads); break;
        case 8: hipLaunchKernelGGL((attn_prefill_f32_kernel<HD, 8>), grid, dim3(256), 0, st, q32, kc, vc, out, T, p0, S, heads, kv_heads); break;
        default:
            ar_set_error("prefill attention: heads/kv_heads = %d not in {1,2,4,8}", heads / kv_heads);
            return AR_HIP_ERR_INVALID;
    }
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

}  // namespace

int launch_attention_prefill_f32(const float* q32, const float* kcache, const float* vcache, float* out, int B, int T,
                                 int p0, int S, int heads, int kv_heads, int hd, hipStream_t stream) {
    AR_CHECK_ARG(q32 && kcache && vcache && out && B > 0 && T > 0, "prefill attention: bad arguments");
    AR_CHECK_ARG(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "prefill attention: bad head counts");
    AR_CHECK_ARG(p0 >= 0 && p0 + T <= S, "prefill attention: rows %d..%d outside the %d-row cache", p0, p0 + T, S);
    AR_CHECK_ARG((long long)B * T <= 0x7fffffffLL && kv_heads <= 65535, "prefill attention: grid too large");
    if (hd == 128) return launch_prefill_f32_hd<128>(q32, kcache, vcache, out, B, T, p0, S, heads, kv_heads, stream);
    if (hd == 64) return launch_prefill_f32_hd<64>(q32, kcache, vcache, out, B, T, p0, S, heads, kv_heads, stream);
    ar_set_error("prefill attention: head_dim %d not supported (64, 128)", hd);
    return AR_HIP_ERR_INVALID;
}

size_t attention_partial_floats(int batch, int heads, int max_splits, int hd) {
    return (size_t)batch * heads * max_splits * (size_t)hd;
}

int attention_max_splits(int max_seq, int kv_heads, int batch, bool kv16) {
    if (max_seq <= kShortMax) return 1;  // one block per (sequence, KV head), no combine launch
    const int tmax = kv16 ? kMaxTile16 : kMaxTile;
    const int need = (max_seq + tmax - 1) / tmax;                // rows per split <= tmax
    // about one block per CU: each block then streams a tile long enough to amortise its prologue
    // (C2, 4097 rows: 32 splits of 129 rows; 128 splits of 33 rows measured 2.4x slower)
    const int want = (256 + kv_heads * batch - 1) / (kv_heads * batch);
    const int cap = (max_seq + kAttnMinTile - 1) / kAttnMinTile;  // splits of >= kAttnMinTile rows
    int s = want < cap ? want : cap;
    if (s < need) s = need;
    return s < 1 ? 1 : s;
}

int launch_attention_decode(const AttnLaunch& a, hipStream_t stream) {
    AR_CHECK_ARG((a.qkv || (a.q && a.k && a.v)) && a.kcache && a.vcache && a.out, "attention: null pointer");
    AR_CHECK_ARG(a.pos || (a.pos_value >= 0 && a.pos_value < a.max_seq), "attention: position %d outside %d rows",
                 a.pos_value, a.max_seq);
    AR_CHECK_ARG(a.heads > 0 && a.kv_heads > 0 && a.heads % a.kv_heads == 0, "attention: bad head counts %d/%d",
                 a.heads, a.kv_heads);
    AR_CHECK_ARG(a.max_splits <= kMaxSplits, "attention: %d splits exceed %d", a.max_splits, kMaxSplits);
    const int tmax = a.kv16 ? kMaxTile16 : kMaxTile;
    AR_CHECK_ARG(a.max_splits >= 1 && ((long long)a.max_splits * tmax >= a.max_seq ||
                                       (a.max_splits == 1 && a.max_seq <= kShortMax)),
                 "attention: %d splits of at most %d rows do not cover %d rows", a.max_splits, tmax, a.max_seq);
    AR_CHECK_ARG(a.max_splits == 1 || (a.part_o && a.part_ml), "attention: missing split buffers");
    AR_CHECK_ARG(a.batch >= 1 && a.batch <= 65535, "attention: bad batch %d", a.batch);
    AR_CHECK_ARG((reinterpret_cast<uintptr_t>(a.kcache) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.vcache) & 15) == 0,
                 "attention: caches must be 16-byte aligned");
    if (ar_check_ptrs_enabled()) {  // extents of the attention and combine kernels
        const char* k = "attention";
        const size_t hd = a.head_dim, qd = (size_t)a.heads * hd, kvd = (size_t)a.kv_heads * hd, B1 = a.batch - 1;
        const size_t elem = a.kv16 ? 2 : 4, cache = (size_t)a.batch * kvd * a.max_seq * elem;
        if (a.qkv) {
            AR_TRY(ar_check_range(a.qkv, (B1 * a.qkv_stride + qd + 2 * kvd) * 4, k, "q/k/v rows"));
        } else {
            AR_TRY(ar_check_range(a.q, (B1 * a.qkv_stride + qd) * 4, k, "q rows"));
            AR_TRY(ar_check_range(a.k, (B1 * a.qkv_stride + kvd) * 4, k, "k rows"));
            AR_TRY(ar_check_range(a.v, (B1 * a.qkv_stride + kvd) * 4, k, "v rows"));
        }
        AR_TRY(ar_check_range(a.q_norm, qd * 4, k, "q norm gain"));
        AR_TRY(ar_check_range(a.k_norm, kvd * 4, k, "k norm gain"));
        AR_TRY(ar_check_range(a.kcache, cache, k, "key cache"));
        AR_TRY(ar_check_range(a.vcache, cache, k, "value cache"));
        AR_TRY(ar_check_range(a.pos, 4, k, "position"));
        AR_TRY(ar_check_range(a.rope_tab, (size_t)a.max_seq * (hd / 2) * sizeof(float2), k, "RoPE table"));
        if (a.max_splits > 1) {
            AR_TRY(ar_check_range(a.part_o, attention_partial_floats(a.batch, a.heads, a.max_splits, a.head_dim) * 4,
                                  k, "split partials"));
            AR_TRY(ar_check_range(a.part_ml, (size_t)a.batch * a.heads * a.max_splits * 2 * 4, k, "split maxima / sums"));
        }
        AR_TRY(ar_check_range(a.out, (B1 * a.out_stride + qd) * 4, k, "output"));
        AR_TRY(ar_check_range(a.out_hi, (B1 * a.out_stride + qd) * 2, k, "output hi plane"));
        AR_TRY(ar_check_range(a.out_lo, (B1 * a.out_stride + qd) * 2, k, "output lo plane"));
    }
    if (a.head_dim == 128) return a.kv16 ? pick_g<128, true>(a, stream) : pick_g<128, false>(a, stream);
    if (a.head_dim == 64) return a.kv16 ? pick_g<64, true>(a, stream) : pick_g<64, false>(a, stream);
    ar_set_error("attention: head_dim %d not supported (64, 128)", a.head_dim);
    return AR_HIP_ERR_INVALID;
}
