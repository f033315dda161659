// Persistent decode step: every layer of one batch-1 Qwen3 decode step, then its logits, in one launch.
//
// The step the reference builds per layer (engine/ml/.../AttentionFeatures.java:785-929,
// FeedForwardFeatures.java:147-156, NormalizationLayerFeatures.java:584-595) is five all-to-all
// dependencies per layer: each GEMV needs the whole output of the previous stage.  Launched as
// separate kernels, every stage pays a launch, the cold HBM round trip of its first weight loads
// and an idle tail, which at the 0.6B decode shapes (8-25 MB per GEMV) costs as much as the weight
// stream itself.  Here one block per CU runs all layers:
//  * each stage's weight rows for this block are issued into registers before the block waits for
//    the stage's input, so the HBM latency and stream overlap the cross-block exchange;
//  * stages exchange their outputs through 64-bit words that carry an epoch next to the fp32
//    value, stored and loaded at device scope (they bypass the XCD-private L2s): a reader polls
//    the words it needs until every epoch is the current one, so the data's arrival is the
//    synchronisation (no counters, no fences, no contention on a shared address);
//  * every wait is bounded: a block that waits too long flags the error word and stops waiting,
//    so the grid always drains; the host reports the flag as an error.
//
// Stages of layer l (epoch e = base + l + 1, exchange buffers double-buffered by l's parity):
//   P1 QKV      qkv = Wqkv . (rmsnorm(x) * attn_norm) (+ bias)             rows of all blocks
//   P2 attention per (KV head, split): QK-norm, RoPE, cache-row write at pos, online softmax over
//               the split's cache rows -> unnormalised partials (o, max, sum)
//   P2b merge   per query head (one block each): o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s
//   P3 O        x_mid = x + Wo . o
//   P4 gate/up  h = (W3 . xn) * silu(W1 . xn), xn = rmsnorm(x_mid) * ffn_norm
//   P5 down     x' = x_mid + W2 . h          (the last layer also stores x' in the model's x)
// then once: P6 final RMSNorm, logits (stored when asked), greedy-token keys.
// The block grid is fixed (one block per CU); each GEMV's rows divide evenly over all of it or, for
// dims that do not split 256 ways into whole wavefront rows, over its first blocks (pick_rq, pick_ro).
#include <cstdint>

#include "ar_hip_internal.h"
#include "gemv_impl.h"

// Stage timeline (diagnostic build only, -DAR_PK_TRACE): thread 0 of every block records the wall
// clock (100 MHz, common to all CUs) at each stage boundary of every layer; ar_hip_pk_trace_read
// copies the table out.  The default build compiles the marks away.
#ifdef AR_PK_TRACE
constexpr int kTraceLayers = 64, kTraceMarks = 24;
__device__ unsigned long long g_pk_trace[kTraceLayers][256][kTraceMarks];
#define PK_MARK(l, k)                                                                              \
    do {                                                                                           \
        if (threadIdx.x == 0 && (l) < kTraceLayers) g_pk_trace[(l)][blockIdx.x][(k)] = wall_clock64(); \
    } while (0)
extern "C" int ar_hip_pk_trace_read(void* dst, size_t bytes) {
    if (bytes < sizeof(g_pk_trace)) return AR_HIP_ERR_INVALID;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_pk_trace), sizeof(g_pk_trace)) == hipSuccess ? AR_HIP_OK
                                                                                                : AR_HIP_ERR_HIP;
}
#else
#define PK_MARK(l, k) \
    do {              \
    } while (0)
#endif

namespace {

constexpr int kPB = 256;           // blocks: one per CU
constexpr int kPT = 512;           // threads per block
constexpr int kPW = kPT / 64;      // wavefronts per block
constexpr int kRowsPerSplit = 32;  // cache rows per split before another split is opened
constexpr unsigned kSpinLimit = 1u << 18;  // default polls before a wait is abandoned (~0.3 s)
constexpr int kPadLds = 64 * 1024;         // dynamic LDS: keeps a second block off each CU, holds copied down rows
constexpr int kMaxLayers = 64;             // layer table held in LDS
// gate/up hold-back of the blocks without attention, wall-clock ticks (10 ns): see the O stage
template <typename TW>
constexpr unsigned kGateUpDelay = sizeof(TW) == 4 ? 150 : 250;

struct PLayer {
    const void* wqkv;  // projection weights in the model's weight type (fp32 or bf16)
    const void* wo;
    const void* w1;
    const void* w3;
    const void* w2;
    const float* attn_norm;
    const float* ffn_norm;
    const float* q_norm;
    const float* k_norm;
    const float* bqkv;
};

struct PParams {
    const PLayer* layers;
    int L;
    float* x;          // [dim]: the step's input (embedding row) and, after the last layer, its output
    void* kcache;      // [L][KV][S][HD], fp32 or fp16 (the KT instantiation)
    void* vcache;
    int S;
    const float2* rope_tab;  // [S][HD/2] (cos, sin)
    int* state;        // [0] position, [3] epoch base (advanced by L at the end of every launch)
    uint64_t* ll;      // exchange words, two parities
    int* err;          // set to 1 when a wait timed out
    unsigned spin_limit;  // polls before a wait is abandoned
    float eps;
    int per_head;      // QK-norm: one RMS per head (else over the whole q / k vector)
    // after the last layer: final RMSNorm, logits and greedy-token keys
    const float* final_norm;
    const void* lm_head;   // [vocab][dim], weight type
    int vocab;
    float* logits;         // [vocab], or null: not stored
    unsigned long long* keys;  // [kArgmaxSlots] packed (value, index) maxima, zero before the launch
};

// Loads through pointers read from the layer table.  The compiler sees those pointers as generic,
// and a generic (flat) load counts against the LDS counter as well as the vector-memory counter (every
// LDS wait behind it would also wait for the weight rows); they point to device memory, so they are
// loaded as global.  The base is cast before the offset is added (a cast of a finished per-lane
// address folds back into a generic load); the host pass compiles these bodies without running them.
// The 16-byte weight loads are nontemporal: every weight byte is read once per step, and streaming
// them past the caches' normal retention measured C3 0.608 -> 0.594 and C4 1.005 -> 0.975 ms per step.
typedef __attribute__((address_space(3))) void pk_lds_void;
typedef const __attribute__((address_space(1))) float gfloat;
__device__ inline float4 gld4(const float* base, size_t off) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef float v4 __attribute__((ext_vector_type(4)));
    const v4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) v4*)((gfloat*)base + off));
    return make_float4(v.x, v.y, v.z, v.w);
#else
    return *reinterpret_cast<const float4*>(base + off);
#endif
}
__device__ inline float gld(const float* base, size_t off) {
#if defined(__HIP_DEVICE_COMPILE__)
    return ((gfloat*)base)[off];
#else
    return base[off];
#endif
}
// Weight rows in 16-byte loads: fp32 (4 values) or bf16 (8 values, widened exactly by a shift), dotted
// with fp32 inputs in the same order as the fp32 rows.
typedef const __attribute__((address_space(1))) uint32_t guint;
__device__ inline uint4 gld4u(const void* base, size_t off16) {  // off16: offset in 16-byte units
#if defined(__HIP_DEVICE_COMPILE__)
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u4*)((guint*)base + 4 * off16));
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return reinterpret_cast<const uint4*>(base)[off16];
#endif
}
template <typename TW>
struct WRow;
template <>
struct WRow<float> {
    static constexpr int V = 4;  // values per 16-byte load
    typedef float4 raw;
    __device__ static raw load(const void* base, size_t off) { return gld4((const float*)base, off); }
    __device__ static float dot(const raw& w, const float* x, float a) {
        a = fmaf(w.x, x[0], a);
        a = fmaf(w.y, x[1], a);
        a = fmaf(w.z, x[2], a);
        a = fmaf(w.w, x[3], a);
        return a;
    }
};
template <>
struct WRow<uint16_t> {
    static constexpr int V = 8;
    typedef uint4 raw;
    __device__ static raw load(const void* base, size_t off) { return gld4u(base, off / 8); }
    __device__ static float lo(uint32_t u) { return __uint_as_float(u << 16); }
    __device__ static float hi(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }
    __device__ static float dot(const raw& w, const float* x, float a) {
        a = fmaf(lo(w.x), x[0], a);
        a = fmaf(hi(w.x), x[1], a);
        a = fmaf(lo(w.y), x[2], a);
        a = fmaf(hi(w.y), x[3], a);
        a = fmaf(lo(w.z), x[4], a);
        a = fmaf(hi(w.z), x[5], a);
        a = fmaf(lo(w.w), x[6], a);
        a = fmaf(hi(w.w), x[7], a);
        return a;
    }
};

// The block's "stop waiting" flag in LDS, through relaxed workgroup-scope atomics (LDS accesses the
// compiler neither caches in a register nor turns into generic ones).
__device__ inline int dead_get(int* d) { return __hip_atomic_load(d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ inline void dead_set(int* d) { __hip_atomic_store(d, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }

__device__ inline void ll_put(uint64_t* p, unsigned ep, float v) {
    __hip_atomic_store(p, ((uint64_t)ep << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t ll_get(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline bool ll_ok(uint64_t w, unsigned ep) { return (unsigned)(w >> 32) == ep; }
__device__ inline float ll_val(uint64_t w) { return __uint_as_float((unsigned)w); }

// Waits for N words at base[idx[j]] to carry epoch ep (or the block to be marked dead).
template <int N>
__device__ inline void ll_wait(const uint64_t* base, const int (&idx)[N], float (&out)[N], unsigned ep,
                               int* dead, int* err, unsigned limit) {
    uint64_t w[N];
#pragma unroll
    for (int j = 0; j < N; j++) w[j] = idx[j] >= 0 ? ll_get(base + idx[j]) : ((uint64_t)ep << 32);
    unsigned spins = 0;
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < N; j++) ok &= ll_ok(w[j], ep);
        if (ok || dead_get(dead)) break;
        if (++spins > limit) {
            dead_set(dead);
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
        for (int j = 0; j < N; j++)
            if (!ll_ok(w[j], ep)) w[j] = ll_get(base + idx[j]);
    }
#pragma unroll
    for (int j = 0; j < N; j++) out[j] = ll_val(w[j]);
}

// Block barrier over LDS only: waits for this wave's LDS operations, not for its global loads
// and stores (the prefetched weight rows stay in flight across it).
__device__ inline void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A copy of the thread index the compiler cannot see through, taken at the start of every stage: the
// per-thread addresses are then computed inside the stage instead of being hoisted out of the layer
// loop and held in registers across all stages.
#define STAGE_IDS()                                            \
    int tid = tid0;                                            \
    asm volatile("" : "+v"(tid));                              \
    const int lane = tid & 63;                                 \
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); \
    (void)lane;                                                \
    (void)wave

// Sum over the block's threads (every thread gets the total, summed in wavefront order).
__device__ inline float block_sum(float v, float* red, int lane, int wave) {
    v = gemv::dpp_sum_lane63(v);
    if (lane == 63) red[wave] = v;
    lds_barrier();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kPW; w++) t += red[w];
    return t;
}

// Row distribution of the GEMV stages over the kPB blocks.  QKV: RQ rows per block (a multiple of the
// wavefront count, all rows of a block in one head), the smallest such that QKVD / RQ blocks cover
// the rows.  O / down: RO rows per block, each split over WPR = kPW / RO wavefronts, the smallest RO
// for which DIM / RO blocks cover the rows and the O / down input widths split into whole 64-lane
// chunks per wavefront.  Blocks past QKVD / RQ (DIM / RO) have no rows in that stage.
constexpr int pick_rq(int qkvd, int hd) {
    for (int rq = kPW; rq <= 64; rq += kPW)
        if (qkvd % rq == 0 && qkvd / rq <= kPB && hd % rq == 0) return rq;
    return 0;
}
constexpr int pick_ro(int dim, int qd, int f, int cw) {
    for (int ro = 1; ro <= kPW; ro *= 2) {
        const int wpr = kPW / ro;
        if (dim % ro == 0 && dim / ro <= kPB && qd % (wpr * cw) == 0 && f % (wpr * cw) == 0) return ro;
    }
    return 0;
}

template <typename TW, typename KT, int DIM, int F, int H, int KV, int HD, int SMAX>
__global__ __launch_bounds__(kPT, 1) void decode_persistent_kernel(PParams p) {
    using WR = WRow<TW>;
    typedef typename WR::raw wraw;
    // fp16 cache: rows are widened as they are read; the step's new k / v row is rounded to fp16
    // before it is used, so every step sees exactly the values the cache holds
    constexpr bool kv16 = sizeof(KT) == 2;
    static_assert(sizeof(KT) == 4 || sizeof(KT) == 2, "fp32 or fp16 cache");
    constexpr int CW = 64 * WR::V;  // columns per 16-byte load of a wavefront
    constexpr int QD = H * HD, KVD = KV * HD, QKVD = QD + 2 * KVD, G = H / KV, FD = HD / 2;
    // P1: RQ rows per block on the first NQB blocks, RPWq per wavefront, NCq CW-column chunks per row
    constexpr int RQ = pick_rq(QKVD, HD), NQB = RQ ? QKVD / RQ : 1, RPWq = RQ / kPW, NCq = DIM / CW;
    // P3 / P5: RO (= RD) rows per block on the first NOB blocks, each split over WPR wavefronts
    constexpr int RO = pick_ro(DIM, QD, F, CW), NOB = RO ? DIM / RO : 1, WPR = RO ? kPW / RO : 1;
    constexpr int NCo = QD / (WPR * CW), NCd = F / (WPR * CW);
    // down-row chunks per wavefront copied into the dynamic LDS after the gate/up input (see P4)
    constexpr bool kDownDma = sizeof(TW) == 4 && kPW * NCd * 1024 <= kPadLds && KV * SMAX >= NOB;
    constexpr int kDmaChunks = kDownDma ? NCd : 0;
    // P4: RG gate/up row pairs per block; wavefronts 0..kPW/2-1 take gate rows, the rest up rows
    constexpr int RG = F / kPB, RPWg = 2 * RG / kPW, NCg = DIM / CW;
    // inputs of DIM / QD / F values: this many per thread of the block
    constexpr int NXD = (DIM + kPT - 1) / kPT, NXA = (QD + kPT - 1) / kPT;
    static_assert(RQ > 0 && RPWq >= 1, "QKV rows must split over the blocks' waves");
    // (constant true when every block has rows in the stage)
    const bool has_q = NQB >= kPB || (int)blockIdx.x < NQB, has_o = NOB >= kPB || (int)blockIdx.x < NOB;
    static_assert(DIM % CW == 0 && RO > 0, "dim must split over the blocks' waves");
    static_assert(F % kPB == 0 && (2 * RG) % kPW == 0 && RG % RPWg == 0 && 2 * RG <= 64, "gate/up rows");
    static_assert(HD == 128 || HD == 64, "head size");
    constexpr int XMAX = QD > F ? (QD > DIM ? QD : DIM) : (F > DIM ? F : DIM);
    // exchange layout per parity (words)
    constexpr int OFF_XA = 0, OFF_XM = DIM, OFF_QKV = 2 * DIM, OFF_PART = OFF_QKV + QKVD;
    constexpr int PART_STRIDE = HD + 2;  // o[HD], max (natural log units), sum
    constexpr int OFF_A = OFF_PART + KV * SMAX * G * PART_STRIDE;  // merged attention output [QD]
    constexpr int OFF_H = OFF_A + QD;
    // sums of squares of each QKV block's rows (q blocks, then k blocks) for the QK-norm
    constexpr int NSQ = QD / RQ, NSK = KVD / RQ;
    constexpr int OFF_SS = OFF_H + F;
    constexpr int PAR_WORDS = OFF_SS + NSQ + NSK;
    static_assert(QD % RQ == 0 && KVD % RQ == 0 && HD % RQ == 0, "a QKV block's rows lie in one head");
    static_assert(KV * SMAX <= kPB - H, "attention and merge blocks must not overlap");

    __shared__ __attribute__((aligned(16))) float xr[DIM];    // layer input x_l
    __shared__ __attribute__((aligned(16))) float xmr[DIM];   // x_mid (after the O residual)
    __shared__ __attribute__((aligned(16))) float xin[XMAX];  // the stage's GEMV input
    __shared__ float red[kPW];
    __shared__ float rows_s[64];
    // attention
    __shared__ __attribute__((aligned(16))) float q_s[G][HD];
    __shared__ __attribute__((aligned(16))) float k_new[HD];
    __shared__ __attribute__((aligned(16))) float v_new[HD];
    __shared__ float ss_s[(G + 1) * (HD / RQ)];  // per-head QK-norm: the partial sums of the block's heads
    __shared__ float2 red2[kPW];
    __shared__ __attribute__((aligned(16))) float red_acc[kPW][G][HD];
    __shared__ float red_m[kPW][G], red_l[kPW][G];
    __shared__ __attribute__((aligned(16))) float mrg_o[SMAX][HD];  // split merge
    __shared__ float2 mrg_ml[SMAX];
    constexpr int SMAX4 = (SMAX + 3) / 4 * 4;
    __shared__ __attribute__((aligned(16))) float mrg_w[SMAX4];  // split weights and sums, 16-byte reads
    __shared__ __attribute__((aligned(16))) float mrg_l[SMAX4];
    __shared__ int dead_s;
    // the layer table, read from LDS: a global load of it inside the loop would make the wavefront
    // wait for every weight load it has in flight
    __shared__ PLayer lay_s[kMaxLayers];

    extern __shared__ __attribute__((aligned(1024))) unsigned char dyn_lds[];  // kPadLds bytes
    const int tid0 = threadIdx.x, b = blockIdx.x;
    int* dead = &dead_s;
    if (tid0 == 0) dead_s = 0;
    const int pos = p.state[0];
    const unsigned base = (unsigned)p.state[3];
    if (pos < 0 || pos >= p.S) {  // the host never steps past the cache; every block takes this exit
        if (b == 0 && tid0 == 0) __hip_atomic_store(p.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const int n = pos + 1;
    int nsplit = (n + kRowsPerSplit - 1) / kRowsPerSplit;
    nsplit = nsplit < 1 ? 1 : (nsplit > SMAX ? SMAX : nsplit);
    const int tile = (n + nsplit - 1) / nsplit;
    const float2* rope_row = p.rope_tab + (size_t)pos * FD;
    for (int i = tid0; i < p.L * (int)(sizeof(PLayer) / 8); i += kPT)
        reinterpret_cast<uint64_t*>(lay_s)[i] = reinterpret_cast<const uint64_t*>(p.layers)[i];
    __syncthreads();

    // QKV rows: layer 0's before the loop, layer l+1's after layer l's down stores (fp32 weights) or at
    // the start of layer l's gate/up stage (bf16 weights, whose register budget has no room for them
    // there).  A wavefront's memory operations leave a CU in issue order, so rows issued at the
    // gate/up stage's start sit ahead of that stage's input poll and its stores (each waited ~1.5 us
    // longer, stage timeline); issued after the down stores they only delay the next QKV stage's dot
    // products: C3 0.593 -> 0.584 ms per step.
    constexpr bool kQkvAfterDown = sizeof(TW) == 4;
    wraw wq[RPWq][NCq];
    auto load_wq = [&](const void* W, int wave, int lane) {
        if (!has_q) return;  // no QKV rows in this block
        const int r0 = b * RQ + wave * RPWq;
#pragma unroll
        for (int i = 0; i < RPWq; i++)
#pragma unroll
            for (int c = 0; c < NCq; c++) wq[i][c] = WR::load(W, (size_t)(r0 + i) * DIM + c * CW + lane * WR::V);
    };
    {
        STAGE_IDS();
        load_wq(lay_s[0].wqkv, wave, lane);
    }
    for (int l = 0; l < p.L; l++) {
        const PLayer& Ly = lay_s[l];
        const unsigned ep = base + (unsigned)l + 1u;
        uint64_t* cur = p.ll + (size_t)(l & 1) * PAR_WORDS;
        const uint64_t* prev = p.ll + (size_t)((l + 1) & 1) * PAR_WORDS;

        // ================= P1: QKV =================================================
        PK_MARK(l, 0);
        lds_barrier();  // the previous layer's readers of xin / xr are done
        {
        STAGE_IDS();
        {
            constexpr int NX = NXD;
            // the gains are loaded before the wait, so the wait's completion covers them
            float gv[NX];
#pragma unroll
            for (int j = 0; j < NX; j++) gv[j] = tid + j * kPT < DIM ? gld(Ly.attn_norm, tid + j * kPT) : 0.f;
            float xv[NX];
            if (l == 0) {
#pragma unroll
                for (int j = 0; j < NX; j++) xv[j] = tid + j * kPT < DIM ? p.x[tid + j * kPT] : 0.f;
            } else {
                int idx[NX];
#pragma unroll
                for (int j = 0; j < NX; j++) idx[j] = tid + j * kPT < DIM ? OFF_XA + tid + j * kPT : -1;
                ll_wait<NX>(prev, idx, xv, base + (unsigned)l, dead, p.err, p.spin_limit);
            }
            PK_MARK(l, 1);
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NX; j++) {
                const int i = tid + j * kPT;
                if (i < DIM) {
                    ss = fmaf(xv[j], xv[j], ss);
                    xr[i] = xv[j];
                    xin[i] = xv[j] * gv[j];
                }
            }
            const float tot = block_sum(ss, red, lane, wave);  // (its barrier also publishes xr / xin)
            PK_MARK(l, 15);
            const float rn = 1.0f / sqrtf(tot / (float)DIM + p.eps);
            float ssq = 0.f;
            float av[RPWq];
#pragma unroll
            for (int i = 0; i < RPWq; i++) {
                float a = 0.f;
                if (has_q) {
#pragma unroll
                    for (int c = 0; c < NCq; c++) a = WR::dot(wq[i][c], &xin[c * CW + lane * WR::V], a);
                }
                av[i] = a;
            }
            gemv::dpp_sum_lane63_n(av);
#pragma unroll
            for (int i = 0; i < RPWq; i++) {
                if (!has_q) break;
                const float a = av[i] * rn;
                if (lane == 63) {
                    const int row = b * RQ + wave * RPWq + i;
                    const float v = Ly.bqkv ? a + gld(Ly.bqkv, row) : a;
                    ll_put(cur + OFF_QKV + row, ep, v);
                    ssq = fmaf(v, v, ssq);
                }
            }
            // a block of q or k rows also publishes their sum of squares: the attention blocks then
            // wait for NSQ + NSK partial sums instead of every q and k value
            if (b < NSQ + NSK) {
                if (lane == 63) rows_s[wave] = ssq;
                lds_barrier();
                if (tid == 0) {
                    float t = 0.f;
#pragma unroll
                    for (int w = 0; w < kPW; w++) t += rows_s[w];
                    ll_put(cur + OFF_SS + b, ep, t);
                }
            }
        }
        }

        PK_MARK(l, 2);
        const unsigned long long t_p1 = wall_clock64();  // (100 MHz)
        // ================= P2: attention (blocks of (KV head, split)) ==============
        // The split's cache rows are dealt round-robin to the wavefronts; a lane holds HD / 64
        // dimensions of a row, so each score is one full-wavefront sum (DPP into lane 63, read back as
        // a uniform value) and every wavefront runs its own online softmax over its rows; the eight
        // wavefront states merge through LDS.  (Rows in 16-lane groups, four groups per wavefront,
        // needed two lane-swap merges of the 2 x 8 accumulators per lane: 2.75 -> 2.2 us from the
        // attention inputs to the partials' stores, C3 0.596 -> 0.588 ms per step.)
        if (b < KV * nsplit) {
            STAGE_IDS();
            constexpr int DPL = HD / 64;                  // cache dimensions per lane
            constexpr int RW = SMAX <= 8 ? 6 : 10;        // cache rows per wavefront per chunk
            static_assert(DPL == 1 || DPL == 2, "head size 64 or 128");
            const int g = b / nsplit, s = b - g * nsplit;
            const int t0 = s * tile, t1 = min(t0 + tile, n);
            const size_t head_base = ((size_t)l * KV + g) * (size_t)p.S * HD;
            KT* kc = reinterpret_cast<KT*>(p.kcache) + head_base;
            KT* vc = reinterpret_cast<KT*>(p.vcache) + head_base;
            // row j of chunk c of this wavefront (uniform over the wavefront)
            auto row_of = [&](int c, int j) { return t0 + c * (kPW * RW) + wave + kPW * j; };
            float kr[RW][DPL], vr[RW][DPL];
            auto load_rows = [&](float (&dst)[RW][DPL], const KT* src, int c) {
#pragma unroll
                for (int j = 0; j < RW; j++) {
                    const KT* r = src + (size_t)min(row_of(c, j), t1 - 1) * HD + lane * DPL;
                    if constexpr (kv16 && DPL == 2) {
                        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
                        const h2 v = *reinterpret_cast<const h2*>(r);
                        dst[j][0] = (float)v.x;
                        dst[j][1] = (float)v.y;
                    } else if constexpr (DPL == 2) {
                        const float2 v = *reinterpret_cast<const float2*>(r);
                        dst[j][0] = v.x;
                        dst[j][1] = v.y;
                    } else {
                        dst[j][0] = (float)r[0];
                    }
                }
            };
            const int nch = t1 > t0 ? (t1 - t0 + kPW * RW - 1) / (kPW * RW) : 0;
            // With 10 rows per wavefront (long splits: 80 KB of K and V per block) the V rows follow
            // the wait: all of them ahead of it held the poll back (C4 0.886 -> 0.881 ms per step);
            // the K rows after the wait as well cost 0.870 -> 0.897
            constexpr bool kLateV = RW > 6;
            if (nch > 0) {  // cache rows before pos are final: issued before the wait for q / k / v
                load_rows(kr, kc, 0);
                if (!kLateV) load_rows(vr, vc, 0);
            }
            // thread layout: q rotation pairs of the G heads, k pairs, v values, QK-norm partial sums
            constexpr int RPH = HD / RQ;                           // QKV blocks per head
            constexpr int T_K = G * FD, T_V = T_K + FD, T_S = T_V + HD;
            static_assert(T_S + NSQ + NSK <= kPT && T_S + (G + 1) * RPH <= kPT, "attention thread layout");
            // this thread's rotation pair and QK-norm gains, also ahead of the wait
            const int rj = tid / FD, rf = tid - rj * FD;  // (tid < T_V: vector rj = q head g*G+rj, or k)
            float2 rcs = make_float2(1.f, 0.f);
            float rg1 = 1.f, rg2 = 1.f;
            const float* gn = rj < G ? Ly.q_norm : Ly.k_norm;
            if (tid < T_V) {
                rcs = rope_row[rf];
                const size_t o = rj < G ? (size_t)(g * G + rj) * HD : (size_t)g * HD;
                if (gn) {
                    rg1 = gld(gn, o + rf);
                    rg2 = gld(gn, o + rf + FD);
                }
            }
            asm volatile("" ::: "memory");  // (keeps these loads ahead of the polls)
            int idx[2] = {-1, -1};
            if (tid < T_K) {
                idx[0] = OFF_QKV + (g * G + rj) * HD + rf;
                idx[1] = idx[0] + FD;
            } else if (tid < T_V) {
                idx[0] = OFF_QKV + QD + g * HD + rf;
                idx[1] = idx[0] + FD;
            } else if (tid < T_S) {
                idx[0] = OFF_QKV + QD + KVD + g * HD + (tid - T_V);
            } else if (p.per_head) {  // the partial sums of heads g*G .. g*G+G-1 and of KV head g
                const int i = tid - T_S, h = i / RPH, k = i - h * RPH;
                if (h < G) idx[0] = OFF_SS + (g * G + h) * RPH + k;
                else if (h == G) idx[0] = OFF_SS + NSQ + g * RPH + k;
            } else if (tid - T_S < NSQ + NSK) {  // every q and k partial: one RMS over each vector
                idx[0] = OFF_SS + (tid - T_S);
            }
            float qv[2];
            ll_wait<2>(cur, idx, qv, ep, dead, p.err, p.spin_limit);  // (words not waited for read as 0)
            if (kLateV && nch > 0) load_rows(vr, vc, 0);
            PK_MARK(l, 3);
            if (p.per_head) {
                if (tid >= T_S && tid - T_S < (G + 1) * RPH) ss_s[tid - T_S] = qv[0];
            } else {
                const bool isq = tid >= T_S && tid - T_S < NSQ;
                float sq = isq ? qv[0] : 0.f, sk = (tid >= T_S && !isq) ? qv[0] : 0.f;
                float sqk[2] = {sq, sk};
                gemv::dpp_sum_lane63_n(sqk);
                sq = sqk[0];
                sk = sqk[1];
                if (lane == 63) red2[wave] = make_float2(sq, sk);
            }
            if (tid >= T_V && tid < T_S) v_new[tid - T_V] = kv16 ? (float)(KT)qv[0] : qv[0];
            lds_barrier();
            PK_MARK(l, 16);
            const bool has_pos = pos >= t0 && pos < t1;
            // normalised, rotated q (G heads) and k from the pair this thread holds; the block holding
            // pos writes the cache rows
            if (tid < T_V) {
                float tot = 0.f;
                if (p.per_head) {
#pragma unroll
                    for (int k = 0; k < RPH; k++) tot += ss_s[rj * RPH + k];
                } else {
#pragma unroll
                    for (int w = 0; w < kPW; w++) tot += rj < G ? red2[w].x : red2[w].y;
                }
                const float nv = p.per_head ? (float)HD : (rj < G ? (float)QD : (float)KVD);
                const float r = 1.0f / sqrtf(tot / nv + p.eps);
                float x1 = qv[0], x2 = qv[1];
                if (gn) {  // (q gains span the whole q vector, as the k gains the k vector)
                    x1 = (rg1 * x1) * r;
                    x2 = (rg2 * x2) * r;
                }
                const float o1 = x1 * rcs.x - x2 * rcs.y, o2 = x2 * rcs.x + x1 * rcs.y;
                if (rj < G) {
                    q_s[rj][rf] = o1;
                    q_s[rj][rf + FD] = o2;
                } else {
                    const KT k1 = (KT)o1, k2 = (KT)o2;
                    k_new[rf] = (float)k1;
                    k_new[rf + FD] = (float)k2;
                    if (has_pos) {
                        kc[(size_t)pos * HD + rf] = k1;
                        kc[(size_t)pos * HD + rf + FD] = k2;
                    }
                }
            } else if (tid < T_S && has_pos) {
                vc[(size_t)pos * HD + (tid - T_V)] = (KT)qv[0];
            }
            lds_barrier();
            PK_MARK(l, 17);

            const float c2 = 1.4426950408889634f / sqrtf((float)HD);
            float qf[G][DPL];
#pragma unroll
            for (int gg = 0; gg < G; gg++)
#pragma unroll
                for (int e = 0; e < DPL; e++) qf[gg][e] = q_s[gg][lane * DPL + e] * c2;
            float m[G], lsum[G], acc[G][DPL];
#pragma unroll
            for (int gg = 0; gg < G; gg++) {
                m[gg] = -INFINITY;
                lsum[gg] = 0.f;
#pragma unroll
                for (int e = 0; e < DPL; e++) acc[gg][e] = 0.f;
            }
            for (int c = 0; c < nch; c++) {
                if (has_pos) {
#pragma unroll
                    for (int j = 0; j < RW; j++)
                        if (min(row_of(c, j), t1 - 1) == pos)
#pragma unroll
                            for (int e = 0; e < DPL; e++) {
                                kr[j][e] = k_new[lane * DPL + e];
                                vr[j][e] = v_new[lane * DPL + e];
                            }
                }
                float sc[G][RW];  // (uniform over the wavefront)
                {
                    // the G x RW dot products' wavefront sums, interleaved step by step
                    float dd[G * RW];
#pragma unroll
                    for (int j = 0; j < RW; j++)
#pragma unroll
                        for (int gg = 0; gg < G; gg++) {
                            float d = 0.f;
#pragma unroll
                            for (int e = 0; e < DPL; e++) d = fmaf(qf[gg][e], kr[j][e], d);
                            dd[j * G + gg] = d;
                        }
                    gemv::dpp_sum_lane63_n(dd);
#pragma unroll
                    for (int j = 0; j < RW; j++) {
                        const bool valid = row_of(c, j) < t1;
#pragma unroll
                        for (int gg = 0; gg < G; gg++) {
                            const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dd[j * G + gg]), 63));
                            sc[gg][j] = valid ? d : -INFINITY;
                        }
                    }
                }
                if (c + 1 < nch) load_rows(kr, kc, c + 1);
#pragma unroll
                for (int gg = 0; gg < G; gg++) {
                    float mc = sc[gg][0];
#pragma unroll
                    for (int j = 1; j < RW; j++) mc = fmaxf(mc, sc[gg][j]);
                    const float mn = fmaxf(m[gg], mc);
                    if (mn == -INFINITY) continue;
                    const float alpha = (m[gg] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[gg] - mn);
                    lsum[gg] *= alpha;
#pragma unroll
                    for (int e = 0; e < DPL; e++) acc[gg][e] *= alpha;
#pragma unroll
                    for (int j = 0; j < RW; j++) {
                        const float pj = __builtin_amdgcn_exp2f(sc[gg][j] - mn);
                        lsum[gg] += pj;
#pragma unroll
                        for (int e = 0; e < DPL; e++) acc[gg][e] = fmaf(pj, vr[j][e], acc[gg][e]);
                    }
                    m[gg] = mn;
                }
                if (c + 1 < nch) load_rows(vr, vc, c + 1);
            }
            PK_MARK(l, 18);
            // the wavefronts' states through LDS
#pragma unroll
            for (int gg = 0; gg < G; gg++) {
#pragma unroll
                for (int e = 0; e < DPL; e++) red_acc[wave][gg][lane * DPL + e] = acc[gg][e];
                if (lane == 0) {
                    red_m[wave][gg] = m[gg];
                    red_l[wave][gg] = lsum[gg];
                }
            }
            lds_barrier();
            PK_MARK(l, 19);
            for (int idx = tid; idx < G * HD; idx += kPT) {
                const int gg = idx / HD, i = idx - gg * HD;
                float M = -INFINITY;
#pragma unroll
                for (int w = 0; w < kPW; w++) M = fmaxf(M, red_m[w][gg]);
                float Ls = 0.f, o = 0.f;
#pragma unroll
                for (int w = 0; w < kPW; w++) {
                    const float wt = (red_m[w][gg] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(red_m[w][gg] - M);
                    Ls = fmaf(red_l[w][gg], wt, Ls);
                    o = fmaf(red_acc[w][gg][i], wt, o);
                }
                uint64_t* slot = cur + OFF_PART + ((g * SMAX + s) * G + gg) * PART_STRIDE;
                ll_put(slot + i, ep, o);
                if (i == 0) {
                    ll_put(slot + HD, ep, M * 0.6931471805599453f);  // natural-log units
                    ll_put(slot + HD + 1, ep, Ls);
                }
            }
            PK_MARK(l, 4);
        }

        // O rows and gate/up rows of this block (held from their issue to the O and gate/up stages)
        wraw wo[NCo];
        wraw wg[RPWg][NCg];
        // With fp32 weights the blocks that run neither attention nor a merge also issue their down
        // rows behind the gate/up rows, so the down stage's poll has nothing queued ahead of it on
        // those CUs (C3 0.5612-0.5644 -> 0.5575-0.5616 ms per step over three runs); the attention
        // blocks doing the same (0.585) or every block (0.586) delays the attention chain instead.
        // (bf16 at d 2048 has no register room for them.)
        wraw wd[NCd];
        const bool early_d = sizeof(TW) == 4 && has_o && b >= KV * nsplit && b < kPB - H;
        // issue_o_gu(wave, lane, i0, i1, with_o): the O rows (when with_o and i0 == 0) and gate/up rows
        // i0 .. i1-1 of the wavefront
        auto issue_o_gu = [&](int wave, int lane, int i0, int i1, bool with_o = true) {
            const int row = b * RO + wave / WPR, col0 = (wave % WPR) * (QD / WPR);
            if (with_o && i0 == 0 && has_o) {
#pragma unroll
                for (int c = 0; c < NCo; c++)
                    wo[c] = WR::load(Ly.wo, (size_t)row * QD + col0 + c * CW + lane * WR::V);
            }
            // The blocks that are not busy with attention hold the gate/up rows back kGateUpDelay
            // after their QKV stage: issued at once they queue in HBM ahead of the attention's cache
            // rows and exchanges.  Measured at C3 (ms per step) with the current schedule: at once
            // 0.569, after 0.5 / 1 / 1.5 / 2 / 2.5 us 0.571 / 0.569 / 0.560 / 0.564 / 0.576; with the
            // attention blocks' late gate/up rows, 1 / 1.5 / 2 us 0.555 / 0.552 / 0.559.
            if (b >= KV * nsplit && i0 == 0 && with_o)
                while (wall_clock64() < t_p1 + kGateUpDelay<TW>) __builtin_amdgcn_s_sleep(4);
            const bool up = wave >= kPW / 2;
            const int r0 = b * RG + (up ? wave - kPW / 2 : wave) * RPWg;
            const void* W = up ? Ly.w3 : Ly.w1;
#pragma unroll
            for (int i = 0; i < RPWg; i++)
                if (i >= i0 && i < i1)
#pragma unroll
                    for (int c = 0; c < NCg; c++) wg[i][c] = WR::load(W, (size_t)(r0 + i) * DIM + c * CW + lane * WR::V);
            if (early_d && i1 == RPWg) {
                const int rowd = b * RO + wave / WPR, cold = (wave % WPR) * (F / WPR);
#pragma unroll
                for (int c = 0; c < NCd; c++) wd[c] = WR::load(Ly.w2, (size_t)rowd * F + cold + c * CW + lane * WR::V);
            }
        };

        // ================= P2b: merge the splits of each query head ==================
        // The merge blocks' O and gate/up rows stream while the attention runs: issued after the
        // merge, they arrive last of all and hold up every block's gate/up input (C3: 0.668 ->
        // 0.635 ms per step).  Where the rows and the merge's words do not fit in registers together
        // (bf16 at d 2048: 96 VGPRs of gate/up rows, 28 splits), they follow the merge.
        // With fp32 weights and the attention blocks a minority of the O-row holders (C3), the merge
        // blocks keep one gate/up row per wavefront before the merge and issue the rest after their O
        // stores, as the attention blocks do (C3 0.5512-0.5518 -> 0.5505-0.5508 ms per step).
        constexpr bool kMergeLate = sizeof(TW) == 4 && KV * SMAX < NOB && RPWg > 1;
        constexpr int kMergeEarlyRows = kMergeLate ? 1 : RPWg * NCg <= 12 ? RPWg : RPWg / 3;
        if (b >= kPB - H) {  // one block per query head (never an attention block)
            STAGE_IDS();
            issue_o_gu(wave, lane, 0, kMergeEarlyRows);
            // thread t: dimension t % HD of splits (t / HD) * SPT .. + SPT - 1
            constexpr int SPT = SMAX * HD / kPT;
            static_assert(SMAX * HD % kPT == 0 && SPT >= 1, "split merge: threads per split");
            const int h = b - (kPB - H), kvh = h / G, gg = h - kvh * G;
            // and thread t < 2 * SMAX: the maximum (even t) or the sum (odd t) of split t / 2
            static_assert(2 * SMAX <= kPT, "split merge: one (max, sum) word per thread");
            const int i = tid % HD, s0 = (tid / HD) * SPT;
            int idx[SPT + 1];
#pragma unroll
            for (int k = 0; k < SPT; k++) {
                const int s = s0 + k;
                idx[k] = s < nsplit ? OFF_PART + ((kvh * SMAX + s) * G + gg) * PART_STRIDE + i : -1;
            }
            const int sml = tid >> 1;
            idx[SPT] = tid < 2 * SMAX && sml < nsplit
                           ? OFF_PART + ((kvh * SMAX + sml) * G + gg) * PART_STRIDE + HD + (tid & 1)
                           : -1;
            float v[SPT + 1];
            ll_wait<SPT + 1>(cur, idx, v, ep, dead, p.err, p.spin_limit);
            PK_MARK(l, 5);
#pragma unroll
            for (int k = 0; k < SPT; k++) mrg_o[s0 + k][i] = v[k];
            if (tid < 2 * SMAX) {
                if (tid & 1) mrg_ml[sml].y = v[SPT];
                else mrg_ml[sml].x = sml < nsplit ? v[SPT] : -INFINITY;
            }
            lds_barrier();
            PK_MARK(l, 20);
            // the split weights once per block, one split per thread (each thread of the HD lanes
            // computing all of them took ~2.7 us at 28 splits); splits past nsplit have max -inf and
            // zero partials, so their weight is 0 and they add exact zeros below
            if (tid < SMAX4) {
                float M = -INFINITY;
#pragma unroll
                for (int s = 0; s < SMAX; s++) M = fmaxf(M, mrg_ml[s].x);
                mrg_w[tid] = tid < SMAX ? expf(mrg_ml[tid].x - M) : 0.f;
                mrg_l[tid] = tid < SMAX ? mrg_ml[tid].y : 0.f;
            }
            lds_barrier();
            if (tid < HD) {
                // four weights and sums per LDS read (the bf16 instance has no registers to spare for
                // loads issued ahead, so every read would be a round trip of its own)
                float Ls = 0.f, o = 0.f;
#pragma unroll
                for (int s4 = 0; s4 < SMAX4 / 4; s4++) {
                    const float4 w4 = *reinterpret_cast<const float4*>(&mrg_w[4 * s4]);
                    const float4 l4 = *reinterpret_cast<const float4*>(&mrg_l[4 * s4]);
                    const float w[4] = {w4.x, w4.y, w4.z, w4.w}, lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const int s = 4 * s4 + k;
                        if (s < SMAX) {
                            Ls = fmaf(lv[k], w[k], Ls);
                            o = fmaf(mrg_o[s][tid], w[k], o);
                        }
                    }
                }
                ll_put(cur + OFF_A + h * HD + tid, ep, o / Ls);
            }
            PK_MARK(l, 6);
        }

        // ================= P3: O projection + residual ==============================
        lds_barrier();  // xin readers (P1) are done
        {
            STAGE_IDS();
            const int col0 = (wave % WPR) * (QD / WPR);
            // The gate/up rows (the largest stage, 24 MB at C3) are issued with the O rows, so they
            // stream while the attention chain runs instead of at the start of their own stage (the
            // merge blocks issued both before their merge).
            // Where the attention blocks are a minority of the O-row holders (fp32 weights; C3: 64 of
            // 256), they come to the O stage last, and their O input poll queued behind all their gate/up
            // rows; they now issue one gate/up row per wavefront before the poll and the rest after
            // their O stores (C3 0.5602-0.5610 -> 0.5500-0.5505 ms per step; two before the poll
            // 0.5524-0.5531; with their down rows behind the late ones 0.576; at the stories110M
            // shape, 192 attention blocks of 256, it cost 0.1797 -> 0.1805 ms, so that shape keeps
            // the one issue).  The bf16 instance has no register room for the split (it spills).
            constexpr bool kAttLateGu = sizeof(TW) == 4 && KV * SMAX < NOB && RPWg > 1;
            constexpr int kAttEarlyRows = kAttLateGu ? 1 : RPWg;
            const bool att_late = kAttLateGu && b < KV * nsplit;
            if (b < kPB - H) issue_o_gu(wave, lane, 0, att_late ? kAttEarlyRows : RPWg);
            else if (kMergeEarlyRows < RPWg && !kMergeLate) issue_o_gu(wave, lane, kMergeEarlyRows, RPWg);
            constexpr int NA = NXA;
            int idx[NA];
#pragma unroll
            for (int j = 0; j < NA; j++) idx[j] = has_o && (QD % kPT == 0 || tid + j * kPT < QD) ? OFF_A + tid + j * kPT : -1;
            float av[NA];
            ll_wait<NA>(cur, idx, av, ep, dead, p.err, p.spin_limit);
            PK_MARK(l, 7);
#pragma unroll
            for (int j = 0; j < NA; j++)
                if (QD % kPT == 0 || tid + j * kPT < QD) xin[tid + j * kPT] = av[j];
            lds_barrier();
            PK_MARK(l, 21);
            float a = 0.f;
            if (has_o) {
#pragma unroll
                for (int c = 0; c < NCo; c++) a = WR::dot(wo[c], &xin[col0 + c * CW + lane * WR::V], a);
            }
            a = gemv::dpp_sum_lane63(a);
            if (lane == 63) rows_s[wave] = a;
            lds_barrier();
            if (tid < RO && has_o) {
                float sum = 0.f;
#pragma unroll
                for (int k = 0; k < WPR; k++) sum += rows_s[tid * WPR + k];
                const int r = b * RO + tid;
                ll_put(cur + OFF_XM + r, ep, xr[r] + sum);
            }
            if (att_late) issue_o_gu(wave, lane, kAttEarlyRows, RPWg, false);
            else if (kMergeLate && b >= kPB - H) issue_o_gu(wave, lane, kMergeEarlyRows, RPWg, false);
            PK_MARK(l, 8);
        }

        // ================= P4: gate/up + SwiGLU =====================================
        lds_barrier();  // xin / rows_s readers (P3) are done
        {
            STAGE_IDS();
            if (!kQkvAfterDown && l + 1 < p.L) load_wq(lay_s[l + 1].wqkv, wave, lane);
            constexpr int NX = NXD;
            float gv[NX];
#pragma unroll
            for (int j = 0; j < NX; j++) gv[j] = tid + j * kPT < DIM ? gld(Ly.ffn_norm, tid + j * kPT) : 0.f;
            int idx[NX];
#pragma unroll
            for (int j = 0; j < NX; j++) idx[j] = tid + j * kPT < DIM ? OFF_XM + tid + j * kPT : -1;
            float xv[NX];
            ll_wait<NX>(cur, idx, xv, ep, dead, p.err, p.spin_limit);
            PK_MARK(l, 9);
            // Where attention blocks hold most of the down rows (llama2.c stories110M: 192 attention
            // blocks, down rows on the first 96), the blocks that did not take theirs early copy them
            // into LDS (direct global-to-LDS loads, no registers) once the gate/up input is here, so they
            // stream during the gate/up stage: 5,443 -> 5,561 tok/s; at C3, whose free blocks hold them
            // in registers, the same copies by the attention and merge blocks cost 0.560 -> 0.571 ms, and
            // at C4 (bf16: 8 of 12 chunks fit) copying part of them cost 0.872 -> 0.885 ms.
            if (kDmaChunks > 0 && has_o && !early_d) {
                const int rowd = b * RO + wave / WPR, cold = (wave % WPR) * (F / WPR);
                const char* src = reinterpret_cast<const char*>(Ly.w2) + ((size_t)rowd * F + cold) * sizeof(TW) + lane * 16;
#pragma unroll
                for (int c = 0; c < kDmaChunks; c++)
                    __builtin_amdgcn_global_load_lds((const void*)(src + (size_t)c * CW * sizeof(TW)),
                                                     (pk_lds_void*)(dyn_lds + (wave * kDmaChunks + c) * 1024), 16, 0, 0);
            }
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NX; j++) {
                const int i = tid + j * kPT;
                if (i < DIM) {
                    ss = fmaf(xv[j], xv[j], ss);
                    xmr[i] = xv[j];
                    xin[i] = xv[j] * gv[j];
                }
            }
            const float tot = block_sum(ss, red, lane, wave);
            PK_MARK(l, 22);
            const float rn = 1.0f / sqrtf(tot / (float)DIM + p.eps);
            float av[RPWg];
#pragma unroll
            for (int i = 0; i < RPWg; i++) {
                float a = 0.f;
#pragma unroll
                for (int c = 0; c < NCg; c++) a = WR::dot(wg[i][c], &xin[c * CW + lane * WR::V], a);
                av[i] = a;
            }
            gemv::dpp_sum_lane63_n(av);
#pragma unroll
            for (int i = 0; i < RPWg; i++)
                if (lane == 63) rows_s[wave * RPWg + i] = av[i] * rn;
            lds_barrier();
            if (tid < RG) {
                const float gt = rows_s[tid], u = rows_s[RG + tid];
                const float sg = 1.0f / (expf(-gt) + 1.0f);
                ll_put(cur + OFF_H + b * RG + tid, ep, u * (gt * sg));
            }
            PK_MARK(l, 10);
        }

        // ================= P5: down + residual ======================================
        lds_barrier();  // xin / rows_s readers (P4) are done
        {
            STAGE_IDS();
            const int row = b * RO + wave / WPR, col0 = (wave % WPR) * (F / WPR);
            if (has_o && !early_d) {  // (the chunks past the copied ones)
#pragma unroll
                for (int c = kDmaChunks; c < NCd; c++)
                    wd[c] = WR::load(Ly.w2, (size_t)row * F + col0 + c * CW + lane * WR::V);
            }
            constexpr int NH = F / kPT > 0 ? (F + kPT - 1) / kPT : 1;
            int idx[NH];
#pragma unroll
            for (int j = 0; j < NH; j++) idx[j] = has_o && tid + j * kPT < F ? OFF_H + tid + j * kPT : -1;
            float hv[NH];
            ll_wait<NH>(cur, idx, hv, ep, dead, p.err, p.spin_limit);
            PK_MARK(l, 11);
            if (kDmaChunks > 0 && has_o && !early_d) {
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's copies have landed
#pragma unroll
                for (int c = 0; c < kDmaChunks; c++)
                    wd[c] = *reinterpret_cast<const wraw*>(dyn_lds + (wave * kDmaChunks + c) * 1024 + lane * 16);
            }
#pragma unroll
            for (int j = 0; j < NH; j++)
                if (tid + j * kPT < F) xin[tid + j * kPT] = hv[j];
            lds_barrier();
            PK_MARK(l, 23);
            float a = 0.f;
            if (has_o) {
#pragma unroll
                for (int c = 0; c < NCd; c++) a = WR::dot(wd[c], &xin[col0 + c * CW + lane * WR::V], a);
            }
            a = gemv::dpp_sum_lane63(a);
            if (lane == 63) rows_s[wave] = a;
            lds_barrier();
            if (tid < RO && has_o) {
                float sum = 0.f;
#pragma unroll
                for (int k = 0; k < WPR; k++) sum += rows_s[tid * WPR + k];
                const int r = b * RO + tid;
                const float xn = xmr[r] + sum;
                ll_put(cur + OFF_XA + r, ep, xn);
                if (l + 1 == p.L) p.x[r] = xn;
            }
            PK_MARK(l, 12);
            if (kQkvAfterDown && l + 1 < p.L) load_wq(lay_s[l + 1].wqkv, wave, lane);
        }
    }

    // ================= P6: final RMSNorm + logits + greedy keys ======================
    // (Qwen3.java:401-405; the tied head reads the embedding rows.)  Wavefront gw of the grid takes
    // RB consecutive vocabulary rows at a time, batches kPB * kPW * RB rows apart (all wavefronts
    // stream neighbouring rows together), the next batch in flight while one is used (the first
    // before the wait for x).
    lds_barrier();
    {
        STAGE_IDS();
        constexpr int RB = 4, NCl = DIM / CW;
        const int r1 = p.vocab;
        const int gw = b * kPW + wave;
        wraw wa[RB][NCl], wb[RB][NCl];
        auto load_batch = [&](wraw (&w)[RB][NCl], int rbase) {
#pragma unroll
            for (int i = 0; i < RB; i++) {
                const int r = min(rbase + i, r1 - 1);
#pragma unroll
                for (int c = 0; c < NCl; c++) w[i][c] = WR::load(p.lm_head, (size_t)r * DIM + c * CW + lane * WR::V);
            }
        };
        const int first = gw * RB;
        if (first < r1) load_batch(wa, first);
        constexpr int NX = NXD;
        float gv[NX];
#pragma unroll
        for (int j = 0; j < NX; j++) gv[j] = tid + j * kPT < DIM ? gld(p.final_norm, tid + j * kPT) : 0.f;
        int idx[NX];
#pragma unroll
        for (int j = 0; j < NX; j++) idx[j] = tid + j * kPT < DIM ? OFF_XA + tid + j * kPT : -1;
        float xv[NX];
        ll_wait<NX>(p.ll + (size_t)((p.L - 1) & 1) * PAR_WORDS, idx, xv, base + (unsigned)p.L, dead, p.err, p.spin_limit);
        PK_MARK(p.L - 1, 13);
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NX; j++) {
            const int i = tid + j * kPT;
            if (i < DIM) {
                ss = fmaf(xv[j], xv[j], ss);
                xin[i] = xv[j] * gv[j];
            }
        }
        const float tot = block_sum(ss, red, lane, wave);
        const float rn = 1.0f / sqrtf(tot / (float)DIM + p.eps);
        float xq[NCl][WR::V];
#pragma unroll
        for (int c = 0; c < NCl; c++)
#pragma unroll
            for (int v = 0; v < WR::V; v += 4) {
                const float4 t = *reinterpret_cast<const float4*>(&xin[c * CW + lane * WR::V + v]);
                xq[c][v] = t.x; xq[c][v + 1] = t.y; xq[c][v + 2] = t.z; xq[c][v + 3] = t.w;
            }
        unsigned long long best = 0ull;  // (lane 63)
        auto use_batch = [&](const wraw (&w)[RB][NCl], int rbase) {
            float av[RB];
#pragma unroll
            for (int i = 0; i < RB; i++) {
                float a = 0.f;
#pragma unroll
                for (int c = 0; c < NCl; c++) a = WR::dot(w[i][c], xq[c], a);
                av[i] = a;
            }
            gemv::dpp_sum_lane63_n(av);
#pragma unroll
            for (int i = 0; i < RB; i++) {
                const float a = av[i] * rn;
                const int r = rbase + i;
                if (lane == 63 && r < r1) {
                    if (p.logits) p.logits[r] = a;
                    const unsigned long long k = gemv::argmax_key(a, r);
                    best = k > best ? k : best;
                }
            }
        };
        constexpr int STEP = RB * kPB * kPW;
        for (int rb = first; rb < r1; rb += 2 * STEP) {
            if (rb + STEP < r1) load_batch(wb, rb + STEP);
            use_batch(wa, rb);
            if (rb + STEP >= r1) break;
            if (rb + 2 * STEP < r1) load_batch(wa, rb + 2 * STEP);
            use_batch(wb, rb + STEP);
        }
        if (lane == 63 && best) atomicMax(p.keys + ((b * kPW + wave) & (kArgmaxSlots - 1)), best);
    }
    PK_MARK(p.L - 1, 14);

    // every block read the epoch base before block 0 could get here (block 0's last stage waited
    // for every block's last output), so the next launch's base can be published now
    if (b == 0 && tid0 == 0) p.state[3] = (int)(base + (unsigned)p.L);
}

template <int DIM, int F, int H, int KV, int HD, int SMAX>
constexpr size_t ll_words() {
    constexpr int QD = H * HD, KVD = KV * HD, G = H / KV;
    constexpr int RQ = pick_rq(QD + 2 * KVD, HD);
    return 2 * (size_t)(2 * DIM + QD + 2 * KVD + KV * SMAX * G * (HD + 2) + QD + F + (QD + KVD) / RQ);
}

template <typename TW, typename KT, int DIM, int F, int H, int KV, int HD, int SMAX>
int launch_t(const DecodePersistentLaunch& a, hipStream_t st) {
    PParams p;
    p.layers = reinterpret_cast<const PLayer*>(a.layers);
    p.L = a.layer_count;
    p.x = a.x; p.kcache = a.kcache; p.vcache = a.vcache; p.S = a.max_seq; p.rope_tab = a.rope_tab;
    p.state = a.state; p.ll = a.ll; p.err = a.err; p.eps = a.eps; p.per_head = a.per_head_norm;
    p.spin_limit = a.wait_limit ? a.wait_limit : kSpinLimit;
    p.final_norm = a.final_norm; p.lm_head = a.lm_head; p.vocab = a.vocab; p.logits = a.logits; p.keys = a.keys;
    auto kern = decode_persistent_kernel<TW, KT, DIM, F, H, KV, HD, SMAX>;  // (its LDS attribute is set by fits_t)
    // A plain launch (a cooperative one measured ~20 us longer per step): every block must be resident
    // at once, which decode_persistent_supported checks (one 512-thread block per CU, kPB CUs) and
    // which holds while nothing else runs on the device; if some block were not, the others' waits
    // time out, the error flag is set and the launch still completes.  (ar_launch: while a timing
    // hook is installed the dispatch itself records the start / stop events.)
    ar_launch(kern, dim3(kPB), dim3(kPT), kPadLds, st, p);
    AR_LAUNCH_CHECK();
    return AR_HIP_OK;
}

template <typename TW, typename KT, int DIM, int F, int H, int KV, int HD, int SMAX>
int fits_t(int* blocks_per_cu) {
    auto kern = decode_persistent_kernel<TW, KT, DIM, F, H, KV, HD, SMAX>;
    // no private (scratch) memory: the dispatcher may hold back waves that need scratch beyond the
    // runtime's scratch allocation, and every block of this kernel must be resident at once
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, (const void*)kern) != hipSuccess || fa.localSizeBytes != 0) return 0;
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kPadLds) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, (const void*)kern, kPT, kPadLds) != hipSuccess)
        return 0;
    return 1;
}

// The instantiated shapes, each with an fp32 and an fp16 KV cache: (weight type, dim, FFN, heads, KV
// heads, head size, attention splits per KV head).  Qwen3-0.6B with fp32 weights (contexts of a few hundred rows: 8 splits), Qwen3-1.7B with bf16
// weights (2K-row contexts: 28 splits of ~80 rows, 224 attention blocks), and the llama2.c stories110M
// shape with fp32 weights (12 heads of 64, no QK-norm gains, 1K-row contexts: 16 splits of <= 64 rows,
// 192 attention blocks; QKV rows on 144 blocks, O / down rows on 96).
#define AR_PERSISTENT_SHAPES(X)                         \
    X(AR_DTYPE_F32, float, 1024, 3072, 16, 8, 128, 8)  \
    X(AR_DTYPE_BF16, uint16_t, 2048, 6144, 16, 8, 128, 28) \
    X(AR_DTYPE_F32, float, 768, 2048, 12, 12, 64, 16)

}  // namespace

size_t decode_persistent_layer_bytes() { return sizeof(PLayer); }

size_t decode_persistent_ll_words(int wdtype, int dim, int F, int heads, int kv_heads, int hd) {
#define AR_X(DT, TW, D, FF, HH, KK, HDD, SM) \
    if (wdtype == DT && dim == D && F == FF && heads == HH && kv_heads == KK && hd == HDD) return ll_words<D, FF, HH, KK, HDD, SM>();
    AR_PERSISTENT_SHAPES(AR_X)
#undef AR_X
    return 0;
}

int decode_persistent_layer_entry(void* dst, const void* wqkv, const void* wo, const void* w1, const void* w3,
                                  const void* w2, const float* attn_norm, const float* ffn_norm, const float* q_norm,
                                  const float* k_norm, const float* bqkv) {
    PLayer e{wqkv, wo, w1, w3, w2, attn_norm, ffn_norm, q_norm, k_norm, bqkv};
    __builtin_memcpy(dst, &e, sizeof(e));
    return AR_HIP_OK;
}

bool decode_persistent_supported(int wdtype, int dim, int F, int heads, int kv_heads, int hd, bool kv16) {
    if (decode_persistent_ll_words(wdtype, dim, F, heads, kv_heads, hd) == 0) return false;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
    int ok = 0;
#define AR_X(DT, TW, D, FF, HH, KK, HDD, SM)                                                              \
    if (wdtype == DT && dim == D && F == FF && heads == HH && kv_heads == KK && hd == HDD)                \
        ok = kv16 ? fits_t<TW, _Float16, D, FF, HH, KK, HDD, SM>(&per_cu) : fits_t<TW, float, D, FF, HH, KK, HDD, SM>(&per_cu);
    AR_PERSISTENT_SHAPES(AR_X)
#undef AR_X
    return ok && per_cu >= 1 && (long long)per_cu * cus >= kPB;
}

int launch_decode_persistent(const DecodePersistentLaunch& a, hipStream_t st) {
    AR_CHECK_ARG(a.layers && a.x && a.kcache && a.vcache && a.rope_tab && a.state && a.ll && a.err && a.layer_count > 0 &&
                     a.final_norm && a.lm_head && a.keys,
                 "persistent decode: null argument");
    AR_CHECK_ARG(a.vocab >= kPB, "persistent decode: vocabulary %d below %d rows", a.vocab, kPB);
    AR_CHECK_ARG(a.max_seq > 0, "persistent decode: empty cache");
    AR_CHECK_ARG(a.layer_count <= kMaxLayers, "persistent decode: %d layers exceed %d", a.layer_count, kMaxLayers);
    if (ar_check_ptrs_enabled()) {
        const char* k = "persistent decode";
        const size_t wb = a.wdtype == AR_DTYPE_BF16 ? 2 : 4, D = a.dim, L = a.layer_count;
        const size_t cache = L * a.kv_heads * (size_t)a.max_seq * a.head_dim * (a.kv16 ? 2 : 4);
        AR_TRY(ar_check_range(a.layers, L * decode_persistent_layer_bytes(), k, "layer table"));
        AR_TRY(ar_check_range(a.x, D * 4, k, "residual row"));
        AR_TRY(ar_check_range(a.kcache, cache, k, "key cache"));
        AR_TRY(ar_check_range(a.vcache, cache, k, "value cache"));
        AR_TRY(ar_check_range(a.rope_tab, (size_t)a.max_seq * (a.head_dim / 2) * sizeof(float2), k, "RoPE table"));
        AR_TRY(ar_check_range(a.state, 4 * sizeof(int), k, "loop state"));
        AR_TRY(ar_check_range(a.ll, decode_persistent_ll_words(a.wdtype, a.dim, a.hidden_dim, a.heads, a.kv_heads,
                                                               a.head_dim) * 8, k, "exchange words"));
        AR_TRY(ar_check_range(a.err, sizeof(int), k, "error flag"));
        AR_TRY(ar_check_range(a.final_norm, D * 4, k, "final norm gain"));
        AR_TRY(ar_check_range(a.lm_head, (size_t)a.vocab * D * wb, k, "head"));
        AR_TRY(ar_check_range(a.logits, (size_t)a.vocab * 4, k, "logits"));
        AR_TRY(ar_check_range(a.keys, (size_t)kArgmaxSlots * 8, k, "argmax keys"));
    }
#define AR_X(DT, TW, D, FF, HH, KK, HDD, SM)                                                                          \
    if (a.wdtype == DT && a.dim == D && a.hidden_dim == FF && a.heads == HH && a.kv_heads == KK && a.head_dim == HDD) \
        return a.kv16 ? launch_t<TW, _Float16, D, FF, HH, KK, HDD, SM>(a, st) : launch_t<TW, float, D, FF, HH, KK, HDD, SM>(a, st);
    AR_PERSISTENT_SHAPES(AR_X)
#undef AR_X
    ar_set_error("persistent decode: weight type %d, dim %d, hidden %d, heads %d/%d, head size %d has no instantiation",
                 a.wdtype, a.dim, a.hidden_dim, a.heads, a.kv_heads, a.head_dim);
    return AR_HIP_ERR_INVALID;
}
