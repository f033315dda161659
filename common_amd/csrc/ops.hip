// Stand-alone operator entry points of the C-ABI (device pointers, context stream).
// Each mirrors one reference layer feature; see include/ar_hip.h for the citations.
#include <cmath>

#include "ar_hip_internal.h"

extern "C" int ar_hip_rmsnorm(ar_hip_ctx* ctx, const float* x, const float* w, float* y, int rows, int n, float eps) {
    AR_CHECK_ARG(ctx, "ctx is null");
    return launch_rmsnorm(x, w, y, rows, n, eps, ctx->stream);
}

extern "C" int ar_hip_dense(ar_hip_ctx* ctx, const void* W, int w_dtype, const float* bias, const float* x,
                            const float* norm_w, float eps, float* y, int rows, int cols, int batch) {
    AR_CHECK_ARG(ctx, "ctx is null");
    GemvLaunch a;
    a.w = W; a.wdtype = w_dtype; a.bias = bias; a.x = x; a.x_stride = cols; a.norm_w = norm_w; a.eps = eps;
    a.y = y; a.y_stride = rows; a.rows = rows; a.cols = cols; a.batch = batch; a.epilogue = GEMV_EPI_STORE;
    return launch_gemv(a, ctx->stream);
}

extern "C" int ar_hip_swiglu(ar_hip_ctx* ctx, const void* W_gate, const void* W_up, int w_dtype, const float* x,
                             const float* norm_w, float eps, float* y, int rows, int cols, int batch) {
    AR_CHECK_ARG(ctx, "ctx is null");
    GemvLaunch a;
    a.w = W_gate; a.w2 = W_up; a.wdtype = w_dtype; a.x = x; a.x_stride = cols; a.norm_w = norm_w; a.eps = eps;
    a.y = y; a.y_stride = rows; a.rows = rows; a.cols = cols; a.batch = batch; a.epilogue = GEMV_EPI_SWIGLU;
    return launch_gemv(a, ctx->stream);
}

extern "C" int ar_hip_rope(ar_hip_ctx* ctx, float* x, int heads, int head_dim, int pos, double theta, int rows) {
    AR_CHECK_ARG(ctx, "ctx is null");
    return launch_rope(x, heads, head_dim, pos, theta, rows, heads * head_dim, ctx->stream);
}

extern "C" int ar_hip_index_of_max(ar_hip_ctx* ctx, const float* x, int rows, int n, int32_t* out_device) {
    AR_CHECK_ARG(ctx, "ctx is null");
    return launch_index_of_max(x, rows, n, out_device, ctx->stream);
}

namespace {
// Workspace the stand-alone ops keep between calls (attention split partials, the sampler's
// passes).  Grown on demand; freed with the context's allocations.
struct AttnScratch {
    size_t part_floats = 0, ml_floats = 0, smp_bytes = 0;
    float* part_o = nullptr;
    float* part_ml = nullptr;
    void* smp = nullptr;
};
std::mutex g_attn_mu;
std::unordered_map<ar_hip_ctx*, AttnScratch> g_attn;

int grow(ar_hip_ctx* ctx, void** p, size_t* have, size_t need, size_t elem) {
    if (*have >= need && *p) return AR_HIP_OK;
    if (*p) AR_TRY(ar_ctx_free(ctx, *p));
    *p = nullptr;
    *have = 0;
    AR_TRY(ar_ctx_alloc(ctx, need * elem, p));
    *have = need;
    return AR_HIP_OK;
}
}  // namespace

namespace {
int attention_args(ar_hip_ctx* ctx, const float* q, const float* k, const float* v, const float* q_norm,
                   const float* k_norm, float qk_eps, int qk_norm_mode, float* k_cache, float* v_cache, int max_seq,
                   int pos, int heads, int kv_heads, int head_dim, double rope_theta, float* out, AttnLaunch* a) {
    AR_CHECK_ARG(ctx && q && k && v && k_cache && v_cache && out, "attention: null pointer");
    AR_CHECK_ARG(pos >= 0 && pos < max_seq, "attention: position %d outside cache of %d rows", pos, max_seq);
    AR_CHECK_ARG(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "attention: bad head counts");
    AR_CHECK_ARG(qk_norm_mode == AR_QK_NORM_WHOLE || qk_norm_mode == AR_QK_NORM_PER_HEAD, "attention: bad qk-norm mode");
    a->q = q; a->k = k; a->v = v; a->qkv_stride = 0; a->q_norm = q_norm; a->k_norm = k_norm; a->qk_eps = qk_eps;
    a->per_head_norm = qk_norm_mode == AR_QK_NORM_PER_HEAD; a->kcache = k_cache; a->vcache = v_cache;
    a->max_seq = max_seq; a->pos = nullptr; a->pos_value = pos; a->heads = heads; a->kv_heads = kv_heads;
    a->head_dim = head_dim; a->rope_theta = rope_theta; a->max_splits = attention_max_splits(max_seq, kv_heads, 1, false);
    a->out = out; a->out_stride = heads * head_dim; a->batch = 1;
    return AR_HIP_OK;
}
}  // namespace

extern "C" int ar_hip_attention_decode(ar_hip_ctx* ctx, const float* q, const float* k, const float* v,
                                       const float* q_norm, const float* k_norm, float qk_eps, int qk_norm_mode,
                                       float* k_cache, float* v_cache, int max_seq, int pos, int heads, int kv_heads,
                                       int head_dim, double rope_theta, float* out) {
    AttnLaunch a;
    AR_TRY(attention_args(ctx, q, k, v, q_norm, k_norm, qk_eps, qk_norm_mode, k_cache, v_cache, max_seq, pos, heads,
                          kv_heads, head_dim, rope_theta, out, &a));
    std::lock_guard<std::mutex> lk(g_attn_mu);
    AttnScratch& s = g_attn[ctx];
    AR_TRY(grow(ctx, (void**)&s.part_o, &s.part_floats, attention_partial_floats(1, heads, a.max_splits, head_dim),
                sizeof(float)));
    AR_TRY(grow(ctx, (void**)&s.part_ml, &s.ml_floats, (size_t)heads * a.max_splits * 2, sizeof(float)));
    a.part_o = s.part_o;
    a.part_ml = s.part_ml;
    return launch_attention_decode(a, ctx->stream);
}

// ---- allocation-free attention -----------------------------------------------------------
// The split partials of ar_hip_attention_decode_noalloc live in this fixed array: each GPU the
// library runs on holds one copy (1 MiB) until the process ends.  Host code never passes the
// array's name to a kernel: ar_ops_init looks up this device's address of it once per context,
// with the context's device current, and launches use that address.
constexpr size_t kNoAllocScratchFloats = (size_t)1 << 18;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
std::atomic<float*> g_scratch_addr[kMaxDevices];  // per device: its copy's address, once looked up
}

int ar_ops_init(ar_hip_ctx* ctx) {
    const bool cached = ctx->device >= 0 && ctx->device < kMaxDevices;
    float* addr = cached ? g_scratch_addr[ctx->device].load() : nullptr;
    if (!addr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            ar_set_error("hipGetSymbolAddress(scratch) on device %d: %s", ctx->device,
                         e != hipSuccess ? hipGetErrorString(e) : "null address");
            return AR_HIP_ERR_HIP;
        }
        addr = static_cast<float*>(ptr);
        if (cached) g_scratch_addr[ctx->device].store(addr);
    }
    ctx->noalloc_scratch = addr;
    return AR_HIP_OK;
}

extern "C" int ar_hip_attention_decode_noalloc(ar_hip_ctx* ctx, const float* q, const float* k, const float* v,
                                               const float* q_norm, const float* k_norm, float qk_eps,
                                               int qk_norm_mode, float* k_cache, float* v_cache, int max_seq, int pos,
                                               int heads, int kv_heads, int head_dim, double rope_theta, float* out) {
    AttnLaunch a;
    AR_TRY(attention_args(ctx, q, k, v, q_norm, k_norm, qk_eps, qk_norm_mode, k_cache, v_cache, max_seq, pos, heads,
                          kv_heads, head_dim, rope_theta, out, &a));
    AR_CHECK_ARG(ctx->noalloc_scratch, "attention (no-alloc): scratch address of device %d unknown", ctx->device);
    // partial outputs [heads][splits][hd] at the start, (max, sum) pairs [heads][splits][2] after
    // them at a 256-byte boundary.  Nothing needs clearing: the combine uses only the splits this
    // call's attention launch writes (it may load the stale slots past them, never uses them).
    const size_t o_floats = attention_partial_floats(1, heads, a.max_splits, head_dim);
    const size_t ml_off = (o_floats + 63) / 64 * 64;
    const size_t need = ml_off + (size_t)heads * a.max_splits * 2;
    AR_CHECK_ARG(need <= kNoAllocScratchFloats,
                 "attention (no-alloc): %d heads x %d splits x (%d + 2) floats of partials exceed the %zu-float "
                 "scratch (cache of %d rows); use ar_hip_attention_decode",
                 heads, a.max_splits, head_dim, kNoAllocScratchFloats, max_seq);
    a.part_o = ctx->noalloc_scratch;
    a.part_ml = ctx->noalloc_scratch + ml_off;
    return launch_attention_decode(a, ctx->stream);
}

extern "C" int ar_hip_sample(ar_hip_ctx* ctx, const float* logits, int rows, int n, int mode, double temperature,
                             double top_p, uint64_t* rng_state, int32_t* out) {
    AR_CHECK_ARG(ctx && logits && out, "sample: null pointer");
    AR_CHECK_ARG(rows > 0 && n > 0, "sample: empty input");
    AR_CHECK_ARG(mode == AR_SAMPLE_TOKEN || mode == AR_SAMPLE_MODEL, "sample: unknown mode %d", mode);
    if (sample_is_greedy(mode, temperature))  // first maximum, no draw (AutoregressiveModel.java:327-337,419-420)
        return launch_index_of_max(logits, rows, n, out, ctx->stream);
    AR_CHECK_ARG(rng_state, "sample: null generator state");
    std::lock_guard<std::mutex> lk(g_attn_mu);
    AttnScratch& s = g_attn[ctx];
    AR_TRY(grow(ctx, &s.smp, &s.smp_bytes, sample_workspace_bytes(rows, n), 1));
    AR_TRY(sample_workspace_clear(s.smp, rows, n, ctx->stream));  // the layout depends on (rows, n)
    SampleLaunch l;
    l.logits = logits; l.logits_stride = n; l.rows = rows; l.vocab = n; l.mode = mode; l.temperature = temperature;
    l.top_p = top_p; l.work = s.smp; l.rng = (unsigned long long*)rng_state; l.out = out;
    return launch_sample(l, ctx->stream);
}

// Called from ar_hip_destroy's owner before the context goes away.
void ar_ops_release(ar_hip_ctx* ctx) {
    std::lock_guard<std::mutex> lk(g_attn_mu);
    g_attn.erase(ctx);  // the allocations themselves are freed with the context
}

extern "C" int ar_hip_gemm_bf16(ar_hip_ctx* ctx, const uint16_t* A, const uint16_t* W, const uint16_t* W2,
                                const float* bias, float* C, uint16_t* O, int M, int N, int K, int epilogue) {
    AR_CHECK_ARG(ctx, "ctx is null");
    GemmLaunch g;
    g.A = A; g.W = W; g.W2 = W2; g.M = M; g.N = N; g.K = K; g.lda = K; g.ldw = K; g.bias = bias; g.C = C; g.ldc = N;
    g.O = O; g.ldo = N;
    switch (epilogue) {
        case AR_GEMM_STORE: g.epilogue = GEMV_EPI_STORE; break;
        case AR_GEMM_RESIDUAL: g.epilogue = GEMV_EPI_RESIDUAL; break;
        case AR_GEMM_SWIGLU: g.epilogue = GEMV_EPI_SWIGLU; break;
        default: AR_CHECK_ARG(false, "GEMM: unknown epilogue %d", epilogue);
    }
    return launch_gemm(g, ctx->stream);
}

extern "C" int ar_hip_gemm_f32(ar_hip_ctx* ctx, const float* A, const float* W, const float* W2, const float* bias,
                               float* C, int M, int N, int K, int epilogue) {
    AR_CHECK_ARG(ctx, "ctx is null");
    GemmF32Launch g;
    g.A = A; g.W = W; g.W2 = W2; g.bias = bias; g.C = C; g.M = M; g.N = N; g.K = K; g.lda = K; g.ldw = K; g.ldc = N;
    switch (epilogue) {
        case AR_GEMM_STORE: g.epilogue = GEMV_EPI_STORE; break;
        case AR_GEMM_RESIDUAL: g.epilogue = GEMV_EPI_RESIDUAL; break;
        case AR_GEMM_SWIGLU: g.epilogue = GEMV_EPI_SWIGLU; break;
        default: AR_CHECK_ARG(false, "GEMM f32: unknown epilogue %d", epilogue);
    }
    return launch_gemm_f32(g, ctx->stream);
}
