// Qwen3 decode-step plan: device-resident weights, KV caches and token loop.
//
// Stands in for Qwen3.model + CompiledModel + AutoregressiveModel
// (engine/ml/.../qwen3/Qwen3.java:334-415, domain/graph/.../model/CompiledModel.java:189-197,
//  engine/ml/.../AutoregressiveModel.java:203-220,295-308,405-434).  The reference runs ~877
// generated ops per layer with host-side cache writes; one step here is
//   embed, then per layer [QKV GEMV (+RMSNorm) | attention (+QK-norm, RoPE, cache write) |
//   O GEMV (+residual) | gate/up GEMV (+RMSNorm, SwiGLU) | down GEMV (+residual)],
//   then logits GEMV (+final RMSNorm, argmax, position advance)
// on one stream, optionally replayed from a captured HIP graph.  Tokens and the position stay
// on the device, so many steps can be enqueued without a host round trip.
#include <cmath>
#include <cstring>
#include <string>
#include <algorithm>
#include <vector>

#include "ar_hip_internal.h"

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Slot {
    void* dst = nullptr;     // device destination
    int64_t elems = 0;
    bool matrix = false;     // stored in the model's weight dtype (else fp32)
    bool required = true;
    bool filled = false;
};

struct Layer {
    void* wqkv = nullptr;    // rows: q (q_dim) | k (kv_dim) | v (kv_dim), cols dim
    void* wo = nullptr;
    void* w1 = nullptr;      // gate
    void* w3 = nullptr;      // up
    void* w2 = nullptr;      // down
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    float* q_norm = nullptr;
    float* k_norm = nullptr;
    float* bqkv = nullptr;
    // fragment-ordered copies of wo, w1, w3, w2 for the batched decode GEMVs (gemv_frag.hip)
    uint16_t* fo = nullptr;
    uint16_t* f1 = nullptr;
    uint16_t* f3 = nullptr;
    uint16_t* f2 = nullptr;
};

}  // namespace

struct ar_qwen3 {
    ar_hip_ctx* ctx = nullptr;
    ar_qwen3_cfg cfg{};
    int q_dim = 0, kv_dim = 0, qkv_dim = 0, B = 1, S = 0;
    size_t wbytes = 4;
    char* arena = nullptr;
    size_t arena_bytes = 0;
    std::vector<Layer> layers;
    void* embed = nullptr;
    void* lm_head = nullptr;
    float* final_norm = nullptr;
    std::unordered_map<std::string, Slot> slots;
    bool finalized = false;

    // activations and state
    float* x = nullptr;       // [B][dim] residual stream
    float* qkv = nullptr;     // [B][qkv_dim]
    float* attn = nullptr;    // [B][q_dim]
    float* act = nullptr;     // [B][F]
    float* logits = nullptr;  // [B][V]
    void* kcache = nullptr;   // [L][B][KV][S][hd], fp32 or fp16 (cfg.kv_dtype)
    void* vcache = nullptr;
    size_t kv_elem = 4;
    float* part_o = nullptr;
    float* part_ml = nullptr;
    // bf16 operand planes (hi then lo, [B][width] each) of the inputs of the MFMA-path GEMVs
    // (batch >= 3, bf16 weights), written by the kernel producing each input: residual stream x
    // (scaled by the next RMSNorm gain), attention output, SwiGLU output
    uint16_t* pl_x = nullptr;
    uint16_t* pl_attn = nullptr;
    uint16_t* pl_act = nullptr;
    // k-split workspace of the batch >= 3 MFMA GEMVs with few row tiles (O, down): partial tiles and
    // one arrival counter per 16-row tile of the residual stream (kept zero between launches)
    float* gv_part = nullptr;
    int gv_part_floats = 0;
    unsigned* gv_count = nullptr;
    int gv_count_n = 0;
    // batches of 3..8 with bf16 weights: the layers' O, gate/up and down matrices also in MFMA
    // fragment order (one buffer, made at finalize), read by those GEMVs of the decode step unless
    // switched off (ar_hip_qwen3_use_fragment_gemv); gv_ss [dim/16][16]: per-16-row sums of squares
    // of the residual stream after the O projection, published by it for the gate/up RMSNorm
    uint16_t* gv_frag = nullptr;
    float* gv_ss = nullptr;
    bool frag_on = true;
    unsigned long long* am_keys = nullptr;  // [B][kArgmaxSlots] greedy-token keys
    // token selection: greedy unless a sampling temperature is set (AR_SAMPLE_*); one
    // java.util.Random state per sequence, the sampler's workspace allocated on first use
    int smp_mode = AR_SAMPLE_MODEL;
    double smp_temperature = 0.0, smp_top_p = 1.0;
    unsigned long long* smp_rng = nullptr;  // [B]
    void* smp_work = nullptr;
    float2* rope_tab = nullptr;             // [S][hd/2] (cos, sin), computed in double on the host
    int* tokens = nullptr;    // [B][S+1]
    int* state = nullptr;     // {current position, prompt length, next position}
    float* staging = nullptr; // fp32 upload staging for dtype conversion
    size_t staging_floats = 0;
    int max_splits = 1;

    int host_pos = 0;
    int prompt_len = 0;
    std::vector<int> prompt_set;

    bool use_graph = true;
    hipGraphExec_t graph[2] = {nullptr, nullptr};  // [store logits]
    // set by the kernel-loop probe, which overwrites the step state: steps are refused until reset()
    bool needs_reset = false;

    // prefill buffers, sized for pf_rows = batch x prompt rows on first use
    size_t pf_rows = 0;
    float* pf_x = nullptr;       // [R][dim] residual stream
    uint16_t* pf_h = nullptr;    // [R][max(dim, q_dim)] fp16 GEMM input (normalised x / attention out);
                                 // fp32 for fp32 weights (as are pf_q and pf_act)
    float* pf_qkv = nullptr;     // [R][qkv_dim]
    uint16_t* pf_q = nullptr;    // [R][q_dim] fp16 normalised, rotated queries
    uint16_t* pf_act = nullptr;  // [R][F] fp16 SwiGLU output
    float* pf_part = nullptr;    // [kMaxKSplit][R][dim] k-slices of split residual projections
    size_t pf_part_rows = 0;
    uint16_t* pf_k16 = nullptr;  // [B][KV][Tp][hd] fp16 keys of the prompt rows
    uint16_t* pf_vt16 = nullptr; // [B][KV][hd][Tp] fp16 values, transposed (zeroed once: padded keys
                                 // get weight 0 and must not hold NaN bit patterns)
    int pf_tp = 0;
    // fp16 copies of the projection matrices for the prefill GEMMs (made on the first prefill)
    uint16_t* pf_w16 = nullptr;
    bool pf_w16_valid = false;
    // fp16 range flags (device): [0] an activation stored as fp16 overflowed during the last prefill,
    // [1] a weight did in the fp16 copies; either sends the prompt through the decode step instead
    int* pf_flag = nullptr;
    bool pf_w16_in_range = true;  // host copy of pf_flag[1] after the fp16 copies were made
    int pf_by_steps = 0;          // prefill calls that went through the decode step
    int pf_gemm = AR_PREFILL_GEMM_ROCBLAS;  // ar_hip_qwen3_prefill_gemm: products of the fp16 prefill
    uint16_t* pf_gu = nullptr;    // [R][2F] fp16 gate/up rows of the rocBLAS path
    size_t pf_gu_elems = 0;

    // persistent decode step (batch 1, fp32 or bf16 weights, fp32 or fp16 cache): every layer, the final RMSNorm, the
    // logits and the greedy keys in one launch (decode_persistent.hip) after the step-begin kernel
    bool pk_ok = false;          // shape, dtypes and device qualify; buffers below allocated
    bool pk_on = true;           // ar_hip_qwen3_use_persistent
    void* pk_layers = nullptr;   // device table of the layers' weight pointers
    uint64_t* pk_ll = nullptr;   // exchange words (uncached memory: ar_uncached_get)
    size_t pk_ll_words = 0;
    int* pk_err = nullptr;       // timeout / position flag of the last launches
    unsigned pk_wait_limit = 0;  // polls per cross-block wait before it is abandoned (0: kernel default)
    bool pk_suspended = false;   // steps being recomputed as separate launches after a timed-out step
    int pk_recomputed = 0;       // steps recomputed so (ar_hip_qwen3_persistent_recomputed)
    unsigned long long* smp_rng_saved = nullptr;  // [B] generator states before the last persistent call

    int timed = AR_KT_NONE;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> events;
    size_t events_used = 0;
};

namespace {

int alloc_zero(ar_qwen3* m, size_t bytes, void** p) {
    AR_TRY(ar_ctx_alloc(m->ctx, bytes, p));
    AR_HIP_TRY(hipMemsetAsync(*p, 0, bytes, m->ctx->stream));
    return AR_HIP_OK;
}

void release(ar_qwen3* m) {
    if (!m) return;
    for (auto& g : m->graph)
        if (g) hipGraphExecDestroy(g);
    for (auto& e : m->events) {
        hipEventDestroy(e.first);
        hipEventDestroy(e.second);
    }
    void* bufs[] = {m->arena, m->x, m->qkv, m->attn, m->act, m->logits, m->kcache, m->vcache, m->part_o,
                    m->part_ml, m->pl_x, m->pl_attn, m->pl_act, m->gv_part, m->gv_count, m->gv_frag, m->gv_ss,
                    m->am_keys, m->smp_rng,
                    m->smp_rng_saved, m->smp_work, m->rope_tab, m->tokens, m->state, m->staging,
                    m->pf_x, m->pf_h, m->pf_qkv, m->pf_q, m->pf_act, m->pf_part, m->pf_w16, m->pf_k16, m->pf_vt16,
                    m->pf_flag, m->pf_gu, m->pk_layers, m->pk_err};
    for (void* b : bufs)
        if (b) ar_ctx_free(m->ctx, b);
    if (m->pk_ll) {  // (uncached: back to the process-wide free list once no launch uses it)
        hipStreamSynchronize(m->ctx->stream);
        ar_uncached_put(m->pk_ll);
    }
    delete m;
}

int add_slot(ar_qwen3* m, const std::string& key, void* dst, int64_t elems, bool matrix, bool required = true) {
    Slot s;
    s.dst = dst;
    s.elems = elems;
    s.matrix = matrix;
    s.required = required;
    m->slots[key] = s;
    return AR_HIP_OK;
}

int invalidate_graphs(ar_qwen3* m) {
    for (auto& g : m->graph) {
        if (g) {
            AR_HIP_TRY(hipGraphExecDestroy(g));
            g = nullptr;
        }
    }
    return AR_HIP_OK;
}

// One decode step on the model's stream.
// The sampler over this step's logits: its draw replaces the greedy key that the next step feeds
// (only when that step is past the prompt, which the kernel reads from the loop state).
int enqueue_sample(ar_qwen3* m) {
    SampleLaunch s;
    s.logits = m->logits; s.logits_stride = m->cfg.vocab_size; s.rows = m->B; s.vocab = m->cfg.vocab_size;
    s.mode = m->smp_mode; s.temperature = m->smp_temperature; s.top_p = m->smp_top_p; s.work = m->smp_work;
    s.rng = m->smp_rng; s.state = m->state; s.keys = m->am_keys; s.keys_stride = kArgmaxSlots;
    return launch_sample(s, m->ctx->stream);
}

// bf16 operand planes of the decode step (hi then lo) of x (width dim), the attention output
// (q_dim) and the SwiGLU output (F), or nulls when the GEMVs convert their inputs themselves
struct StepPlanes {
    uint16_t *xh = nullptr, *xl = nullptr, *ah = nullptr, *al = nullptr, *hh = nullptr, *hl = nullptr;
};

StepPlanes step_planes(const ar_qwen3* m) {
    StepPlanes pl;
    const size_t B = m->B;
    pl.xh = m->pl_x;
    pl.xl = pl.xh ? pl.xh + B * m->cfg.dim : nullptr;
    pl.ah = m->pl_attn;
    pl.al = pl.ah ? pl.ah + B * m->q_dim : nullptr;
    pl.hh = m->pl_act;
    pl.hl = pl.hh ? pl.hh + B * m->cfg.hidden_dim : nullptr;
    return pl;
}

// The batched decode GEMVs read the fragment-ordered weight copies (gemv_frag.hip).
bool frag_active(const ar_qwen3* m) { return m->gv_frag != nullptr && m->frag_on; }

// Points an O / gate-up / down launch at the fragment-ordered copies and the shared workspace.
void use_frag(const ar_qwen3* m, GemvLaunch& g, const uint16_t* w, const uint16_t* w2, bool norm_in, bool ss_out) {
    g.w_frag = w;
    g.w2_frag = w2;
    g.ss_in = norm_in ? m->gv_ss : nullptr;
    g.ss_out = ss_out ? m->gv_ss : nullptr;
    g.kpart = m->gv_part;
    g.kpart_floats = m->gv_part_floats;
    g.kcount = m->gv_count;
    g.kcount_n = m->gv_count_n;
}

// One kernel class (AR_KT_*) of the decode step for layer l (the logits class ignores l), launched
// exactly as the step launches it.
int launch_class(ar_qwen3* m, int which, int l, const StepPlanes& pl, bool store_logits) {
    const ar_qwen3_cfg& c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int B = m->B, dim = c.dim, F = c.hidden_dim;
    switch (which) {
        case AR_KT_QKV: {  // QKV projection with the pre-attention RMSNorm fused in (AttentionFeatures.java:830-900)
            const Layer& L = m->layers[l];
            GemvLaunch g;
            g.wdtype = c.weight_dtype; g.batch = B; g.eps = (float)c.epsilon;
            g.w = L.wqkv; g.rows = m->qkv_dim; g.cols = dim; g.x = m->x; g.x_stride = dim; g.norm_w = L.attn_norm;
            g.bias = L.bqkv; g.y = m->qkv; g.y_stride = m->qkv_dim; g.epilogue = GEMV_EPI_STORE;
            g.x_hi = pl.xh; g.x_lo = pl.xl;
            // (QKV stays on the row-major MFMA GEMV: its planes-in-registers persistent form measured
            // 16.2 us per C5 layer in the step against 17.8 for the fragment-ordered form)
            return launch_gemv(g, st);
        }
        case AR_KT_ATTENTION: {
            const Layer& L = m->layers[l];
            const size_t layer_cache = (size_t)B * c.kv_head_count * m->S * c.head_size;
            AttnLaunch a;
            a.qkv = m->qkv; a.qkv_stride = m->qkv_dim; a.q_norm = L.q_norm; a.k_norm = L.k_norm;
            a.qk_eps = (float)c.epsilon; a.per_head_norm = c.qk_norm_mode == AR_QK_NORM_PER_HEAD;
            a.kcache = (char*)m->kcache + l * layer_cache * m->kv_elem;
            a.vcache = (char*)m->vcache + l * layer_cache * m->kv_elem;
            a.kv16 = c.kv_dtype == AR_DTYPE_F16; a.max_seq = m->S;
            a.pos = m->state; a.heads = c.head_count; a.kv_heads = c.kv_head_count; a.head_dim = c.head_size;
            a.rope_theta = c.rope_theta; a.rope_tab = m->rope_tab; a.max_splits = m->max_splits;
            a.part_o = m->part_o; a.part_ml = m->part_ml; a.out = m->attn; a.out_stride = m->q_dim; a.batch = B;
            a.out_hi = pl.ah; a.out_lo = pl.al;
            return launch_attention_decode(a, st);
        }
        case AR_KT_O: {  // O projection + residual (AttentionFeatures.java:922, :1704)
            const Layer& L = m->layers[l];
            GemvLaunch o;
            o.wdtype = c.weight_dtype; o.batch = B; o.w = L.wo; o.rows = dim; o.cols = m->q_dim; o.x = m->attn;
            o.x_stride = m->q_dim; o.y = m->x; o.y_stride = dim; o.epilogue = GEMV_EPI_RESIDUAL;
            o.x_hi = pl.ah; o.x_lo = pl.al; o.y_hi = pl.xh; o.y_lo = pl.xl; o.y_gain = L.ffn_norm;
            o.kpart = m->gv_part; o.kpart_floats = m->gv_part_floats; o.kcount = m->gv_count;
            o.kcount_n = m->gv_count ? (dim + 15) / 16 : 0;
            if (frag_active(m)) use_frag(m, o, L.fo, nullptr, false, true);
            return launch_gemv(o, st);
        }
        case AR_KT_GATE_UP: {  // gate/up with the pre-FFN RMSNorm and SwiGLU fused (FeedForwardFeatures.java:147-155)
            const Layer& L = m->layers[l];
            GemvLaunch u;
            u.wdtype = c.weight_dtype; u.batch = B; u.eps = (float)c.epsilon; u.w = L.w1; u.w2 = L.w3; u.rows = F;
            u.cols = dim; u.x = m->x; u.x_stride = dim; u.norm_w = L.ffn_norm; u.y = m->act; u.y_stride = F;
            u.epilogue = GEMV_EPI_SWIGLU;
            u.x_hi = pl.xh; u.x_lo = pl.xl; u.y_hi = pl.hh; u.y_lo = pl.hl;
            if (frag_active(m)) use_frag(m, u, L.f1, L.f3, true, false);
            return launch_gemv(u, st);
        }
        case AR_KT_DOWN: {  // down projection + residual (FeedForwardFeatures.java:156; AttentionFeatures.java:1705)
            const Layer& L = m->layers[l];
            GemvLaunch d;
            d.wdtype = c.weight_dtype; d.batch = B; d.w = L.w2; d.rows = dim; d.cols = F; d.x = m->act; d.x_stride = F;
            d.y = m->x; d.y_stride = dim; d.epilogue = GEMV_EPI_RESIDUAL;
            d.x_hi = pl.hh; d.x_lo = pl.hl; d.y_hi = pl.xh; d.y_lo = pl.xl;
            d.y_gain = l + 1 < c.layer_count ? m->layers[l + 1].attn_norm : m->final_norm;
            d.kpart = m->gv_part; d.kpart_floats = m->gv_part_floats; d.kcount = m->gv_count;
            d.kcount_n = m->gv_count ? (dim + 15) / 16 : 0;
            if (frag_active(m)) use_frag(m, d, L.f2, nullptr, false, false);
            return launch_gemv(d, st);
        }
        case AR_KT_LOGITS: {  // final RMSNorm + tied logits + greedy token (Qwen3.java:401-405)
            GemvLaunch h;
            h.wdtype = c.weight_dtype; h.batch = B; h.eps = (float)c.epsilon; h.w = m->lm_head; h.rows = c.vocab_size;
            const bool sampling = !sample_is_greedy(m->smp_mode, m->smp_temperature);
            h.cols = dim; h.x = m->x; h.x_stride = dim; h.norm_w = m->final_norm;
            h.y = (store_logits || sampling) ? m->logits : nullptr;
            h.y_stride = c.vocab_size; h.epilogue = GEMV_EPI_ARGMAX; h.keys = m->am_keys;
            h.x_hi = pl.xh; h.x_lo = pl.xl;
            return launch_gemv(h, st);
        }
    }
    ar_set_error("unknown kernel class %d", which);
    return AR_HIP_ERR_INVALID;
}

// The persistent kernel runs the layers and the logits of the step unless it is switched off, a kernel
// class of the multi-launch step is being timed, or a timed-out step is being recomputed.
bool persistent_active(const ar_qwen3* m) {
    return m->pk_ok && m->pk_on && !m->pk_suspended && (m->timed == AR_KT_NONE || m->timed == AR_KT_LAYERS);
}

int enqueue_step(ar_qwen3* m, bool store_logits) {
    const ar_qwen3_cfg& c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int B = m->B, dim = c.dim;
    // the timed class's kernels carry a start / stop event pair in their dispatches (ar_launch)
    LaunchTiming timing;
    struct TimingReset {  // an early error return must not leave the hook pointing at `timing`
        ~TimingReset() { g_launch_timing = nullptr; }
    } timing_reset;
    auto timed_begin = [&](int which) -> int {
        if (m->timed != which) return AR_HIP_OK;
        if (m->events_used == m->events.size()) {
            hipEvent_t a, b;
            AR_HIP_TRY(hipEventCreate(&a));
            AR_HIP_TRY(hipEventCreate(&b));
            m->events.push_back({a, b});
        }
        timing.start = m->events[m->events_used].first;
        timing.stop = m->events[m->events_used].second;
        timing.started = false;
        g_launch_timing = &timing;
        return AR_HIP_OK;
    };
    auto timed_end = [&](int which) -> int {
        if (m->timed != which) return AR_HIP_OK;
        g_launch_timing = nullptr;
        m->events_used++;
        return AR_HIP_OK;
    };
    auto timed_class = [&](int which, int l) -> int {
        AR_TRY(timed_begin(which));
        AR_TRY(launch_class(m, which, l, step_planes(m), store_logits));
        return timed_end(which);
    };

    if (persistent_active(m)) {
        const StepPlanes pl = step_planes(m);
        AR_TRY(launch_step_begin(m->embed, c.weight_dtype, dim, c.vocab_size, m->tokens, m->S + 1, m->am_keys,
                                 m->state, B, m->x, dim, pl.xh, pl.xl, m->layers[0].attn_norm, nullptr, st));
        DecodePersistentLaunch d;
        d.layers = m->pk_layers; d.layer_count = c.layer_count; d.wdtype = c.weight_dtype; d.dim = dim;
        d.hidden_dim = c.hidden_dim;
        d.heads = c.head_count; d.kv_heads = c.kv_head_count; d.head_dim = c.head_size; d.x = m->x;
        d.kcache = m->kcache; d.vcache = m->vcache; d.kv16 = c.kv_dtype == AR_DTYPE_F16; d.max_seq = m->S;
        d.rope_tab = m->rope_tab;
        d.state = m->state; d.ll = m->pk_ll; d.err = m->pk_err; d.wait_limit = m->pk_wait_limit;
        d.eps = (float)c.epsilon;
        d.per_head_norm = c.qk_norm_mode == AR_QK_NORM_PER_HEAD;
        const bool sampling = !sample_is_greedy(m->smp_mode, m->smp_temperature);
        d.final_norm = m->final_norm; d.lm_head = m->lm_head; d.vocab = c.vocab_size;
        d.logits = (store_logits || sampling) ? m->logits : nullptr; d.keys = m->am_keys;
        if (m->timed == AR_KT_LAYERS) {  // the launch's dispatch records the start / stop events
            AR_TRY(timed_begin(AR_KT_LAYERS));
            AR_TRY(launch_decode_persistent(d, st));
            AR_TRY(timed_end(AR_KT_LAYERS));
        } else {
            AR_TRY(launch_decode_persistent(d, st));
        }
        if (sampling) AR_TRY(enqueue_sample(m));
        return AR_HIP_OK;
    }
    const StepPlanes pl = step_planes(m);
    AR_TRY(launch_step_begin(m->embed, c.weight_dtype, dim, c.vocab_size, m->tokens, m->S + 1, m->am_keys, m->state,
                             B, m->x, dim, pl.xh, pl.xl, m->layers[0].attn_norm, nullptr, st));
    for (int l = 0; l < c.layer_count; l++) {
        for (int which : {AR_KT_QKV, AR_KT_ATTENTION, AR_KT_O, AR_KT_GATE_UP, AR_KT_DOWN}) AR_TRY(timed_class(which, l));
    }
    AR_TRY(timed_class(AR_KT_LOGITS, 0));
    if (!sample_is_greedy(m->smp_mode, m->smp_temperature)) AR_TRY(enqueue_sample(m));
    return AR_HIP_OK;
}

int run_step(ar_qwen3* m, bool store_logits) {
    hipStream_t st = m->ctx->stream;
    // (the persistent step is two launches, enqueued directly: replaying them from a graph measured
    // ~5 us per step slower)
    if (!m->use_graph || m->timed != AR_KT_NONE || persistent_active(m)) return enqueue_step(m, store_logits);
    hipGraphExec_t& ex = m->graph[store_logits ? 1 : 0];
    if (!ex) {
        hipGraph_t g = nullptr;
        AR_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_step(m, store_logits);
        hipError_t ce = hipStreamEndCapture(st, &g);
        if (rc != AR_HIP_OK) {
            if (g) hipGraphDestroy(g);
            return rc;
        }
        if (ce != hipSuccess) {
            ar_set_error("hipStreamEndCapture: %s", hipGetErrorString(ce));
            return AR_HIP_ERR_HIP;
        }
        hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (ie != hipSuccess) {
            ex = nullptr;
            ar_set_error("hipGraphInstantiate: %s", hipGetErrorString(ie));
            return AR_HIP_ERR_HIP;
        }
    }
    AR_HIP_TRY(hipGraphLaunch(ex, st));
    return AR_HIP_OK;
}

int upload(ar_qwen3* m, Slot& s, const void* src, int src_dtype, int64_t n) {
    hipStream_t st = m->ctx->stream;
    const int dst_dtype = s.matrix ? m->cfg.weight_dtype : AR_DTYPE_F32;
    if (src_dtype == dst_dtype) {
        const size_t bytes = (size_t)n * (dst_dtype == AR_DTYPE_BF16 ? 2 : 4);
        AR_HIP_TRY(hipMemcpyAsync(s.dst, src, bytes, hipMemcpyHostToDevice, st));
        AR_HIP_TRY(hipStreamSynchronize(st));
        return AR_HIP_OK;
    }
    if (src_dtype == AR_DTYPE_F32 && dst_dtype == AR_DTYPE_BF16) {
        // fp32 host values -> device staging -> bf16 (round to nearest even) in place
        const int64_t chunk = (int64_t)m->staging_floats;
        for (int64_t off = 0; off < n; off += chunk) {
            const int64_t len = std::min(chunk, n - off);
            AR_HIP_TRY(hipMemcpyAsync(m->staging, (const float*)src + off, (size_t)len * 4, hipMemcpyHostToDevice, st));
            AR_TRY(launch_f32_to_bf16(m->staging, (uint16_t*)s.dst + off, (size_t)len, st));
            AR_HIP_TRY(hipStreamSynchronize(st));
        }
        return AR_HIP_OK;
    }
    ar_set_error("weight upload from dtype %d into dtype %d is not supported", src_dtype, dst_dtype);
    return AR_HIP_ERR_INVALID;
}

}  // namespace

extern "C" int ar_hip_qwen3_create(ar_hip_ctx* ctx, const ar_qwen3_cfg* cfg, ar_qwen3** out) {
    AR_CHECK_ARG(ctx && cfg && out, "null argument");
    *out = nullptr;
    const ar_qwen3_cfg& c = *cfg;
    AR_CHECK_ARG(c.dim > 0 && c.hidden_dim > 0 && c.layer_count > 0 && c.vocab_size > 0 && c.seq_len > 0,
                 "Qwen3: sizes must be positive");
    AR_CHECK_ARG(c.head_count > 0 && c.kv_head_count > 0 && c.head_count % c.kv_head_count == 0,
                 "headCount (%d) must be divisible by kvHeadCount (%d)", c.head_count, c.kv_head_count);
    const int G = c.head_count / c.kv_head_count;
    AR_CHECK_ARG(G == 1 || G == 2 || G == 4 || G == 8, "Qwen3: heads per KV head %d not in {1,2,4,8}", G);
    AR_CHECK_ARG(c.head_size == 64 || c.head_size == 128, "Qwen3: head size %d not in {64,128}", c.head_size);
    AR_CHECK_ARG(c.max_batch >= 1 && c.max_batch <= 8, "Qwen3: batch %d outside 1..8", c.max_batch);
    AR_CHECK_ARG(c.weight_dtype == AR_DTYPE_F32 || c.weight_dtype == AR_DTYPE_BF16, "Qwen3: bad weight dtype");
    AR_CHECK_ARG(c.kv_dtype == AR_DTYPE_F32 || c.kv_dtype == AR_DTYPE_F16, "Qwen3: KV cache dtype %d not fp32 / fp16",
                 c.kv_dtype);
    AR_CHECK_ARG(c.qk_norm_mode == AR_QK_NORM_WHOLE || c.qk_norm_mode == AR_QK_NORM_PER_HEAD, "Qwen3: bad qk-norm mode");
    AR_CHECK_ARG(c.dim % 8 == 0 && c.hidden_dim % 8 == 0, "Qwen3: dim and hidden dim must be multiples of 8");
    auto* m = new ar_qwen3();
    m->ctx = ctx;
    m->cfg = c;
    m->q_dim = c.head_count * c.head_size;
    m->kv_dim = c.kv_head_count * c.head_size;
    m->qkv_dim = m->q_dim + 2 * m->kv_dim;
    m->B = c.max_batch;
    m->S = c.seq_len;
    m->wbytes = c.weight_dtype == AR_DTYPE_BF16 ? 2 : 4;
    m->kv_elem = c.kv_dtype == AR_DTYPE_F16 ? 2 : 4;
    m->layers.resize(c.layer_count);
    m->prompt_set.assign(m->B, 0);
    m->max_splits = attention_max_splits(m->S, c.kv_head_count, m->B, c.kv_dtype == AR_DTYPE_F16);

    // ---- weight arena: every tensor 256-byte aligned --------------------------------
    const size_t d = c.dim, F = c.hidden_dim, V = c.vocab_size, wb = m->wbytes;
    struct Pending { std::string key; size_t off; int64_t elems; bool matrix; bool required; };
    std::vector<Pending> plan;
    size_t off = 0;
    auto place = [&](const std::string& key, int64_t elems, bool matrix, bool required = true) {
        plan.push_back({key, off, elems, matrix, required});
        off = align_up(off + (size_t)elems * (matrix ? wb : 4), 256);
        return plan.back().off;
    };
    const size_t emb_off = place("model.embed_tokens.weight", (int64_t)(V * d), true);
    const size_t head_off = c.shared_weights ? emb_off : place("lm_head.weight", (int64_t)(V * d), true);
    const size_t fnorm_off = place("model.norm.weight", (int64_t)d, false);
    std::vector<size_t> lo(c.layer_count * 12);
    for (int l = 0; l < c.layer_count; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        size_t* o = &lo[l * 12];
        o[0] = place(p + "self_attn.qkv", (int64_t)m->qkv_dim * d, true);  // q|k|v rows, filled by 3 keys
        o[1] = place(p + "self_attn.o_proj.weight", (int64_t)d * m->q_dim, true);
        o[2] = place(p + "mlp.gate_proj.weight", (int64_t)F * d, true);
        o[3] = place(p + "mlp.up_proj.weight", (int64_t)F * d, true);
        o[4] = place(p + "mlp.down_proj.weight", (int64_t)d * F, true);
        o[5] = place(p + "input_layernorm.weight", (int64_t)d, false);
        o[6] = place(p + "post_attention_layernorm.weight", (int64_t)d, false);
        o[7] = place(p + "self_attn.q_norm.weight", m->q_dim, false, false);
        o[8] = place(p + "self_attn.k_norm.weight", m->kv_dim, false, false);
        o[9] = c.qkv_bias ? place(p + "self_attn.qkv_bias", m->qkv_dim, false) : (size_t)-1;
    }
    m->arena_bytes = off;
    int rc = ar_ctx_alloc(ctx, m->arena_bytes, (void**)&m->arena);
    if (rc != AR_HIP_OK) {
        delete m;
        return rc;
    }
    char* A = m->arena;
    m->embed = A + emb_off;
    m->lm_head = A + head_off;
    m->final_norm = (float*)(A + fnorm_off);
    for (auto& pd : plan) {
        if (pd.key.find(".self_attn.qkv") != std::string::npos) continue;  // split into q/k/v slots below
        add_slot(m, pd.key, A + pd.off, pd.elems, pd.matrix, pd.required);
    }
    if (c.shared_weights) add_slot(m, "lm_head.weight", nullptr, (int64_t)(V * d), true, false);
    for (int l = 0; l < c.layer_count; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        size_t* o = &lo[l * 12];
        Layer& L = m->layers[l];
        L.wqkv = A + o[0];
        L.wo = A + o[1];
        L.w1 = A + o[2];
        L.w3 = A + o[3];
        L.w2 = A + o[4];
        L.attn_norm = (float*)(A + o[5]);
        L.ffn_norm = (float*)(A + o[6]);
        L.q_norm = (float*)(A + o[7]);
        L.k_norm = (float*)(A + o[8]);
        char* qkv = (char*)L.wqkv;
        add_slot(m, p + "self_attn.q_proj.weight", qkv, (int64_t)m->q_dim * d, true);
        add_slot(m, p + "self_attn.k_proj.weight", qkv + (size_t)m->q_dim * d * wb, (int64_t)m->kv_dim * d, true);
        add_slot(m, p + "self_attn.v_proj.weight", qkv + (size_t)(m->q_dim + m->kv_dim) * d * wb,
                 (int64_t)m->kv_dim * d, true);
        if (c.qkv_bias) {
            L.bqkv = (float*)(A + o[9]);
            add_slot(m, p + "self_attn.q_proj.bias", L.bqkv, m->q_dim, false);
            add_slot(m, p + "self_attn.k_proj.bias", L.bqkv + m->q_dim, m->kv_dim, false);
            add_slot(m, p + "self_attn.v_proj.bias", L.bqkv + m->q_dim + m->kv_dim, m->kv_dim, false);
        }
    }

    // ---- activations, caches, loop state -------------------------------------------
    const size_t B = m->B;
    const size_t cache = (size_t)c.layer_count * B * c.kv_head_count * m->S * c.head_size;
    m->staging_floats = 16u << 20;
#define ALLOC(ptr, bytes)                                          \
    do {                                                           \
        int _r = alloc_zero(m, (bytes), (void**)&m->ptr);          \
        if (_r != AR_HIP_OK) { release(m); return _r; }            \
    } while (0)
    ALLOC(x, B * d * 4);
    ALLOC(qkv, B * m->qkv_dim * 4);
    ALLOC(attn, B * m->q_dim * 4);
    ALLOC(act, B * F * 4);
    ALLOC(logits, B * V * 4);
    ALLOC(kcache, cache * m->kv_elem);
    ALLOC(vcache, cache * m->kv_elem);
    ALLOC(part_o, attention_partial_floats(m->B, c.head_count, m->max_splits, c.head_size) * 4);
    ALLOC(part_ml, B * c.head_count * m->max_splits * 2 * 4);
    if (B >= 3 && c.weight_dtype == AR_DTYPE_BF16 && d % 32 == 0 && m->q_dim % 32 == 0 && F % 32 == 0) {
        ALLOC(pl_x, (size_t)2 * B * d * 2);
        ALLOC(pl_attn, (size_t)2 * B * m->q_dim * 2);
        ALLOC(pl_act, (size_t)2 * B * F * 2);
        size_t part = (size_t)((d + 15) / 16) * 4 * 256;  // up to 4 k-slices of every tile
        int counters = (d + 15) / 16;
        const int cus = ar_device_cus(m->ctx->stream);
        const bool frag = B <= 8 && gemv_frag_fits(d, m->q_dim, (int)B, cus) && gemv_frag_fits(F, d, (int)B, cus) &&
                          gemv_frag_fits(d, F, (int)B, cus) && d % 16 == 0;
        if (frag) {
            const size_t per_layer = gemv_frag_elems(d, m->q_dim) + 2 * gemv_frag_elems(F, d) + gemv_frag_elems(d, F);
            ALLOC(gv_frag, per_layer * c.layer_count * 2);
            ALLOC(gv_ss, (size_t)(d / 16) * 16 * 4);
            part = std::max({part, gemv_frag_part_floats(d, cus, 1), gemv_frag_part_floats(F, cus, 2)});
            counters = std::max({counters, (int)(F / 16)});
            uint16_t* f = m->gv_frag;
            for (int l = 0; l < c.layer_count; l++) {
                Layer& L = m->layers[l];
                L.fo = f; f += gemv_frag_elems(d, m->q_dim);
                L.f1 = f; f += gemv_frag_elems(F, d);
                L.f3 = f; f += gemv_frag_elems(F, d);
                L.f2 = f; f += gemv_frag_elems(d, F);
            }
        }
        m->gv_part_floats = (int)part;
        m->gv_count_n = counters;
        ALLOC(gv_part, part * 4);
        ALLOC(gv_count, (size_t)counters * 4);
    }
    ALLOC(am_keys, B * kArgmaxSlots * 8);
    ALLOC(smp_rng, B * 8);
    ALLOC(smp_rng_saved, B * 8);
    {
        // every sequence starts with new Random(0)
        std::vector<unsigned long long> st0(B, 0x5DEECE66DULL & ((1ULL << 48) - 1));
        hipError_t e = hipMemcpyAsync(m->smp_rng, st0.data(), (size_t)B * 8, hipMemcpyHostToDevice, m->ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->ctx->stream);
        if (e != hipSuccess) {
            release(m);
            ar_set_error("hipMemcpy: %s", hipGetErrorString(e));
            return AR_HIP_ERR_HIP;
        }
    }
    ALLOC(rope_tab, (size_t)m->S * (c.head_size / 2) * sizeof(float2));
    ALLOC(tokens, B * (m->S + 1) * 4);
    ALLOC(state, 64);
    ALLOC(staging, m->staging_floats * 4);
#undef ALLOC
    {
        // RoPE (cos, sin) for every cache position, in double as computeRopeFreqs defines them
        // (engine/ml/.../RotationFeatures.java:189-208): invf[f] = exp(f * -2 ln(theta) / hd).
        const int fd = c.head_size / 2;
        std::vector<float2> tab((size_t)m->S * fd);
        const double cexp = -2.0 * std::log(c.rope_theta) / (double)c.head_size;
        for (int pos = 0; pos < m->S; pos++)
            for (int f = 0; f < fd; f++) {
                const double ang = (double)pos * std::exp((double)f * cexp);
                tab[(size_t)pos * fd + f] = make_float2((float)std::cos(ang), (float)std::sin(ang));
            }
        if (hipMemcpyAsync(m->rope_tab, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice,
                           ctx->stream) != hipSuccess) {
            release(m);
            ar_set_error("RoPE table upload failed");
            return AR_HIP_ERR_HIP;
        }
    }
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) {
        release(m);
        ar_set_error("stream synchronize after allocation failed");
        return AR_HIP_ERR_HIP;
    }
    *out = m;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_destroy(ar_qwen3* m) {
    if (!m) return AR_HIP_OK;
    hipStreamSynchronize(m->ctx->stream);
    release(m);
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_set_weight(ar_qwen3* m, const char* key, const void* src, int src_dtype, int64_t n) {
    AR_CHECK_ARG(m && key && src, "null argument");
    if (!strcmp(key, AR_ROPE_TABLE_KEY)) {
        // a given (cos, sin) table replaces the one computed from rope_theta, as a model built with
        // a freqCis producer uses it (Llama2.java model(), Llama2Weights.freqCis): rows for
        // positions 0.., (head_size / 2) pairs each; the first seq_len rows are used
        const int64_t per_pos = m->cfg.head_size;  // head_size / 2 pairs of two values
        AR_CHECK_ARG(src_dtype == AR_DTYPE_F32, "%s: fp32 values expected", key);
        AR_CHECK_ARG(n % per_pos == 0 && n / per_pos >= m->S, "%s: %lld values do not hold %d positions x %lld",
                     key, (long long)n, m->S, (long long)per_pos);
        AR_HIP_TRY(hipMemcpyAsync(m->rope_tab, src, (size_t)m->S * per_pos * sizeof(float), hipMemcpyHostToDevice,
                                  m->ctx->stream));
        AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
        return AR_HIP_OK;
    }
    auto it = m->slots.find(key);
    if (it == m->slots.end()) {
        ar_set_error("unknown weight key '%s'", key);
        return AR_HIP_ERR_NOT_FOUND;
    }
    Slot& s = it->second;
    if (!s.dst) return AR_HIP_OK;  // lm_head.weight with tied embeddings: the embedding is the head
    AR_CHECK_ARG(n == s.elems, "weight '%s': %lld elements given, %lld expected", key, (long long)n,
                 (long long)s.elems);
    AR_TRY(upload(m, s, src, src_dtype, n));
    s.filled = true;
    m->finalized = false;
    m->pf_w16_valid = false;
    return AR_HIP_OK;
}

// Decides whether the persistent decode kernel can run this model's step and, the first time it can,
// allocates its exchange words, error flag and layer table; the table is rewritten on every finalize.
static int setup_persistent(ar_qwen3* m) {
    const ar_qwen3_cfg& c = m->cfg;
    m->pk_ok = false;
    if (m->B != 1) return AR_HIP_OK;
    if (!decode_persistent_supported(c.weight_dtype, c.dim, c.hidden_dim, c.head_count, c.kv_head_count, c.head_size,
                                     c.kv_dtype == AR_DTYPE_F16))
        return AR_HIP_OK;
    const size_t eb = decode_persistent_layer_bytes();
    if (!m->pk_ll) {
        const size_t words =
            decode_persistent_ll_words(c.weight_dtype, c.dim, c.hidden_dim, c.head_count, c.kv_head_count, c.head_size);
        // exchange words in uncached memory: C3 0.630 -> 0.606 ms per step against cached memory
        AR_TRY(ar_uncached_get(m->ctx->device, words * 8, (void**)&m->pk_ll));
        m->pk_ll_words = words;
        AR_HIP_TRY(hipMemsetAsync(m->pk_ll, 0, words * 8, m->ctx->stream));
        AR_TRY(alloc_zero(m, 64, (void**)&m->pk_err));
        AR_TRY(alloc_zero(m, eb * c.layer_count, &m->pk_layers));
    }
    std::vector<char> tab(eb * c.layer_count);
    for (int l = 0; l < c.layer_count; l++) {
        const Layer& L = m->layers[l];
        AR_TRY(decode_persistent_layer_entry(tab.data() + l * eb, L.wqkv, L.wo, L.w1, L.w3, L.w2, L.attn_norm,
                                             L.ffn_norm, L.q_norm, L.k_norm, L.bqkv));
    }
    AR_HIP_TRY(hipMemcpyAsync(m->pk_layers, tab.data(), tab.size(), hipMemcpyHostToDevice, m->ctx->stream));
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    m->pk_ok = true;
    return AR_HIP_OK;
}

// After a synchronisation: the persistent kernel's error flag of the launches since the last check
// (0 none, 1 a cross-block wait timed out, 2 position outside the cache), cleared.
static int persistent_status(ar_qwen3* m, int* status) {
    *status = 0;
    if (!m->pk_err) return AR_HIP_OK;
    AR_HIP_TRY(hipMemcpy(status, m->pk_err, sizeof(int), hipMemcpyDeviceToHost));
    if (*status) AR_HIP_TRY(hipMemset(m->pk_err, 0, sizeof(int)));
    return AR_HIP_OK;
}

// A persistent launch needs every block resident at once; when another kernel or process holds CUs,
// the blocks that did run abandon their waits after the wait limit and the launch drains with invalid
// results.  The steps [start, start + n) of the call are then recomputed as separate launches before
// the call returns, and the model stays on separate launches until use_persistent(1):
//  * the exchange words are cleared: a block that started after block 0 had published the next
//    launch's epoch base wrote words tagged with that launch's epochs;
//  * the generators of a sampling model are restored to their state before the call (the sampler ran
//    on the invalid logits);
//  * the loop state returns to position start.  The token fed at start was stored by the call's first
//    step-begin, from the keys of the last valid step, so the recompute reads it as a prompt token (the
//    prompt length seen by the step-begin is max(prompt_len, start + 1) during the recompute; every
//    later step decides prompt / generated exactly as before), and the prompt length is restored after.
static int recompute_timed_out(ar_qwen3* m, int start, int n, bool store_logits) {
    hipStream_t st = m->ctx->stream;
    AR_HIP_TRY(hipStreamSynchronize(st));
    AR_HIP_TRY(hipMemsetAsync(m->pk_ll, 0, m->pk_ll_words * 8, st));
    if (!sample_is_greedy(m->smp_mode, m->smp_temperature))
        AR_HIP_TRY(hipMemcpyAsync(m->smp_rng, m->smp_rng_saved, (size_t)m->B * 8, hipMemcpyDeviceToDevice, st));
    const int loop[3] = {start, std::max(m->prompt_len, start + 1), start};
    AR_HIP_TRY(hipMemcpyAsync(m->state, loop, sizeof(loop), hipMemcpyHostToDevice, st));
    m->pk_suspended = true;
    int rc = AR_HIP_OK;
    for (int i = 0; i < n && rc == AR_HIP_OK; i++) rc = run_step(m, store_logits);
    m->pk_suspended = false;
    AR_TRY(rc);
    AR_HIP_TRY(hipMemcpyAsync(m->state + 1, &m->prompt_len, sizeof(int), hipMemcpyHostToDevice, st));
    AR_HIP_TRY(hipStreamSynchronize(st));
    m->pk_on = false;
    m->pk_recomputed += n;
    ar_log("persistent decode step timed out (blocks not resident together); %d step(s) from position %d "
           "recomputed as separate launches, the model now runs separate launches", n, start);
    return AR_HIP_OK;
}

// Before a call that enqueues persistent steps of a sampling model: the generators' state, so a
// recompute draws what the steps would have drawn.
static int save_generators(ar_qwen3* m) {
    if (persistent_active(m) && !sample_is_greedy(m->smp_mode, m->smp_temperature))
        AR_HIP_TRY(hipMemcpyAsync(m->smp_rng_saved, m->smp_rng, (size_t)m->B * 8, hipMemcpyDeviceToDevice,
                                  m->ctx->stream));
    return AR_HIP_OK;
}

// After the synchronisation that ends a call of n steps from position start: a timed-out persistent
// step is recomputed (returns 1 in *redone, the outputs must be copied again), a position outside the
// cache (the host never steps there) is an error.
static int finish_persistent(ar_qwen3* m, int start, int n, bool store_logits, int* redone) {
    *redone = 0;
    int status = 0;
    AR_TRY(persistent_status(m, &status));
    if (status == 2) {
        ar_set_error("persistent decode step: position outside the KV cache");
        return AR_HIP_ERR_HIP;
    }
    if (status == 1) {
        AR_TRY(recompute_timed_out(m, start, n, store_logits));
        *redone = 1;
    }
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_finalize(ar_qwen3* m) {
    AR_CHECK_ARG(m, "null model");
    for (auto& kv : m->slots) {
        if (kv.second.dst && kv.second.required && !kv.second.filled) {
            ar_set_error("weight '%s' was never set", kv.first.c_str());
            return AR_HIP_ERR_STATE;
        }
    }
    // QK-norm gains are optional (Qwen3.java:378-379, AttentionFeatures.java:839,885): a gain that
    // was never set means that norm is skipped.
    for (int l = 0; l < m->cfg.layer_count; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        Layer& L = m->layers[l];
        const Slot& qs = m->slots[p + "self_attn.q_norm.weight"];
        const Slot& ks = m->slots[p + "self_attn.k_norm.weight"];
        L.q_norm = qs.filled ? (float*)qs.dst : nullptr;
        L.k_norm = ks.filled ? (float*)ks.dst : nullptr;
    }
    AR_TRY(invalidate_graphs(m));
    AR_TRY(setup_persistent(m));
    if (m->gv_frag) {  // fragment-ordered copies of the layers' projections
        const ar_qwen3_cfg& c = m->cfg;
        const int d = c.dim, F = c.hidden_dim;
        hipStream_t st = m->ctx->stream;
        for (const Layer& L : m->layers) {
            AR_TRY(launch_frag_copy((const uint16_t*)L.wo, L.fo, d, m->q_dim, st));
            AR_TRY(launch_frag_copy((const uint16_t*)L.w1, L.f1, F, d, st));
            AR_TRY(launch_frag_copy((const uint16_t*)L.w3, L.f3, F, d, st));
            AR_TRY(launch_frag_copy((const uint16_t*)L.w2, L.f2, d, F, st));
        }
        AR_HIP_TRY(hipStreamSynchronize(st));
    }
    m->finalized = true;
    return ar_hip_qwen3_reset(m);
}

extern "C" int ar_hip_qwen3_reset(ar_qwen3* m) {
    AR_CHECK_ARG(m, "null model");
    m->host_pos = 0;
    m->needs_reset = false;
    int st[3] = {0, m->prompt_len, 0};
    AR_HIP_TRY(hipMemcpyAsync(m->state, st, sizeof(st), hipMemcpyHostToDevice, m->ctx->stream));
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_set_prompt(ar_qwen3* m, int seq, const int32_t* ids, int n) {
    AR_CHECK_ARG(m && (ids || n == 0), "null argument");
    AR_CHECK_ARG(seq >= 0 && seq < m->B, "sequence %d outside batch of %d", seq, m->B);
    AR_CHECK_ARG(n >= 0 && n <= m->S, "prompt of %d tokens exceeds the %d-position cache", n, m->S);
    for (int i = 0; i < n; i++)
        AR_CHECK_ARG(ids[i] >= 0 && ids[i] < m->cfg.vocab_size, "prompt token %d at %d outside vocab", ids[i], i);
    // All sequences of a batch share one prompt length.  A prompt of another length replaces the
    // batch's length: the other sequences' prompts are dropped and must be set again (at the new
    // length) before the next step, which check_ready enforces.  setPrompt itself accepts any
    // length at any time (AutoregressiveModel.java:272-275).
    if (n != m->prompt_len)
        for (int b = 0; b < m->B; b++)
            if (b != seq) m->prompt_set[b] = 0;
    if (n > 0)
        AR_HIP_TRY(hipMemcpyAsync(m->tokens + (size_t)seq * (m->S + 1), ids, (size_t)n * 4, hipMemcpyHostToDevice,
                                  m->ctx->stream));
    m->prompt_len = n;
    m->prompt_set[seq] = 1;
    AR_HIP_TRY(hipMemcpyAsync(m->state + 1, &m->prompt_len, sizeof(int), hipMemcpyHostToDevice, m->ctx->stream));
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    return AR_HIP_OK;
}

static int check_ready(ar_qwen3* m, int steps) {
    AR_CHECK_ARG(m, "null model");
    if (!m->finalized) {
        ar_set_error("model not finalized (call ar_hip_qwen3_finalize after setting weights)");
        return AR_HIP_ERR_STATE;
    }
    if (m->needs_reset) {
        ar_set_error("the kernel-loop probe overwrote the step state: reset() before the next step");
        return AR_HIP_ERR_STATE;
    }
    if (m->prompt_len < 1) {
        ar_set_error("no prompt: set at least one prompt token before stepping");
        return AR_HIP_ERR_STATE;
    }
    for (int b = 0; b < m->B; b++)
        if (!m->prompt_set[b]) {
            ar_set_error("sequence %d has no prompt", b);
            return AR_HIP_ERR_STATE;
        }
    if (m->host_pos + steps > m->S) {
        ar_set_error("position %d + %d steps exceeds the %d-position KV cache", m->host_pos, steps, m->S);
        return AR_HIP_ERR_STATE;
    }
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_next(ar_qwen3* m, int32_t* tokens_out, float* logits_out) {
    AR_TRY(check_ready(m, 1));
    hipStream_t st = m->ctx->stream;
    AR_TRY(save_generators(m));
    AR_TRY(run_step(m, logits_out != nullptr));
    for (int pass = 0; pass < 2; pass++) {
        if (tokens_out)
            for (int b = 0; b < m->B; b++)
                AR_HIP_TRY(hipMemcpyAsync(tokens_out + b, m->tokens + (size_t)b * (m->S + 1) + m->host_pos, 4,
                                          hipMemcpyDeviceToHost, st));
        if (logits_out)
            AR_HIP_TRY(hipMemcpyAsync(logits_out, m->logits, (size_t)m->B * m->cfg.vocab_size * 4,
                                      hipMemcpyDeviceToHost, st));
        AR_HIP_TRY(hipStreamSynchronize(st));
        int redone = 0;
        if (pass == 0) AR_TRY(finish_persistent(m, m->host_pos, 1, logits_out != nullptr, &redone));
        if (!redone) break;
    }
    m->host_pos++;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_run(ar_qwen3* m, int steps, int32_t* tokens_out) {
    AR_CHECK_ARG(steps >= 0, "negative step count");
    AR_TRY(check_ready(m, steps));
    hipStream_t st = m->ctx->stream;
    const int start = m->host_pos;
    AR_TRY(save_generators(m));
    for (int i = 0; i < steps; i++) AR_TRY(run_step(m, false));
    for (int pass = 0; pass < 2; pass++) {
        if (tokens_out && steps > 0)
            for (int b = 0; b < m->B; b++)
                AR_HIP_TRY(hipMemcpyAsync(tokens_out + (size_t)b * steps, m->tokens + (size_t)b * (m->S + 1) + start,
                                          (size_t)steps * 4, hipMemcpyDeviceToHost, st));
        AR_HIP_TRY(hipStreamSynchronize(st));
        int redone = 0;
        if (pass == 0) AR_TRY(finish_persistent(m, start, steps, false, &redone));
        if (!redone) break;
    }
    m->host_pos += steps;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_prefill_by_steps(ar_qwen3* m, int* count) {
    AR_CHECK_ARG(m && count, "null argument");
    *count = m->pf_by_steps;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_position(ar_qwen3* m, int* pos) {
    AR_CHECK_ARG(m && pos, "null argument");
    *pos = m->host_pos;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_hidden(ar_qwen3* m, float* out) {
    AR_CHECK_ARG(m && out, "null argument");
    AR_HIP_TRY(hipMemcpyAsync(out, m->x, (size_t)m->B * m->cfg.dim * 4, hipMemcpyDeviceToHost, m->ctx->stream));
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_kernel_timing(ar_qwen3* m, int which) {
    AR_CHECK_ARG(m, "null model");
    AR_CHECK_ARG(which >= AR_KT_NONE && which <= AR_KT_LAYERS, "unknown kernel class %d", which);
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    m->timed = which;
    m->events_used = 0;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_kernel_time(ar_qwen3* m, double* ms, int* launches) {
    AR_CHECK_ARG(m && ms && launches, "null argument");
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    double t = 0.0;
    for (size_t i = 0; i < m->events_used; i++) {
        float e = 0.f;
        AR_HIP_TRY(hipEventElapsedTime(&e, m->events[i].first, m->events[i].second));
        t += e;
    }
    *ms = t;
    *launches = (int)m->events_used;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_kernel_loop(ar_qwen3* m, int which, int reps, double* us_per_launch) {
    AR_CHECK_ARG(m && us_per_launch, "null argument");
    if (!m->finalized) {
        ar_set_error("model not finalized (call ar_hip_qwen3_finalize after setting weights)");
        return AR_HIP_ERR_STATE;
    }
    AR_CHECK_ARG(which == AR_KT_QKV || which == AR_KT_O || which == AR_KT_GATE_UP || which == AR_KT_DOWN ||
                     which == AR_KT_LOGITS,
                 "kernel class %d has no loop probe (the attention class writes KV-cache rows)", which);
    AR_CHECK_ARG(reps >= 1 && reps <= 4096, "reps %d outside 1..4096", reps);
    hipStream_t st = m->ctx->stream;
    AR_HIP_TRY(hipStreamSynchronize(st));
    m->needs_reset = true;  // the launches overwrite the residual stream and the greedy keys
    const StepPlanes pl = step_planes(m);
    if (!m->use_graph) {  // plain launches, back to back between the two events
        hipEvent_t e0 = nullptr, e1 = nullptr;
        AR_HIP_TRY(hipEventCreate(&e0));
        hipError_t e = hipEventCreate(&e1);
        int rc = AR_HIP_OK;
        for (int i = 0; i < 2 && rc == AR_HIP_OK; i++)  // (pass 0 warms the launch path)
            rc = launch_class(m, which, 0, pl, false);
        if (e == hipSuccess && rc == AR_HIP_OK) e = hipEventRecord(e0, st);
        for (int i = 0; i < reps && e == hipSuccess && rc == AR_HIP_OK; i++)
            rc = launch_class(m, which, i % m->cfg.layer_count, pl, false);
        if (e == hipSuccess && rc == AR_HIP_OK) e = hipEventRecord(e1, st);
        if (e == hipSuccess && rc == AR_HIP_OK) e = hipEventSynchronize(e1);
        float ms = 0.f;
        if (e == hipSuccess && rc == AR_HIP_OK) e = hipEventElapsedTime(&ms, e0, e1);
        (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (rc != AR_HIP_OK) return rc;
        if (e != hipSuccess) {
            ar_set_error("kernel loop: %s", hipGetErrorString(e));
            return AR_HIP_ERR_HIP;
        }
        *us_per_launch = 1000.0 * (double)ms / reps;
        return AR_HIP_OK;
    }
    hipGraph_t g = nullptr;
    AR_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int rc = AR_HIP_OK;
    for (int i = 0; i < reps && rc == AR_HIP_OK; i++) rc = launch_class(m, which, i % m->cfg.layer_count, pl, false);
    const hipError_t ce = hipStreamEndCapture(st, &g);
    if (rc != AR_HIP_OK || ce != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        if (rc != AR_HIP_OK) return rc;
        ar_set_error("hipStreamEndCapture: %s", hipGetErrorString(ce));
        return AR_HIP_ERR_HIP;
    }
    hipGraphExec_t ex = nullptr;
    const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ie != hipSuccess) {
        ar_set_error("hipGraphInstantiate: %s", hipGetErrorString(ie));
        return AR_HIP_ERR_HIP;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipGraphLaunch(ex, st);  // warm (first replay uploads the graph)
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    if (e == hipSuccess) e = hipGraphLaunch(ex, st);
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipGraphExecDestroy(ex);
    if (e != hipSuccess) {
        ar_set_error("kernel loop: %s", hipGetErrorString(e));
        return AR_HIP_ERR_HIP;
    }
    *us_per_launch = 1000.0 * (double)ms / reps;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_use_graph(ar_qwen3* m, int enable) {
    AR_CHECK_ARG(m, "null model");
    m->use_graph = enable != 0;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_set_sampling(ar_qwen3* m, int mode, double temperature, double top_p,
                                         const int64_t* seeds) {
    AR_CHECK_ARG(m, "null model");
    AR_CHECK_ARG(mode == AR_SAMPLE_MODEL || mode == AR_SAMPLE_TOKEN, "unknown sampling mode %d", mode);
    AR_CHECK_ARG(temperature == temperature && top_p == top_p, "temperature and top_p must not be NaN");
    hipStream_t st = m->ctx->stream;
    AR_HIP_TRY(hipStreamSynchronize(st));
    if (seeds) {
        std::vector<unsigned long long> states(m->B);
        for (int b = 0; b < m->B; b++)  // new Random(seed): (seed ^ 0x5DEECE66D) mod 2^48
            states[b] = ((unsigned long long)seeds[b] ^ 0x5DEECE66DULL) & ((1ULL << 48) - 1);
        AR_HIP_TRY(hipMemcpyAsync(m->smp_rng, states.data(), states.size() * 8, hipMemcpyHostToDevice, st));
        AR_HIP_TRY(hipStreamSynchronize(st));
    }
    if (!sample_is_greedy(mode, temperature) && !m->smp_work) {
        AR_TRY(ar_ctx_alloc(m->ctx, sample_workspace_bytes(m->B, m->cfg.vocab_size), &m->smp_work));
        AR_TRY(sample_workspace_clear(m->smp_work, m->B, m->cfg.vocab_size, st));
    }
    if (mode != m->smp_mode || temperature != m->smp_temperature || top_p != m->smp_top_p)
        AR_TRY(invalidate_graphs(m));  // the captured step holds the sampler's launches and arguments
    m->smp_mode = mode;
    m->smp_temperature = temperature;
    m->smp_top_p = top_p;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_use_fragment_gemv(ar_qwen3* m, int enable) {
    AR_CHECK_ARG(m, "null model");
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    if (m->frag_on != (enable != 0)) AR_TRY(invalidate_graphs(m));  // the captured step holds either form
    m->frag_on = enable != 0;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_fragment_gemv(ar_qwen3* m, int* active) {
    AR_CHECK_ARG(m && active, "null argument");
    *active = frag_active(m) ? 1 : 0;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_use_persistent(ar_qwen3* m, int enable) {
    AR_CHECK_ARG(m, "null model");
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    if (m->pk_on != (enable != 0)) AR_TRY(invalidate_graphs(m));  // the captured step holds either form
    m->pk_on = enable != 0;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_prefill_gemm(ar_qwen3* m, int backend) {
    AR_CHECK_ARG(m, "null model");
    AR_CHECK_ARG(backend == AR_PREFILL_GEMM_OWN || backend == AR_PREFILL_GEMM_ROCBLAS,
                 "prefill GEMM backend %d is not AR_PREFILL_GEMM_OWN or AR_PREFILL_GEMM_ROCBLAS", backend);
    m->pf_gemm = backend;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_prefill_gemm_backend(ar_qwen3* m, int* backend) {
    AR_CHECK_ARG(m && backend, "null argument");
    *backend = m->pf_gemm;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_persistent(ar_qwen3* m, int* active) {
    AR_CHECK_ARG(m && active, "null argument");
    *active = persistent_active(m) ? 1 : 0;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_persistent_wait_limit(ar_qwen3* m, unsigned polls) {
    AR_CHECK_ARG(m, "null model");
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    m->pk_wait_limit = polls;
    return AR_HIP_OK;
}

extern "C" int ar_hip_qwen3_persistent_recomputed(ar_qwen3* m, int* steps) {
    AR_CHECK_ARG(m && steps, "null argument");
    *steps = m->pk_recomputed;
    return AR_HIP_OK;
}

namespace {

// k-slices for a prefill projection of N outputs over K inputs whose 128 x 128 output tiles would
// not give every CU two blocks (C4's d = 2048 projections): more blocks, same weights read
constexpr int kMaxKSplit = 4;
int prefill_ksplit(const ar_qwen3* m, size_t rows, int N, int K) {
    const long long tiles = (long long)((rows + 127) / 128) * (N / 128);
    int s = 1;
    while (s < kMaxKSplit && tiles * s < 2LL * m->ctx->num_cus && K % (64 * s * 2) == 0 && K / (s * 2) >= 512) s *= 2;
    return s;
}

int ensure_prefill_buffers(ar_qwen3* m, size_t rows) {
    if (!m->pf_flag) AR_TRY(alloc_zero(m, 2 * sizeof(int), (void**)&m->pf_flag));
    if (m->pf_rows >= rows) return AR_HIP_OK;
    void** bufs[] = {(void**)&m->pf_x, (void**)&m->pf_h, (void**)&m->pf_qkv, (void**)&m->pf_q, (void**)&m->pf_act};
    for (void** b : bufs)
        if (*b) {
            AR_TRY(ar_ctx_free(m->ctx, *b));
            *b = nullptr;
        }
    m->pf_rows = 0;
    const ar_qwen3_cfg& c = m->cfg;
    const size_t hw = (size_t)std::max(c.dim, m->q_dim);
    if (c.weight_dtype == AR_DTYPE_F32) {
        // fp32 path: GEMM input rows (normalised x / attention output), queries and SwiGLU output in fp32
        AR_TRY(ar_ctx_alloc(m->ctx, rows * c.dim * 4, (void**)&m->pf_x));
        AR_TRY(ar_ctx_alloc(m->ctx, rows * hw * 4, (void**)&m->pf_h));
        AR_TRY(ar_ctx_alloc(m->ctx, rows * m->qkv_dim * 4, (void**)&m->pf_qkv));
        AR_TRY(ar_ctx_alloc(m->ctx, rows * m->q_dim * 4, (void**)&m->pf_q));
        AR_TRY(ar_ctx_alloc(m->ctx, rows * c.hidden_dim * 4, (void**)&m->pf_act));
        m->pf_rows = rows;
        return AR_HIP_OK;
    }
    AR_TRY(ar_ctx_alloc(m->ctx, rows * c.dim * 4, (void**)&m->pf_x));
    AR_TRY(ar_ctx_alloc(m->ctx, rows * hw * 2, (void**)&m->pf_h));
    AR_TRY(ar_ctx_alloc(m->ctx, rows * m->qkv_dim * 4, (void**)&m->pf_qkv));
    AR_TRY(ar_ctx_alloc(m->ctx, rows * m->q_dim * 2, (void**)&m->pf_q));
    AR_TRY(ar_ctx_alloc(m->ctx, rows * c.hidden_dim * 2, (void**)&m->pf_act));
    m->pf_rows = rows;
    if (!m->pf_k16) {
        m->pf_tp = (m->S + 127) / 128 * 128;  // a multiple of every flash super-tile
        const size_t n = (size_t)m->B * c.kv_head_count * m->pf_tp * c.head_size * 2;
        AR_TRY(ar_ctx_alloc(m->ctx, n, (void**)&m->pf_k16));
        AR_TRY(ar_ctx_alloc(m->ctx, n, (void**)&m->pf_vt16));
        AR_HIP_TRY(hipMemsetAsync(m->pf_k16, 0, n, m->ctx->stream));
        AR_HIP_TRY(hipMemsetAsync(m->pf_vt16, 0, n, m->ctx->stream));
    }
    return AR_HIP_OK;
}

// fp16 copy of a layer's projection matrices, in the same order as the arena: qkv, o, gate, up, down.
int ensure_f16_weights(ar_qwen3* m) {
    if (m->pf_w16_valid) return AR_HIP_OK;
    const ar_qwen3_cfg& c = m->cfg;
    const size_t d = c.dim, F = c.hidden_dim;
    const size_t per_layer = (size_t)m->qkv_dim * d + d * m->q_dim + 3 * F * d;
    if (!m->pf_w16) AR_TRY(ar_ctx_alloc(m->ctx, per_layer * c.layer_count * 2, (void**)&m->pf_w16));
    AR_HIP_TRY(hipMemsetAsync(m->pf_flag + 1, 0, sizeof(int), m->ctx->stream));
    uint16_t* dst = m->pf_w16;
    for (int l = 0; l < c.layer_count; l++) {
        const Layer& L = m->layers[l];
        const void* srcs[5] = {L.wqkv, L.wo, L.w1, L.w3, L.w2};
        const size_t counts[5] = {(size_t)m->qkv_dim * d, d * m->q_dim, F * d, F * d, d * F};
        for (int i = 0; i < 5; i++) {
            AR_TRY(launch_bf16_to_f16((const uint16_t*)srcs[i], dst, counts[i], m->pf_flag + 1, m->ctx->stream));
            dst += counts[i];
        }
    }
    int overflow = 0;
    AR_HIP_TRY(hipMemcpyAsync(&overflow, m->pf_flag + 1, sizeof(int), hipMemcpyDeviceToHost, m->ctx->stream));
    AR_HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    m->pf_w16_in_range = overflow == 0;  // a weight past the fp16 range: every prefill takes the decode step
    m->pf_w16_valid = true;
    return AR_HIP_OK;
}

}  // namespace

// The prompt through the decode step, one token per step (the reference's own prefill), from
// position 0: prompt_len calls of next() leave the model where a batched prefill does.
static int prefill_by_steps(ar_qwen3* m, int T, float* logits_out) {
    m->pf_by_steps++;
    AR_TRY(ar_hip_qwen3_reset(m));
    if (T > 1) AR_TRY(ar_hip_qwen3_run(m, T - 1, nullptr));
    return ar_hip_qwen3_next(m, nullptr, logits_out);
}

// The end of a batched prefill: the last prompt row of every sequence (the residual stream plus the
// `pending` k-slices of the last residual projection) becomes the decode plan's residual stream, the
// final RMSNorm + logits GEMV leaves the greedy keys for the next step, and the loop state moves to
// where prompt_len calls of next() leave it.
static int prefill_finish(ar_qwen3* m, int T, int pending, float* logits_out) {
    const ar_qwen3_cfg& c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int B = m->B, d = c.dim;
    const size_t R = (size_t)B * T;
    AR_TRY(launch_fold_rows(m->pf_x, m->pf_part, pending, R, T - 1, T, B, d, m->x, st));
    AR_HIP_TRY(hipMemsetAsync(m->am_keys, 0, (size_t)B * kArgmaxSlots * 8, st));
    GemvLaunch h;
    h.wdtype = c.weight_dtype; h.batch = B; h.eps = (float)c.epsilon; h.w = m->lm_head; h.rows = c.vocab_size;
    const bool sampling = !sample_is_greedy(m->smp_mode, m->smp_temperature);
    h.cols = d; h.x = m->x; h.x_stride = d; h.norm_w = m->final_norm;
    h.y = (logits_out || sampling) ? m->logits : nullptr;
    h.y_stride = c.vocab_size; h.epilogue = GEMV_EPI_ARGMAX; h.keys = m->am_keys;
    AR_TRY(launch_gemv(h, st));
    const int state[3] = {T - 1, T, T};
    AR_HIP_TRY(hipMemcpyAsync(m->state, state, sizeof(state), hipMemcpyHostToDevice, st));
    if (sampling) AR_TRY(enqueue_sample(m));  // the first generated token
    if (logits_out)
        AR_HIP_TRY(hipMemcpyAsync(logits_out, m->logits, (size_t)B * c.vocab_size * 4, hipMemcpyDeviceToHost, st));
    AR_HIP_TRY(hipStreamSynchronize(st));
    m->host_pos = T;
    return AR_HIP_OK;
}

// k-split of an fp32 residual projection (at most kMaxKSplit slices, consumed by the fold kernels)
static int prefill_f32_ksplit(const ar_qwen3* m, size_t rows, int N, int K) {
    return std::min(kMaxKSplit, gemm_f32_ksplit((int)rows, N, K, m->ctx->num_cus));
}

// fp32 weights: the prompt rows as fp32 MFMA GEMMs (gemm_f32.hip) with the decode path's RMSNorm,
// QK-norm, RoPE and cache write, and fp32 causal attention over the cache rows.
static int prefill_f32(ar_qwen3* m, int T, float* logits_out) {
    const ar_qwen3_cfg& c = m->cfg;
    hipStream_t st = m->ctx->stream;
    const int B = m->B, d = c.dim, F = c.hidden_dim, qd = m->q_dim;
    const size_t R = (size_t)B * T;
    AR_CHECK_ARG(R <= (size_t)INT32_MAX / 16, "prefill: %zu rows too many", R);
    AR_TRY(ensure_prefill_buffers(m, R));
    float* const h32 = reinterpret_cast<float*>(m->pf_h);
    float* const q32 = reinterpret_cast<float*>(m->pf_q);
    float* const act32 = reinterpret_cast<float*>(m->pf_act);
    AR_TRY(launch_embed_rows(m->embed, c.weight_dtype, d, m->tokens, m->S + 1, T, (int)R, m->pf_x, st));
    const size_t layer_cache = (size_t)B * c.kv_head_count * m->S * c.head_size;
    const int so = prefill_f32_ksplit(m, R, d, qd), sd = prefill_f32_ksplit(m, R, d, F);
    if ((so > 1 || sd > 1) && m->pf_part_rows < R) {
        if (m->pf_part) AR_TRY(ar_ctx_free(m->ctx, m->pf_part));
        m->pf_part = nullptr;
        m->pf_part_rows = 0;
        AR_TRY(ar_ctx_alloc(m->ctx, (size_t)kMaxKSplit * R * d * 4, (void**)&m->pf_part));
        m->pf_part_rows = R;
    }
    int pending = 0;
    for (int l = 0; l < c.layer_count; l++) {
        const Layer& L = m->layers[l];
        AR_TRY(launch_fold_rmsnorm_rows_f32(m->pf_x, m->pf_part, pending, L.attn_norm, h32, (int)R, d,
                                            (float)c.epsilon, st));
        pending = 0;
        GemmF32Launch g;
        g.A = h32; g.lda = d; g.W = (const float*)L.wqkv; g.ldw = d; g.M = (int)R; g.N = m->qkv_dim; g.K = d;
        g.bias = L.bqkv; g.C = m->pf_qkv; g.ldc = m->qkv_dim; g.epilogue = GEMV_EPI_STORE;
        AR_TRY(launch_gemm_f32(g, st));
        PrefillPrep pp;
        pp.qkv = m->pf_qkv; pp.qkv_stride = m->qkv_dim; pp.q_norm = L.q_norm; pp.k_norm = L.k_norm;
        pp.eps = (float)c.epsilon; pp.per_head = c.qk_norm_mode == AR_QK_NORM_PER_HEAD; pp.rope_tab = m->rope_tab;
        pp.kcache = (char*)m->kcache + l * layer_cache * m->kv_elem;
        pp.vcache = (char*)m->vcache + l * layer_cache * m->kv_elem;
        pp.B = B; pp.S = m->S; pp.T = T; pp.p0 = 0; pp.heads = c.head_count; pp.kv_heads = c.kv_head_count;
        pp.hd = c.head_size; pp.q32 = q32;
        AR_TRY(launch_qk_prep(pp, st));
        AR_TRY(launch_attention_prefill_f32(q32, (const float*)pp.kcache, (const float*)pp.vcache, h32, B, T, 0, m->S,
                                            c.head_count, c.kv_head_count, c.head_size, st));
        GemmF32Launch o;
        o.A = h32; o.lda = qd; o.W = (const float*)L.wo; o.ldw = qd; o.M = (int)R; o.N = d; o.K = qd;
        o.C = m->pf_x; o.ldc = d; o.epilogue = GEMV_EPI_RESIDUAL;
        if (so > 1) {  // k-slices into pf_part, added into pf_x by the next row RMSNorm
            o.C = m->pf_part; o.epilogue = GEMV_EPI_STORE; o.ksplit = so;
        }
        AR_TRY(launch_gemm_f32(o, st));
        AR_TRY(launch_fold_rmsnorm_rows_f32(m->pf_x, m->pf_part, so > 1 ? so : 0, L.ffn_norm, h32, (int)R, d,
                                            (float)c.epsilon, st));
        GemmF32Launch u;
        u.A = h32; u.lda = d; u.W = (const float*)L.w1; u.W2 = (const float*)L.w3; u.ldw = d; u.M = (int)R;
        u.N = F; u.K = d; u.C = act32; u.ldc = F; u.epilogue = GEMV_EPI_SWIGLU;
        AR_TRY(launch_gemm_f32(u, st));
        GemmF32Launch dn;
        dn.A = act32; dn.lda = F; dn.W = (const float*)L.w2; dn.ldw = F; dn.M = (int)R; dn.N = d; dn.K = F;
        dn.C = m->pf_x; dn.ldc = d; dn.epilogue = GEMV_EPI_RESIDUAL;
        if (sd > 1) {
            dn.C = m->pf_part; dn.epilogue = GEMV_EPI_STORE; dn.ksplit = sd;
            pending = sd;
        }
        AR_TRY(launch_gemm_f32(dn, st));
    }
    return prefill_finish(m, T, pending, logits_out);
}

extern "C" int ar_hip_qwen3_prefill(ar_qwen3* m, float* logits_out) {
    AR_CHECK_ARG(m, "null model");
    const int T = m->prompt_len;
    AR_TRY(check_ready(m, T));
    AR_CHECK_ARG(m->host_pos == 0, "prefill starts a sequence: reset() first (position is %d)", m->host_pos);
    const ar_qwen3_cfg& c = m->cfg;
    if (c.weight_dtype == AR_DTYPE_F32) {
        // fp32 MFMA GEMMs need 64-wide outputs and 32-deep inputs; other shapes take the decode step
        const bool fits = c.dim % 64 == 0 && m->qkv_dim % 64 == 0 && c.hidden_dim % 64 == 0 && m->q_dim % 32 == 0 &&
                          c.kv_dtype == AR_DTYPE_F32;
        return fits ? prefill_f32(m, T, logits_out) : prefill_by_steps(m, T, logits_out);
    }
    hipStream_t st = m->ctx->stream;
    const int B = m->B, d = c.dim, F = c.hidden_dim, qd = m->q_dim;
    const size_t R = (size_t)B * T;
    AR_CHECK_ARG(R <= (size_t)INT32_MAX / 16, "prefill: %zu rows too many", R);
    AR_TRY(ensure_prefill_buffers(m, R));
    AR_TRY(ensure_f16_weights(m));
    if (!m->pf_w16_in_range) return prefill_by_steps(m, T, logits_out);
    AR_HIP_TRY(hipMemsetAsync(m->pf_flag, 0, sizeof(int), st));
    int* const rf = m->pf_flag;
    const size_t dd = d, FF = F;
    const size_t per_layer16 = (size_t)m->qkv_dim * dd + dd * qd + 3 * FF * dd;
    AR_TRY(launch_embed_rows(m->embed, c.weight_dtype, d, m->tokens, m->S + 1, T, (int)R, m->pf_x, st));
    const size_t layer_cache = (size_t)B * c.kv_head_count * m->S * c.head_size;
    // rocBLAS products: O and down add into the residual rows in place (beta 1), so no k-slices;
    // gate/up go through the stacked-weight product and a SwiGLU pass; a QKV projection with a bias
    // stays on gemm.hip's kernel (bias in its epilogue)
    const bool blas = m->pf_gemm == AR_PREFILL_GEMM_ROCBLAS;
    if (blas && m->pf_gu_elems < R * 2 * FF) {
        if (m->pf_gu) AR_TRY(ar_ctx_free(m->ctx, m->pf_gu));
        m->pf_gu = nullptr;
        m->pf_gu_elems = 0;
        AR_TRY(ar_ctx_alloc(m->ctx, R * 2 * FF * 2, (void**)&m->pf_gu));
        m->pf_gu_elems = R * 2 * FF;
    }
    auto gemm = [&](const GemmLaunch& g) {
        return blas && !g.bias ? launch_gemm_blas(m->ctx, g, m->pf_gu, m->pf_gu_elems, st) : launch_gemm(g, st);
    };
    const int so = blas ? 1 : prefill_ksplit(m, R, d, qd), sd = blas ? 1 : prefill_ksplit(m, R, d, F);
    if ((so > 1 || sd > 1) && m->pf_part_rows < R) {
        if (m->pf_part) AR_TRY(ar_ctx_free(m->ctx, m->pf_part));
        m->pf_part = nullptr;
        m->pf_part_rows = 0;
        AR_TRY(ar_ctx_alloc(m->ctx, (size_t)kMaxKSplit * R * d * 4, (void**)&m->pf_part));
        m->pf_part_rows = R;
    }
    int pending = 0;  // k-slices of the last residual projection not yet added into pf_x
    for (int l = 0; l < c.layer_count; l++) {
        const Layer& L = m->layers[l];
        const uint16_t* w16 = m->pf_w16 + per_layer16 * l;
        const uint16_t* wqkv16 = w16;
        const uint16_t* wo16 = wqkv16 + (size_t)m->qkv_dim * dd;
        const uint16_t* w1_16 = wo16 + dd * qd;
        const uint16_t* w3_16 = w1_16 + FF * dd;
        const uint16_t* w2_16 = w3_16 + FF * dd;
        AR_TRY(launch_fold_rmsnorm_rows_f16(m->pf_x, m->pf_part, pending, L.attn_norm, m->pf_h, (int)R, d,
                                            (float)c.epsilon, rf, st));
        pending = 0;
        GemmLaunch g;
        g.A = m->pf_h; g.lda = d; g.W = wqkv16; g.ldw = d; g.M = (int)R; g.N = m->qkv_dim; g.K = d;
        g.bias = L.bqkv; g.C = m->pf_qkv; g.ldc = m->qkv_dim; g.epilogue = GEMV_EPI_STORE; g.f16 = true;
        AR_TRY(gemm(g));
        PrefillPrep pp;
        pp.qkv = m->pf_qkv; pp.qkv_stride = m->qkv_dim; pp.q_norm = L.q_norm; pp.k_norm = L.k_norm;
        pp.eps = (float)c.epsilon; pp.per_head = c.qk_norm_mode == AR_QK_NORM_PER_HEAD; pp.rope_tab = m->rope_tab;
        pp.kcache = (char*)m->kcache + l * layer_cache * m->kv_elem;
        pp.vcache = (char*)m->vcache + l * layer_cache * m->kv_elem;
        pp.kv16 = c.kv_dtype == AR_DTYPE_F16; pp.B = B; pp.S = m->S;
        pp.T = T; pp.p0 = 0; pp.heads = c.head_count; pp.kv_heads = c.kv_head_count; pp.hd = c.head_size;
        pp.qb = m->pf_q; pp.k16 = m->pf_k16; pp.vt16 = m->pf_vt16; pp.Tp = m->pf_tp; pp.range_flag = rf;
        AR_TRY(launch_qk_prep(pp, st));
        AR_TRY(launch_flash_prefill(m->pf_q, m->pf_k16, m->pf_vt16, m->pf_h, B, T, m->pf_tp, c.head_count,
                                    c.kv_head_count, c.head_size, st));
        GemmLaunch o;
        o.A = m->pf_h; o.lda = qd; o.W = wo16; o.ldw = qd; o.M = (int)R; o.N = d; o.K = qd;
        o.C = m->pf_x; o.ldc = d; o.epilogue = GEMV_EPI_RESIDUAL; o.f16 = true;
        if (so > 1) {  // k-slices into pf_part, added into pf_x by the next row RMSNorm
            o.C = m->pf_part; o.epilogue = GEMV_EPI_STORE; o.ksplit = so;
        }
        AR_TRY(gemm(o));
        AR_TRY(launch_fold_rmsnorm_rows_f16(m->pf_x, m->pf_part, so > 1 ? so : 0, L.ffn_norm, m->pf_h, (int)R, d,
                                            (float)c.epsilon, rf, st));
        GemmLaunch u;
        u.A = m->pf_h; u.lda = d; u.W = w1_16; u.W2 = w3_16; u.ldw = d; u.M = (int)R;
        u.N = F; u.K = d; u.O = m->pf_act; u.ldo = F; u.epilogue = GEMV_EPI_SWIGLU; u.f16 = true;
        u.range_flag = rf;
        AR_TRY(gemm(u));
        GemmLaunch dn;
        dn.A = m->pf_act; dn.lda = F; dn.W = w2_16; dn.ldw = F; dn.M = (int)R; dn.N = d; dn.K = F;
        dn.C = m->pf_x; dn.ldc = d; dn.epilogue = GEMV_EPI_RESIDUAL; dn.f16 = true;
        if (sd > 1) {
            dn.C = m->pf_part; dn.epilogue = GEMV_EPI_STORE; dn.ksplit = sd;
            pending = sd;
        }
        AR_TRY(gemm(dn));
    }
    // A value stored as an fp16 MFMA operand left the fp16 range (outlier activations of a real
    // checkpoint): the batched pass is discarded and the prompt goes through the decode step, whose
    // activations stay fp32, leaving the model where the batched pass would.  Checked before the
    // logits and the sampler run, so no draw of a sequence's generator is spent on the discarded pass.
    int overflow = 0;
    AR_HIP_TRY(hipMemcpyAsync(&overflow, m->pf_flag, sizeof(int), hipMemcpyDeviceToHost, st));
    AR_HIP_TRY(hipStreamSynchronize(st));
    if (overflow) return prefill_by_steps(m, T, logits_out);
    return prefill_finish(m, T, pending, logits_out);
}
