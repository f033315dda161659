/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference Qwen3 decode step.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this code, and only as the checker; the product path never links it.
 *
 * This header is instantiated twice by qwen3_oracle.c:
 *   REAL = double, SFX = _f64  -> the reference default precision
 *                                 (AR_HARDWARE_PRECISION=FP64, base/hardware/.../Hardware.java:684)
 *   REAL = float,  SFX = _f32  -> AR_HARDWARE_PRECISION=FP32
 *
 * Every reduction is a sequential left-to-right sum, as the reference's generated
 * JNI C computes them (compute/algebra/.../AggregatedProducerComputation.java:435-457,
 * base/code/.../collect/WeightedSumExpression.java:54-63).  Output rows are spread
 * over OpenMP threads the way the reference strides global_id over its CPU pool;
 * that never changes a result because each output element is summed by one thread.
 *
 * In FP32 mode transcendental functions go through the double-precision libm
 * entry points and are rounded to float, because the generated C calls exp/log/
 * sin/cos (base/code/.../expression/Exp.java:51, Logarithm.java:50, Sine.java:51,
 * Cosine.java:51) on float operands; pow uses powf
 * (base/hardware/.../c/CJNILanguageOperations.java:69-72).
 */

#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define FN(n) CAT(n, SFX)

/* ---- elementary functions at context precision ---------------------------- */
static inline REAL FN(r_exp)(REAL x) { return (REAL)exp((double)x); }
static inline REAL FN(r_log)(REAL x) { return (REAL)log((double)x); }
static inline REAL FN(r_cos)(REAL x) { return (REAL)cos((double)x); }
static inline REAL FN(r_sin)(REAL x) { return (REAL)sin((double)x); }
static inline REAL FN(r_pow_half)(REAL x) {
#if IS_F32
    return powf(x, 0.5f);
#else
    return pow(x, 0.5);
#endif
}

/*
 * rmsnorm -- domain/graph/.../layers/NormalizationLayerFeatures.java:584-595
 *   ss = sum_i x_i*x_i (pow(x,2) is simplified to x*x, base/code/.../expression/Exponent.java:162-163)
 *   ss = ss / size + eps ; r = 1 / pow(ss, 0.5) ; y_i = (w_i * x_i) * r
 */
void FN(oracle_rmsnorm)(REAL *out, const REAL *x, const REAL *w, int n, double eps) {
    REAL ss = 0;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (REAL)n + (REAL)eps;
    REAL r = (REAL)1 / FN(r_pow_half)(ss);
    for (int i = 0; i < n; i++) out[i] = (w[i] * x[i]) * r;
}

/* rmsnorm applied independently to groups of `group` elements (HF per-head QK-norm). */
void FN(oracle_rmsnorm_grouped)(REAL *out, const REAL *x, const REAL *w, int n, int group, double eps) {
    for (int g = 0; g < n / group; g++)
        FN(oracle_rmsnorm)(out + (size_t)g * group, x + (size_t)g * group, w + (size_t)g * group, group, eps);
}

/*
 * dense -- domain/graph/.../layers/LayerFeatures.java:785-830 -> MatrixFeatures.matmul
 * (compute/algebra/.../MatrixFeatures.java:182-337): y[o] = sum_i W[o,i] * x[i] (+ b[o]),
 * W row-major (out, in) as the HF state dict stores it.  Four rows are interleaved per
 * iteration for instruction-level parallelism; each row is still summed in index order.
 */
void FN(oracle_dense)(REAL *y, const REAL *W, const REAL *x, const REAL *bias, int rows, int cols) {
    int nq = rows / 4;
#pragma omp parallel for schedule(static)
    for (int q = 0; q < nq; q++) {
        const REAL *w0 = W + (size_t)(4 * q) * cols;
        const REAL *w1 = w0 + cols, *w2 = w1 + cols, *w3 = w2 + cols;
        REAL s0 = 0, s1 = 0, s2 = 0, s3 = 0;
        for (int i = 0; i < cols; i++) {
            REAL xi = x[i];
            s0 += w0[i] * xi; s1 += w1[i] * xi; s2 += w2[i] * xi; s3 += w3[i] * xi;
        }
        if (bias) { s0 += bias[4 * q]; s1 += bias[4 * q + 1]; s2 += bias[4 * q + 2]; s3 += bias[4 * q + 3]; }
        y[4 * q] = s0; y[4 * q + 1] = s1; y[4 * q + 2] = s2; y[4 * q + 3] = s3;
    }
    for (int o = 4 * nq; o < rows; o++) {
        const REAL *w0 = W + (size_t)o * cols;
        REAL s = 0;
        for (int i = 0; i < cols; i++) s += w0[i] * x[i];
        if (bias) s += bias[o];
        y[o] = s;
    }
}

/*
 * computeRopeFreqs -- engine/ml/.../RotationFeatures.java:189-208
 *   invFreq[f] = exp(f * (-2 ln(theta) / headDim)); angle = pos * invFreq[f]
 *   freqCis[pos, f, 0] = cos(angle), freqCis[pos, f, 1] = sin(angle)
 * out has shape (seq_len, head_dim/2, 2).
 */
void FN(oracle_rope_freqs)(REAL *out, double theta, int head_dim, int seq_len) {
    int fd = head_dim / 2;
    REAL c = (REAL)(-2.0 * log(theta) / head_dim);
    for (int p = 0; p < seq_len; p++)
        for (int f = 0; f < fd; f++) {
            REAL invf = FN(r_exp)((REAL)f * c);
            REAL ang = (REAL)p * invf;
            out[((size_t)p * fd + f) * 2 + 0] = FN(r_cos)(ang);
            out[((size_t)p * fd + f) * 2 + 1] = FN(r_sin)(ang);
        }
}

/*
 * reshapeToSplitHalfRope -- engine/ml/.../AttentionFeatures.java:195-210:
 *   out[h, f, half] = in[h*hd + half*(hd/2) + f]
 * reshapeFromSplitHalfRope -- AttentionFeatures.java:223-237:
 *   out[h*hd + half*(hd/2) + f] = in[h, f, half]
 */
void FN(oracle_split_half)(REAL *out, const REAL *in, int heads, int hd) {
    int fd = hd / 2;
    for (int h = 0; h < heads; h++)
        for (int f = 0; f < fd; f++)
            for (int half = 0; half < 2; half++)
                out[((size_t)h * fd + f) * 2 + half] = in[(size_t)h * hd + half * fd + f];
}

void FN(oracle_unsplit_half)(REAL *out, const REAL *in, int heads, int hd) {
    int fd = hd / 2;
    for (int h = 0; h < heads; h++)
        for (int half = 0; half < 2; half++)
            for (int f = 0; f < fd; f++)
                out[(size_t)h * hd + half * fd + f] = in[((size_t)h * fd + f) * 2 + half];
}

/*
 * ropeRotation -- engine/ml/.../RotationFeatures.java:124-170, applied to the split-half
 * layout (heads, hd/2, 2): out1 = x1*cos - x2*sin ; out2 = x2*cos + x1*sin (lines 161-162),
 * with (cos, sin) = freqCis[pos, f].
 */
void FN(oracle_rope_rotate_split)(REAL *x, int heads, int hd, const REAL *freqs_at_pos) {
    int fd = hd / 2;
    for (int h = 0; h < heads; h++)
        for (int f = 0; f < fd; f++) {
            REAL c = freqs_at_pos[2 * f], s = freqs_at_pos[2 * f + 1];
            REAL x1 = x[((size_t)h * fd + f) * 2], x2 = x[((size_t)h * fd + f) * 2 + 1];
            REAL o1 = x1 * c - x2 * s;
            REAL o2 = x2 * c + x1 * s;
            x[((size_t)h * fd + f) * 2] = o1;
            x[((size_t)h * fd + f) * 2 + 1] = o2;
        }
}

/* Split-half -> rotate -> unsplit on a flat (heads*hd) vector, as the Qwen3 graph chains
 * them (AttentionFeatures.java:847-851 for keys, 893-897 for queries). */
/* The same with a given freqCis row (hd/2 (cos, sin) pairs), as a model built from a
 * checkpoint's table uses it (engine/ml/.../llama2/Llama2.java:181-192, Llama2Weights.freqCis). */
void FN(oracle_rope_flat_row)(REAL *x, int heads, int hd, const REAL *freq_row) {
    REAL *tmp = (REAL *)malloc(sizeof(REAL) * (size_t)heads * hd);
    FN(oracle_split_half)(tmp, x, heads, hd);
    FN(oracle_rope_rotate_split)(tmp, heads, hd, freq_row);
    FN(oracle_unsplit_half)(x, tmp, heads, hd);
    free(tmp);
}

void FN(oracle_rope_flat)(REAL *x, int heads, int hd, int pos, double theta) {
    int fd = hd / 2;
    REAL *fr = (REAL *)malloc(sizeof(REAL) * (size_t)fd * 2);
    REAL c = (REAL)(-2.0 * log(theta) / hd);
    for (int f = 0; f < fd; f++) {
        REAL invf = FN(r_exp)((REAL)f * c);
        REAL ang = (REAL)pos * invf;
        fr[2 * f] = FN(r_cos)(ang);
        fr[2 * f + 1] = FN(r_sin)(ang);
    }
    FN(oracle_rope_flat_row)(x, heads, hd, fr);
    free(fr);
}

/* gqaExpand -- engine/ml/.../AttentionFeatures.java:372-391: query head h reads KV head
 * h / (heads/kvHeads).  out (heads*hd) <- in (kvHeads*hd). */
void FN(oracle_gqa_expand)(REAL *out, const REAL *in, int kv_heads, int heads, int hd) {
    int per = heads / kv_heads;
    for (int h = 0; h < heads; h++)
        for (int i = 0; i < hd; i++) out[(size_t)h * hd + i] = in[(size_t)(h / per) * hd + i];
}

/* Causal mask row -- AttentionFeatures.java:906-917: mask[t] = t > pos ? -10000 : 0. */
void FN(oracle_causal_mask)(REAL *out, int seq_len, int pos) {
    for (int t = 0; t < seq_len; t++) out[t] = (t > pos) ? (REAL)-10000.0 : (REAL)0.0;
}

/* softmax with log-sum-exp stability -- domain/graph/.../ActivationFeatures.java:135-143:
 *   m = max ; z = x - m ; a = exp(z - log(sum exp(z))), per row of n elements. */
void FN(oracle_softmax)(REAL *x, int rows, int n) {
    for (int r = 0; r < rows; r++) {
        REAL *v = x + (size_t)r * n;
        REAL m = v[0];
        for (int t = 1; t < n; t++) if (v[t] > m) m = v[t];
        REAL s = 0;
        for (int t = 0; t < n; t++) s += FN(r_exp)(v[t] - m);
        REAL lse = FN(r_log)(s);
        for (int t = 0; t < n; t++) v[t] = FN(r_exp)((v[t] - m) - lse);
    }
}

/*
 * Attention core for one decode position -- AttentionFeatures.java:901-921:
 *   s[h,t] = (sum_i q[h,i] * K[t,g(h),i]) / sqrt(hd)       attentionKeysStandard :531-559
 *   s[h,t] += t > pos ? -10000 : 0                           causal mask :906-917
 *   a = softmax(s) (log-sum-exp form)                        ActivationFeatures.java:135-143
 *   o[h,i] = sum_t a[h,t] * V[t,g(h),i]                      attentionValuesStandard :572-616
 * The reference stores GQA-expanded caches (seq, heads, hd) (:823-826, :856-877); here the
 * cache is compact (seq, kvHeads, hd) and head h reads KV head g(h) = h/(heads/kvHeads),
 * which reads exactly the values the expanded copy holds.
 * full_seq = 1 scores all seq_len rows with the -10000 mask, as the reference graph does;
 * full_seq = 0 stops at t = pos.  Both give identical results because exp(-10000 - m)
 * underflows to +0 in both precisions; tests check the two modes agree bit for bit.
 */
/* One query head of oracle_attention: q_h (hd), KV head g of the compact caches, rows 0..n-1
 * scored, rows past pos masked; s is scratch of n values. */
static void FN(attention_head)(REAL *out_h, const REAL *q_h, const REAL *kc, const REAL *vc, int kv_heads, int g,
                               int hd, int pos, int n, REAL *s) {
    REAL scale = (REAL)sqrt((double)hd);
    for (int t = 0; t < n; t++) {
        const REAL *k = kc + ((size_t)t * kv_heads + g) * hd;
        REAL acc = 0;
        for (int i = 0; i < hd; i++) acc += q_h[i] * k[i];
        acc = acc / scale;
        s[t] = acc + ((t > pos) ? (REAL)-10000.0 : (REAL)0.0);
    }
    FN(oracle_softmax)(s, 1, n);
    for (int i = 0; i < hd; i++) {
        REAL acc = 0;
        for (int t = 0; t < n; t++) acc += s[t] * vc[((size_t)t * kv_heads + g) * hd + i];
        out_h[i] = acc;
    }
}

void FN(oracle_attention)(REAL *out, const REAL *q, const REAL *kc, const REAL *vc,
                          int heads, int kv_heads, int hd, int pos, int seq_len, int full_seq) {
    int per = heads / kv_heads;
    int n = full_seq ? seq_len : pos + 1;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < heads; h++) {
        REAL *s = (REAL *)malloc(sizeof(REAL) * (size_t)n);
        FN(attention_head)(out + (size_t)h * hd, q + (size_t)h * hd, kc, vc, kv_heads, h / per, hd, pos, n, s);
        free(s);
    }
}

/*
 * One attention block's position-dependent part (the decode-step GQA op):
 * QK-norm (AttentionFeatures.java:840-845 keys, :886-891 queries), split-half RoPE,
 * cache write of k and v at row pos (:858-864, :871-877), then oracle_attention.
 * q (heads*hd), k, v (kv_heads*hd) are the raw projections; they are not modified.
 * qk_group = heads*hd / kv_heads*hd (whole vector, reference) or hd (per head, HF);
 * pass group <= 0 to select the whole-vector form.
 */
static void FN(attention_block_impl)(REAL *out, const REAL *q_raw, const REAL *k_raw, const REAL *v_raw,
                                     const REAL *q_norm, const REAL *k_norm, REAL *kc, REAL *vc,
                                     int heads, int kv_heads, int hd, int pos, int seq_len,
                                     double theta, const REAL *freq_row, double qk_eps, int per_head_norm,
                                     int full_seq) {
    int qd = heads * hd, kd = kv_heads * hd;
    REAL *q = (REAL *)malloc(sizeof(REAL) * (size_t)qd);
    REAL *k = (REAL *)malloc(sizeof(REAL) * (size_t)kd);
    if (q_norm) {
        if (per_head_norm) FN(oracle_rmsnorm_grouped)(q, q_raw, q_norm, qd, hd, qk_eps);
        else FN(oracle_rmsnorm)(q, q_raw, q_norm, qd, qk_eps);
    } else memcpy(q, q_raw, sizeof(REAL) * qd);
    if (k_norm) {
        if (per_head_norm) FN(oracle_rmsnorm_grouped)(k, k_raw, k_norm, kd, hd, qk_eps);
        else FN(oracle_rmsnorm)(k, k_raw, k_norm, kd, qk_eps);
    } else memcpy(k, k_raw, sizeof(REAL) * kd);
    if (freq_row) {
        FN(oracle_rope_flat_row)(k, kv_heads, hd, freq_row);
        FN(oracle_rope_flat_row)(q, heads, hd, freq_row);
    } else {
        FN(oracle_rope_flat)(k, kv_heads, hd, pos, theta);
        FN(oracle_rope_flat)(q, heads, hd, pos, theta);
    }
    memcpy(kc + (size_t)pos * kd, k, sizeof(REAL) * kd);
    memcpy(vc + (size_t)pos * kd, v_raw, sizeof(REAL) * kd);
    FN(oracle_attention)(out, q, kc, vc, heads, kv_heads, hd, pos, seq_len, full_seq);
    free(q);
    free(k);
}

void FN(oracle_attention_block)(REAL *out, const REAL *q_raw, const REAL *k_raw, const REAL *v_raw,
                                const REAL *q_norm, const REAL *k_norm, REAL *kc, REAL *vc,
                                int heads, int kv_heads, int hd, int pos, int seq_len,
                                double theta, double qk_eps, int per_head_norm, int full_seq) {
    FN(attention_block_impl)(out, q_raw, k_raw, v_raw, q_norm, k_norm, kc, vc, heads, kv_heads, hd, pos, seq_len,
                             theta, NULL, qk_eps, per_head_norm, full_seq);
}

/* indexOfMax -- compute/algebra/.../AggregationFeatures.java:111-121: start at index 0,
 * move to index i only when x[i] > x[current] (first maximum wins). */
void FN(oracle_index_of_max)(const REAL *x, int rows, int n, int32_t *out) {
    for (int r = 0; r < rows; r++) {
        const REAL *v = x + (size_t)r * n;
        int best = 0;
        for (int i = 1; i < n; i++) if (v[i] > v[best]) best = i;
        out[r] = best;
    }
}

/* ---- whole model ---------------------------------------------------------- */

typedef struct FN(oracle_layer) {
    REAL *attn_norm, *wq, *wk, *wv, *wo, *bq, *bk, *bv, *q_norm, *k_norm, *ffn_norm, *w1, *w2, *w3;
    REAL *kc, *vc; /* compact caches (seq, kvHeads, hd) */
} FN(oracle_layer);

typedef struct FN(oracle_model) {
    oracle_cfg cfg;
    int q_dim, kv_dim;
    REAL *embed, *final_norm, *lm_head;
    REAL *rope_tab; /* (seq_len, hd/2, 2) freqCis given as a weight, or NULL: computed from theta */
    FN(oracle_layer) *layers;
    int pos;
    REAL *x, *h, *q, *k, *v, *att, *tmp, *g, *u;
} FN(oracle_model);

void *FN(oracle_model_create)(const oracle_cfg *cfg) {
    FN(oracle_model) *m = (FN(oracle_model) *)calloc(1, sizeof(FN(oracle_model)));
    m->cfg = *cfg;
    m->q_dim = cfg->n_heads * cfg->head_dim;
    m->kv_dim = cfg->n_kv_heads * cfg->head_dim;
    m->layers = (FN(oracle_layer) *)calloc((size_t)cfg->n_layers, sizeof(FN(oracle_layer)));
    for (int l = 0; l < cfg->n_layers; l++) {
        m->layers[l].kc = (REAL *)calloc((size_t)cfg->seq_len * m->kv_dim, sizeof(REAL));
        m->layers[l].vc = (REAL *)calloc((size_t)cfg->seq_len * m->kv_dim, sizeof(REAL));
    }
    int mx = cfg->dim;
    if (m->q_dim > mx) mx = m->q_dim;
    if (cfg->ffn_dim > mx) mx = cfg->ffn_dim;
    m->x = (REAL *)calloc((size_t)cfg->dim, sizeof(REAL));
    m->h = (REAL *)calloc((size_t)mx, sizeof(REAL));
    m->q = (REAL *)calloc((size_t)m->q_dim, sizeof(REAL));
    m->k = (REAL *)calloc((size_t)m->kv_dim, sizeof(REAL));
    m->v = (REAL *)calloc((size_t)m->kv_dim, sizeof(REAL));
    m->att = (REAL *)calloc((size_t)m->q_dim, sizeof(REAL));
    m->tmp = (REAL *)calloc((size_t)mx, sizeof(REAL));
    m->g = (REAL *)calloc((size_t)cfg->ffn_dim, sizeof(REAL));
    m->u = (REAL *)calloc((size_t)cfg->ffn_dim, sizeof(REAL));
    return m;
}

static void FN(free_layer)(FN(oracle_layer) *L) {
    REAL *ptrs[] = {L->attn_norm, L->wq, L->wk, L->wv, L->wo, L->bq, L->bk, L->bv,
                    L->q_norm, L->k_norm, L->ffn_norm, L->w1, L->w2, L->w3, L->kc, L->vc};
    for (size_t i = 0; i < sizeof(ptrs) / sizeof(ptrs[0]); i++) free(ptrs[i]);
}

void FN(oracle_model_destroy)(void *mp) {
    FN(oracle_model) *m = (FN(oracle_model) *)mp;
    if (!m) return;
    for (int l = 0; l < m->cfg.n_layers; l++) FN(free_layer)(&m->layers[l]);
    free(m->layers);
    if (m->lm_head != m->embed) free(m->lm_head);
    free(m->embed); free(m->final_norm); free(m->rope_tab);
    free(m->x); free(m->h); free(m->q); free(m->k); free(m->v); free(m->att); free(m->tmp);
    free(m->g); free(m->u);
    free(m);
}

static REAL *FN(copy_in)(const float *src, size_t n) {
    REAL *d = (REAL *)malloc(sizeof(REAL) * n);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) d[i] = (REAL)src[i];
    return d;
}

/* Weight keys follow the HF state-dict names Qwen3.model reads
 * (engine/ml/.../qwen3/Qwen3.java:338-384).  Returns 0 on success, -1 for an unknown
 * key, -2 for a size mismatch. */
int FN(oracle_model_set_weight)(void *mp, const char *key, const float *src, long long n) {
    FN(oracle_model) *m = (FN(oracle_model) *)mp;
    const oracle_cfg *c = &m->cfg;
    long long d = c->dim, qd = m->q_dim, kd = m->kv_dim, F = c->ffn_dim, V = c->vocab;
    if (!strcmp(key, "model.embed_tokens.weight")) {
        if (n != V * d) return -2;
        free(m->embed);
        m->embed = FN(copy_in)(src, (size_t)n);
        if (c->tied) m->lm_head = m->embed;
        return 0;
    }
    if (!strcmp(key, "lm_head.weight")) {
        if (n != V * d) return -2;
        if (c->tied) return 0; /* tied embeddings: the embedding matrix is the head */
        free(m->lm_head);
        m->lm_head = FN(copy_in)(src, (size_t)n);
        return 0;
    }
    if (!strcmp(key, "freq_cis")) { /* (positions >= seq_len, hd/2, 2); the first seq_len rows are kept */
        if (n % c->head_dim != 0 || n / c->head_dim < c->seq_len) return -2;
        free(m->rope_tab);
        m->rope_tab = FN(copy_in)(src, (size_t)c->seq_len * c->head_dim);
        return 0;
    }
    if (!strcmp(key, "model.norm.weight")) {
        if (n != d) return -2;
        free(m->final_norm);
        m->final_norm = FN(copy_in)(src, (size_t)n);
        return 0;
    }
    int l = -1, off = 0;
    if (sscanf(key, "model.layers.%d.%n", &l, &off) != 1 || l < 0 || l >= c->n_layers) return -1;
    const char *s = key + off;
    FN(oracle_layer) *L = &m->layers[l];
    REAL **dst = NULL;
    long long want = 0;
    if (!strcmp(s, "input_layernorm.weight")) { dst = &L->attn_norm; want = d; }
    else if (!strcmp(s, "post_attention_layernorm.weight")) { dst = &L->ffn_norm; want = d; }
    else if (!strcmp(s, "self_attn.q_proj.weight")) { dst = &L->wq; want = qd * d; }
    else if (!strcmp(s, "self_attn.k_proj.weight")) { dst = &L->wk; want = kd * d; }
    else if (!strcmp(s, "self_attn.v_proj.weight")) { dst = &L->wv; want = kd * d; }
    else if (!strcmp(s, "self_attn.o_proj.weight")) { dst = &L->wo; want = d * qd; }
    else if (!strcmp(s, "self_attn.q_proj.bias")) { dst = &L->bq; want = qd; }
    else if (!strcmp(s, "self_attn.k_proj.bias")) { dst = &L->bk; want = kd; }
    else if (!strcmp(s, "self_attn.v_proj.bias")) { dst = &L->bv; want = kd; }
    else if (!strcmp(s, "self_attn.q_norm.weight")) { dst = &L->q_norm; want = qd; }
    else if (!strcmp(s, "self_attn.k_norm.weight")) { dst = &L->k_norm; want = kd; }
    else if (!strcmp(s, "mlp.gate_proj.weight")) { dst = &L->w1; want = F * d; }
    else if (!strcmp(s, "mlp.up_proj.weight")) { dst = &L->w3; want = F * d; }
    else if (!strcmp(s, "mlp.down_proj.weight")) { dst = &L->w2; want = d * F; }
    else return -1;
    if (n != want) return -2;
    free(*dst);
    *dst = FN(copy_in)(src, (size_t)n);
    return 0;
}

/* AutoregressiveModel.reset -- engine/ml/.../AutoregressiveModel.java:203-207: position to 0.
 * Cache contents are left in place; rows past the position are masked. */
void FN(oracle_model_reset)(void *mp) { ((FN(oracle_model) *)mp)->pos = 0; }

int FN(oracle_model_position)(void *mp) { return ((FN(oracle_model) *)mp)->pos; }

/*
 * One forward pass of the Qwen3 graph for token `token` at the current position
 * (Qwen3.model, engine/ml/.../qwen3/Qwen3.java:334-415; AttentionFeatures.transformer
 * :1688-1708; FeedForwardFeatures.feedForward :140-157), then advance()
 * (AutoregressiveModel.java:217-220).  logits_out (vocab REAL values) may be NULL.
 * Returns the greedy next token (indexOfMax of the logits), or -1 on bad state.
 */
int FN(oracle_model_step)(void *mp, int token, REAL *logits_out) {
    FN(oracle_model) *m = (FN(oracle_model) *)mp;
    const oracle_cfg *c = &m->cfg;
    int d = c->dim, qd = m->q_dim, kd = m->kv_dim, F = c->ffn_dim, hd = c->head_dim;
    int pos = m->pos;
    if (pos >= c->seq_len || token < 0 || token >= c->vocab || !m->embed || !m->final_norm || !m->lm_head)
        return -1;
    /* embedding row: AutoregressiveModel.java:430 / Qwen3.java:411-414 */
    memcpy(m->x, m->embed + (size_t)token * d, sizeof(REAL) * d);
    for (int l = 0; l < c->n_layers; l++) {
        FN(oracle_layer) *L = &m->layers[l];
        /* attention branch, accumulated into x (SequentialBlock.accum) */
        FN(oracle_rmsnorm)(m->h, m->x, L->attn_norm, d, c->eps);
        FN(oracle_dense)(m->k, L->wk, m->h, L->bk, kd, d);
        FN(oracle_dense)(m->v, L->wv, m->h, L->bv, kd, d);
        FN(oracle_dense)(m->q, L->wq, m->h, L->bq, qd, d);
        FN(attention_block_impl)(m->att, m->q, m->k, m->v, L->q_norm, L->k_norm, L->kc, L->vc,
                                 c->n_heads, c->n_kv_heads, hd, pos, c->seq_len, c->rope_theta,
                                 m->rope_tab ? m->rope_tab + (size_t)pos * hd : NULL,
                                 c->qk_eps, c->qk_norm_mode == 1, c->full_seq_mask);
        FN(oracle_dense)(m->tmp, L->wo, m->att, NULL, d, qd);
        for (int i = 0; i < d; i++) m->x[i] = m->x[i] + m->tmp[i];
        /* feed-forward branch: x += W2 (W3 h (.) silu(W1 h)) with silu(g) = g * 1/(exp(-g)+1)
         * (ActivationFeatures.java:263-265, ArithmeticFeatures.java:754-756) */
        FN(oracle_rmsnorm)(m->h, m->x, L->ffn_norm, d, c->eps);
        FN(oracle_dense)(m->g, L->w1, m->h, NULL, F, d);
        FN(oracle_dense)(m->u, L->w3, m->h, NULL, F, d);
        for (int i = 0; i < F; i++) {
            REAL gi = m->g[i];
            REAL sg = (REAL)1 / (FN(r_exp)(-gi) + (REAL)1);
            m->g[i] = m->u[i] * (gi * sg);
        }
        FN(oracle_dense)(m->tmp, L->w2, m->g, NULL, d, F);
        for (int i = 0; i < d; i++) m->x[i] = m->x[i] + m->tmp[i];
    }
    /* final norm + tied logits projection: Qwen3.java:401-405 */
    FN(oracle_rmsnorm)(m->h, m->x, m->final_norm, d, c->eps);
    REAL *logits = logits_out ? logits_out : (REAL *)malloc(sizeof(REAL) * (size_t)c->vocab);
    FN(oracle_dense)(logits, m->lm_head, m->h, NULL, c->vocab, d);
    int32_t next = 0;
    FN(oracle_index_of_max)(logits, 1, c->vocab, &next);
    if (!logits_out) free(logits);
    m->pos = pos + 1;
    return next;
}

#include "qwen3_oracle_prefill.h"

/* Copies the current residual-stream vector x (dim values) for activation checks. */
void FN(oracle_model_hidden)(void *mp, REAL *out) {
    FN(oracle_model) *m = (FN(oracle_model) *)mp;
    memcpy(out, m->x, sizeof(REAL) * m->cfg.dim);
}

#undef FN
#undef CAT
#undef CAT2
