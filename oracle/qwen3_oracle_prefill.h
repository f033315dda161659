/*
 * TEST INFRASTRUCTURE ONLY -- the oracle's batched prompt pass (included by qwen3_oracle_impl.h,
 * once per precision).
 *
 * The reference feeds a prompt one token per forward pass (AutoregressiveModel.next,
 * engine/ml/.../AutoregressiveModel.java:295-308).  oracle_model_prefill computes exactly what
 * those T calls of oracle_model_step compute -- every output element is the same sequence of
 * roundings (each dense output a left-to-right sum with separate multiply and add, the same
 * RMSNorm, QK-norm, RoPE, softmax and value sums) -- but lays the work out over all prompt rows at
 * once, so long prompts (8192 rows of a 2560-wide layer) finish in seconds instead of hours:
 *   - dense: rows of the prompt against packed panels of the weight matrix, the weight rows of a
 *     panel in vector lanes, the sum over the input index kept sequential in every lane;
 *   - attention: every (row, KV head) pair independently, the query heads of the group in vector
 *     lanes for the scores, the value dimensions in lanes for the weighted sums;
 *   - the last layer computes its attention, O projection and feed-forward only for the last row,
 *     the only row whose output is used (its K and V rows are still computed for every row, since
 *     the cache holds them);
 *   - cache rows are written for every prompt position before any row's attention reads them;
 *     rows past a row's position are never read (or are masked to exactly zero weight in the
 *     full-sequence form), so this ordering cannot change a result.
 * tests/test_oracle.py checks prefill == T steps bit for bit in both precisions.
 */

/* One weight panel: PR consecutive output rows, stored input-index-major (panel[i][j] = W[o0+j][i]),
 * rows past the matrix zero.  Two vectors of lanes per panel row. */
#define PV (32 / (int)sizeof(REAL)) /* lanes of a 32-byte vector */
#define PR (2 * PV)
typedef REAL FN(vec) __attribute__((vector_size(32)));

/* Y[t][o] (+)= sum_i W[o][i] * X[t][i] (+ bias[o]) for t < T, o < rows, each output summed over i in
 * index order with separate multiply and add, exactly as oracle_dense sums it.
 * mode 0: Y = sum (+ bias);  mode 1: Y = Y + sum (the residual add of the step, done after the sum). */
__attribute__((target_clones("avx2", "default")))
static void FN(gemm_rows)(REAL *Y, int ldy, const REAL *W, const REAL *X, int ldx, const REAL *bias, int T,
                          int rows, int cols, int mode) {
    if (T <= 0 || rows <= 0) return;
    const int np = (rows + PR - 1) / PR;
    const size_t panel = (size_t)cols * PR;
    REAL *Wp = (REAL *)aligned_alloc(64, (sizeof(REAL) * panel * (size_t)np + 63) / 64 * 64);
#pragma omp parallel for schedule(static)
    for (int p = 0; p < np; p++)
        for (int i = 0; i < cols; i++)
            for (int j = 0; j < PR; j++) {
                const int o = p * PR + j;
                Wp[(size_t)p * panel + (size_t)i * PR + j] = o < rows ? W[(size_t)o * cols + i] : (REAL)0;
            }
    const int TC = 128;  /* prompt rows per chunk: the chunk's inputs stay in cache across panels */
    const int nc = (T + TC - 1) / TC;
#pragma omp parallel for collapse(2) schedule(static)
    for (int c = 0; c < nc; c++)
        for (int p = 0; p < np; p++) {
            const FN(vec) *wp = (const FN(vec) *)(Wp + (size_t)p * panel);
            const int t_end = (c + 1) * TC < T ? (c + 1) * TC : T;
            int t = c * TC;
            for (; t + 4 <= t_end; t += 4) {
                const REAL *x0 = X + (size_t)t * ldx, *x1 = x0 + ldx, *x2 = x1 + ldx, *x3 = x2 + ldx;
                FN(vec) a00 = {0}, a01 = {0}, a10 = {0}, a11 = {0}, a20 = {0}, a21 = {0}, a30 = {0}, a31 = {0};
                for (int i = 0; i < cols; i++) {
                    const FN(vec) w0 = wp[2 * i], w1 = wp[2 * i + 1];
                    const REAL b0 = x0[i], b1 = x1[i], b2 = x2[i], b3 = x3[i];
                    a00 = a00 + w0 * b0; a01 = a01 + w1 * b0;
                    a10 = a10 + w0 * b1; a11 = a11 + w1 * b1;
                    a20 = a20 + w0 * b2; a21 = a21 + w1 * b2;
                    a30 = a30 + w0 * b3; a31 = a31 + w1 * b3;
                }
                const FN(vec) *acc[4][2] = {{&a00, &a01}, {&a10, &a11}, {&a20, &a21}, {&a30, &a31}};
                for (int r = 0; r < 4; r++)
                    for (int j = 0; j < PR; j++) {
                        const int o = p * PR + j;
                        if (o >= rows) break;
                        REAL v = (*acc[r][j / PV])[j % PV];
                        REAL *y = Y + (size_t)(t + r) * ldy + o;
                        if (mode == 1) *y = *y + v;
                        else *y = bias ? v + bias[o] : v;
                    }
            }
            for (; t < t_end; t++) {
                const REAL *x0 = X + (size_t)t * ldx;
                FN(vec) a0 = {0}, a1 = {0};
                for (int i = 0; i < cols; i++) {
                    a0 = a0 + wp[2 * i] * x0[i];
                    a1 = a1 + wp[2 * i + 1] * x0[i];
                }
                for (int j = 0; j < PR; j++) {
                    const int o = p * PR + j;
                    if (o >= rows) break;
                    REAL v = j < PV ? a0[j] : a1[j - PV];
                    REAL *y = Y + (size_t)t * ldy + o;
                    if (mode == 1) *y = *y + v;
                    else *y = bias ? v + bias[o] : v;
                }
            }
        }
    free(Wp);
}

/* The G query heads sharing KV head g at position pos, with the arithmetic of attention_head
 * per head: q (G x hd), out (G x hd); s scratch of G * n values, qT of hd * 8. */
__attribute__((target_clones("avx2", "default")))
static void FN(attention_group)(REAL *out, const REAL *q, const REAL *kc, const REAL *vc, int kv_heads, int g,
                                int G, int hd, int pos, int n, REAL *s, REAL *qT) {
    typedef REAL v8 __attribute__((vector_size(8 * sizeof(REAL))));
    const REAL scale = (REAL)sqrt((double)hd);
    for (int i = 0; i < hd; i++)
        for (int h = 0; h < 8; h++) qT[(size_t)i * 8 + h] = h < G ? q[(size_t)h * hd + i] : (REAL)0;
    const v8 *qv = (const v8 *)qT;
    int t = 0;
    for (; t + 4 <= n; t += 4) {
        const REAL *k0 = kc + ((size_t)t * kv_heads + g) * hd, *k1 = k0 + (size_t)kv_heads * hd;
        const REAL *k2 = k1 + (size_t)kv_heads * hd, *k3 = k2 + (size_t)kv_heads * hd;
        v8 a0 = {0}, a1 = {0}, a2 = {0}, a3 = {0};
        for (int i = 0; i < hd; i++) {
            const v8 qi = qv[i];
            a0 = a0 + qi * k0[i]; a1 = a1 + qi * k1[i]; a2 = a2 + qi * k2[i]; a3 = a3 + qi * k3[i];
        }
        const v8 *a[4] = {&a0, &a1, &a2, &a3};
        for (int r = 0; r < 4; r++)
            for (int h = 0; h < G; h++) {
                REAL acc = (*a[r])[h] / scale;
                s[(size_t)h * n + t + r] = acc + ((t + r > pos) ? (REAL)-10000.0 : (REAL)0.0);
            }
    }
    for (; t < n; t++) {
        const REAL *k0 = kc + ((size_t)t * kv_heads + g) * hd;
        v8 a0 = {0};
        for (int i = 0; i < hd; i++) a0 = a0 + qv[i] * k0[i];
        for (int h = 0; h < G; h++) {
            REAL acc = a0[h] / scale;
            s[(size_t)h * n + t] = acc + ((t > pos) ? (REAL)-10000.0 : (REAL)0.0);
        }
    }
    typedef REAL v8u __attribute__((vector_size(8 * sizeof(REAL)), aligned(sizeof(REAL))));
    for (int h = 0; h < G; h++) {
        REAL *sh = s + (size_t)h * n;
        FN(oracle_softmax)(sh, 1, n);
        v8 o[16];  /* hd / 8 <= 16 vectors of value dimensions, each summed over rows in order */
        const int nv = hd / 8;
        for (int j = 0; j < nv; j++) o[j] = (v8){0};
        for (int tt = 0; tt < n; tt++) {
            const REAL a = sh[tt];
            const v8u *v = (const v8u *)(vc + ((size_t)tt * kv_heads + g) * hd);
            for (int j = 0; j < nv; j++) o[j] = o[j] + a * v[j];
        }
        for (int j = 0; j < nv; j++) memcpy(out + (size_t)h * hd + 8 * j, &o[j], sizeof(v8));
    }
}

/*
 * T prompt tokens at positions pos..pos+T-1 (pos = the model's current position), as T calls of
 * oracle_model_step would feed them; logits_out (vocab values, may be NULL) receives the last
 * row's logits.  Returns the greedy token after the last row (indexOfMax of its logits), or -1 on
 * bad arguments.  Afterwards the model is where those T steps leave it.
 */
int FN(oracle_model_prefill)(void *mp, const int32_t *tokens, int T, REAL *logits_out) {
    FN(oracle_model) *m = (FN(oracle_model) *)mp;
    const oracle_cfg *c = &m->cfg;
    const int d = c->dim, qd = m->q_dim, kd = m->kv_dim, F = c->ffn_dim, hd = c->head_dim;
    const int p0 = m->pos, H = c->n_heads, KV = c->n_kv_heads, G = H / KV;
    if (T < 1 || p0 + T > c->seq_len || !m->embed || !m->final_norm || !m->lm_head || G > 8 || hd % 8 != 0 ||
        hd > 128)
        return -1;
    for (int t = 0; t < T; t++)
        if (tokens[t] < 0 || tokens[t] >= c->vocab) return -1;
    const int hw = d > qd ? d : qd;
    REAL *X = (REAL *)malloc(sizeof(REAL) * (size_t)T * d);
    REAL *Hn = (REAL *)malloc(sizeof(REAL) * (size_t)T * hw);
    REAL *Q = (REAL *)malloc(sizeof(REAL) * (size_t)T * qd);
    REAL *K = (REAL *)malloc(sizeof(REAL) * (size_t)T * kd);
    REAL *V = (REAL *)malloc(sizeof(REAL) * (size_t)T * kd);
    REAL *A = (REAL *)malloc(sizeof(REAL) * (size_t)T * qd);
    REAL *Gt = (REAL *)malloc(sizeof(REAL) * (size_t)T * F);
    REAL *U = (REAL *)malloc(sizeof(REAL) * (size_t)T * F);
    if (!X || !Hn || !Q || !K || !V || !A || !Gt || !U) {
        free(X); free(Hn); free(Q); free(K); free(V); free(A); free(Gt); free(U);
        return -1;
    }
    /* embedding rows: AutoregressiveModel.java:430 / Qwen3.java:411-414 */
    for (int t = 0; t < T; t++) memcpy(X + (size_t)t * d, m->embed + (size_t)tokens[t] * d, sizeof(REAL) * d);
    const int full = c->full_seq_mask;
    for (int l = 0; l < c->n_layers; l++) {
        FN(oracle_layer) *L = &m->layers[l];
        /* rows whose attention / feed-forward output is used: all, except in the last layer */
        const int r0 = l + 1 < c->n_layers ? 0 : T - 1;
#pragma omp parallel for schedule(static)
        for (int t = 0; t < T; t++)
            FN(oracle_rmsnorm)(Hn + (size_t)t * hw, X + (size_t)t * d, L->attn_norm, d, c->eps);
        FN(gemm_rows)(K, kd, L->wk, Hn, hw, L->bk, T, kd, d, 0);
        FN(gemm_rows)(V, kd, L->wv, Hn, hw, L->bv, T, kd, d, 0);
        FN(gemm_rows)(Q + (size_t)r0 * qd, qd, L->wq, Hn + (size_t)r0 * hw, hw, L->bq, T - r0, qd, d, 0);
        /* QK-norm, RoPE and the cache write of every row (attention_block_impl's order per row) */
#pragma omp parallel for schedule(static)
        for (int t = 0; t < T; t++) {
            const int pos = p0 + t;
            const REAL *fr = m->rope_tab ? m->rope_tab + (size_t)pos * hd : NULL;
            REAL *k = K + (size_t)t * kd;
            REAL *kn = (REAL *)malloc(sizeof(REAL) * (size_t)kd);
            if (L->k_norm) {
                if (c->qk_norm_mode == 1) FN(oracle_rmsnorm_grouped)(kn, k, L->k_norm, kd, hd, c->qk_eps);
                else FN(oracle_rmsnorm)(kn, k, L->k_norm, kd, c->qk_eps);
            } else memcpy(kn, k, sizeof(REAL) * kd);
            if (fr) FN(oracle_rope_flat_row)(kn, KV, hd, fr);
            else FN(oracle_rope_flat)(kn, KV, hd, pos, c->rope_theta);
            memcpy(L->kc + (size_t)pos * kd, kn, sizeof(REAL) * kd);
            memcpy(L->vc + (size_t)pos * kd, V + (size_t)t * kd, sizeof(REAL) * kd);
            free(kn);
            if (t >= r0) {
                REAL *q = Q + (size_t)t * qd;
                REAL *qn = (REAL *)malloc(sizeof(REAL) * (size_t)qd);
                if (L->q_norm) {
                    if (c->qk_norm_mode == 1) FN(oracle_rmsnorm_grouped)(qn, q, L->q_norm, qd, hd, c->qk_eps);
                    else FN(oracle_rmsnorm)(qn, q, L->q_norm, qd, c->qk_eps);
                } else memcpy(qn, q, sizeof(REAL) * qd);
                if (fr) FN(oracle_rope_flat_row)(qn, H, hd, fr);
                else FN(oracle_rope_flat)(qn, H, hd, pos, c->rope_theta);
                memcpy(q, qn, sizeof(REAL) * qd);
                free(qn);
            }
        }
        /* attention of every (row, KV head) pair, the heaviest rows first */
        const int npairs = (T - r0) * KV;
#pragma omp parallel
        {
            const int nmax = full ? c->seq_len : p0 + T;
            REAL *s = (REAL *)malloc(sizeof(REAL) * (size_t)G * nmax);
            REAL *qT = (REAL *)aligned_alloc(64, (sizeof(REAL) * (size_t)hd * 8 + 63) / 64 * 64);
#pragma omp for schedule(dynamic, 4)
            for (int i = 0; i < npairs; i++) {
                const int t = T - 1 - i / KV, g = i % KV, pos = p0 + t;
                const int n = full ? c->seq_len : pos + 1;
                FN(attention_group)(A + (size_t)t * qd + (size_t)g * G * hd, Q + (size_t)t * qd + (size_t)g * G * hd,
                                    L->kc, L->vc, KV, g, G, hd, pos, n, s, qT);
            }
            free(s);
            free(qT);
        }
        const int R = T - r0;
        /* x += Wo . attention (AttentionFeatures.java:922, :1704) */
        FN(gemm_rows)(X + (size_t)r0 * d, d, L->wo, A + (size_t)r0 * qd, qd, NULL, R, d, qd, 1);
        /* feed-forward (FeedForwardFeatures.java:147-156) */
#pragma omp parallel for schedule(static)
        for (int t = r0; t < T; t++)
            FN(oracle_rmsnorm)(Hn + (size_t)t * hw, X + (size_t)t * d, L->ffn_norm, d, c->eps);
        FN(gemm_rows)(Gt + (size_t)r0 * F, F, L->w1, Hn + (size_t)r0 * hw, hw, NULL, R, F, d, 0);
        FN(gemm_rows)(U + (size_t)r0 * F, F, L->w3, Hn + (size_t)r0 * hw, hw, NULL, R, F, d, 0);
#pragma omp parallel for schedule(static)
        for (int t = r0; t < T; t++)
            for (int i = 0; i < F; i++) {
                REAL gi = Gt[(size_t)t * F + i];
                REAL sg = (REAL)1 / (FN(r_exp)(-gi) + (REAL)1);
                Gt[(size_t)t * F + i] = U[(size_t)t * F + i] * (gi * sg);
            }
        FN(gemm_rows)(X + (size_t)r0 * d, d, L->w2, Gt + (size_t)r0 * F, F, NULL, R, d, F, 1);
    }
    memcpy(m->x, X + (size_t)(T - 1) * d, sizeof(REAL) * d);
    free(X); free(Hn); free(Q); free(K); free(V); free(A); free(Gt); free(U);
    /* final norm + logits of the last row (Qwen3.java:401-405) */
    FN(oracle_rmsnorm)(m->h, m->x, m->final_norm, d, c->eps);
    REAL *logits = logits_out ? logits_out : (REAL *)malloc(sizeof(REAL) * (size_t)c->vocab);
    FN(oracle_dense)(logits, m->lm_head, m->h, NULL, c->vocab, d);
    int32_t next = 0;
    FN(oracle_index_of_max)(logits, 1, c->vocab, &next);
    if (!logits_out) free(logits);
    m->pos = p0 + T;
    return next;
}

#undef PV
#undef PR
