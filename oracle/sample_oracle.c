/*
 * TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's token sampling, the checker for
 * the device sampler (common_amd/csrc/sample.hip).  Loaded by tests/ through oracle/__init__.py;
 * the product library never calls it.
 *
 *  - java.util.Random as its public specification defines it (48-bit LCG, multiplier
 *    0x5DEECE66D, addend 0xB; setSeed scrambles with the multiplier; nextDouble =
 *    ((next(26) << 27) + next(27)) * 2^-53), the generator AutoregressiveModel draws from
 *    (engine/ml/.../AutoregressiveModel.java:416, :379).
 *  - AutoregressiveModel.sampleToken (AutoregressiveModel.java:323-386): greedy first maximum when
 *    temperature <= 0; else softmax of values / temperature in double (max subtracted, sequential
 *    sum, each value divided by the sum), nucleus filtering for top_p < 1 (stable sort by
 *    descending probability, cumulative sum until >= top_p, the rest zeroed, every value divided
 *    by the kept sum), then one nextDouble r and the first index whose running sum exceeds r
 *    (vocabSize - 1 if none does).
 *  - The sample function of AutoregressiveModel.of (AutoregressiveModel.java:413-425): greedy
 *    first maximum at temperature == 0; else logits / temperature, the softmax of
 *    DistributionFeatures.softmax(x, true) (compute/stats/.../DistributionFeatures.java:129-141:
 *    subtractIgnoreZero of the maximum, ArithmeticFeatures.java:215-231 -- a value equal to 0 stays
 *    0, a value equal to the maximum becomes the FP64 machine epsilon (Precision.java:110-121),
 *    others x - max -- then expIgnoreZero, CollectionExponentialComputation.java:50-58 -- 0 stays 0,
 *    and division by the sum), then sampleToken(probabilities, V, 1.0, 1.0, random).
 * Everything is in double, the reference's default precision.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define JR_MULT 0x5DEECE66DULL
#define JR_ADD 0xBULL
#define JR_MASK ((1ULL << 48) - 1)

uint64_t oracle_jrandom_seed(int64_t seed) { return ((uint64_t)seed ^ JR_MULT) & JR_MASK; }

static int32_t jr_next(uint64_t *s, int bits) {
    *s = (*s * JR_MULT + JR_ADD) & JR_MASK;
    return (int32_t)(int64_t)(*s >> (48 - bits));
}

int32_t oracle_jrandom_next_int(uint64_t *s) { return jr_next(s, 32); }

double oracle_jrandom_next_double(uint64_t *s) {
    const int64_t hi = jr_next(s, 26), lo = jr_next(s, 27);
    return (double)((hi << 27) + lo) * 0x1.0p-53;
}

static int first_max(const double *v, int n) {
    int idx = 0;
    double m = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > m) {
            m = v[i];
            idx = i;
        }
    return idx;
}

static const double *g_sort_probs;
static int by_prob_desc(const void *a, const void *b) {
    const int ia = *(const int *)a, ib = *(const int *)b;
    const double pa = g_sort_probs[ia], pb = g_sort_probs[ib];
    if (pa > pb) return -1;
    if (pa < pb) return 1;
    return ia < ib ? -1 : (ia > ib); /* equal probabilities keep index order (a stable sort) */
}

/* The categorical draw of sampleToken over final probabilities; *margin = distance from r to the
 * nearest boundary of the chosen index's interval (how close the draw came to another token). */
static int draw(const double *probs, int n, double r, double *margin) {
    double cumulative = 0.0;
    for (int i = 0; i < n; i++) {
        const double before = cumulative;
        cumulative += probs[i];
        if (r < cumulative) {
            if (margin) *margin = fmin(r - before, cumulative - r);
            return i;
        }
    }
    if (margin) *margin = fabs(r - cumulative);
    return n - 1;
}

int oracle_sample_token(const double *values, int n, double temperature, double top_p, uint64_t *rng,
                        double *r_out, double *margin) {
    if (temperature <= 0.0 || rng == NULL) return first_max(values, n);
    double *probs = malloc(sizeof(double) * (size_t)n);
    double max_logit = -INFINITY;
    for (int i = 0; i < n; i++) {
        probs[i] = values[i] / temperature;
        if (probs[i] > max_logit) max_logit = probs[i];
    }
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        probs[i] = exp(probs[i] - max_logit);
        sum += probs[i];
    }
    for (int i = 0; i < n; i++) probs[i] /= sum;
    if (top_p < 1.0) {
        int *idx = malloc(sizeof(int) * (size_t)n);
        for (int i = 0; i < n; i++) idx[i] = i;
        g_sort_probs = probs;
        qsort(idx, (size_t)n, sizeof(int), by_prob_desc);
        double cum = 0.0, top_sum = 0.0;
        int cutoff = n;
        for (int i = 0; i < n; i++) {
            cum += probs[idx[i]];
            top_sum += probs[idx[i]];
            if (cum >= top_p) {
                cutoff = i + 1;
                break;
            }
        }
        for (int i = cutoff; i < n; i++) probs[idx[i]] = 0.0;
        for (int i = 0; i < n; i++) probs[i] /= top_sum;
        free(idx);
    }
    const double r = oracle_jrandom_next_double(rng);
    if (r_out) *r_out = r;
    const int k = draw(probs, n, r, margin);
    free(probs);
    return k;
}

/* DistributionFeatures.softmax(x, subtractMax = true) in FP64 */
void oracle_softmax_ignore_zero(double *x, int n) {
    const double eps = 2.220446049250313e-16;
    double m = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > m) m = x[i];
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        const double d = (x[i] == 0.0) ? 0.0 : ((x[i] == m) ? eps : x[i] - m);
        x[i] = (d == 0.0) ? 0.0 : exp(d);
        sum += x[i];
    }
    for (int i = 0; i < n; i++) x[i] /= sum;
}

int oracle_model_sample(const double *logits, int n, double temperature, uint64_t *rng, double *r_out,
                        double *margin) {
    if (temperature == 0.0) return first_max(logits, n);
    double *x = malloc(sizeof(double) * (size_t)n);
    for (int i = 0; i < n; i++) x[i] = logits[i] / temperature;
    oracle_softmax_ignore_zero(x, n);
    const int k = oracle_sample_token(x, n, 1.0, 1.0, rng, r_out, margin);
    free(x);
    return k;
}
