/*
 * Seeded synthetic inputs (weights, prompt ids) for the Qwen3 hot path.
 *
 * Counter-based: element i of stream s under seed k is a pure function of (k, s, i), so
 * the values do not depend on thread count, chunking or the order tensors are made in.
 *   z = splitmix64(splitmix64(k ^ s*C1) + i*C2)
 *   u1 = ((z >> 32) + 0.5) / 2^32 in (0,1),  u2 = (z & 0xffffffff) / 2^32 in [0,1)
 *   normal = sqrt(-2 ln u1) * cos(2 pi u2)            (Box-Muller, one draw per counter)
 * evaluated in double with the host libm and rounded to float once.  bf16 rounding, when
 * asked for, is round-to-nearest-even on the float bits.
 */
#include <math.h>
#include <stdint.h>

static inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static inline float bf16_rne(float f) {
    union { float f; uint32_t u; } v = {f};
    uint32_t u = v.u;
    if ((u & 0x7F800000u) != 0x7F800000u) u += 0x7FFFu + ((u >> 16) & 1u);
    v.u = u & 0xFFFF0000u;
    return v.f;
}

void ar_synth_normal(uint64_t seed, uint64_t stream, double mean, double std, float *out, int64_t n,
                     int bf16) {
    uint64_t base = splitmix64(seed ^ (stream * 0xD1B54A32D192ED03ull));
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        uint64_t z = splitmix64(base + (uint64_t)i * 0x9E3779B97F4A7C15ull);
        double u1 = ((double)(z >> 32) + 0.5) * (1.0 / 4294967296.0);
        double u2 = (double)(z & 0xFFFFFFFFull) * (1.0 / 4294967296.0);
        double g = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        float f = (float)(mean + std * g);
        out[i] = bf16 ? bf16_rne(f) : f;
    }
}

/* Uniform integers in [0, bound) by 128-bit multiply-shift (Lemire) of the counter hash. */
void ar_synth_uniform_ids(uint64_t seed, uint64_t stream, int32_t bound, int32_t *out, int64_t n) {
    uint64_t base = splitmix64(seed ^ (stream * 0xD1B54A32D192ED03ull));
    for (int64_t i = 0; i < n; i++) {
        uint64_t z = splitmix64(base + (uint64_t)i * 0x9E3779B97F4A7C15ull);
        out[i] = (int32_t)(((unsigned __int128)(z >> 32) * (uint64_t)bound) >> 32);
    }
}

void ar_synth_bf16_round(float *data, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) data[i] = bf16_rne(data[i]);
}
