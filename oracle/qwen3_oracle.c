/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the Qwen3 decode hot path.
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker / CPU baseline; never part of the product library.
 *
 * Instantiates qwen3_oracle_impl.h at the reference's two context precisions.
 * Built by oracle/Makefile with -ffp-contract=off so no multiply-add is fused.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct oracle_cfg {
    int32_t dim, n_layers, n_heads, n_kv_heads, head_dim, ffn_dim, vocab, seq_len;
    int32_t qk_norm_mode;  /* 0: one RMS over the whole q / k vector (reference), 1: per head (HF) */
    int32_t full_seq_mask; /* 1: score all seq_len cache rows with the -10000 mask (reference form) */
    int32_t tied;          /* 1: logits use the embedding matrix (Qwen3.java:344-345) */
    int32_t reserved;
    double rope_theta, eps, qk_eps;
} oracle_cfg;

int oracle_cfg_size(void) { return (int)sizeof(oracle_cfg); }

#ifdef _OPENMP
#include <omp.h>
#endif
/* Thread count of the oracle's OpenMP loops (the reference's CPU pool size,
 * KernelPreferences.getCpuParallelism = max(2, nproc/2), base/code/.../kernel/KernelPreferences.java:68-71). */
void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int oracle_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

#define REAL double
#define SFX _f64
#define IS_F32 0
#include "qwen3_oracle_impl.h"
#undef REAL
#undef SFX
#undef IS_F32

#define REAL float
#define SFX _f32
#define IS_F32 1
#include "qwen3_oracle_impl.h"
#undef REAL
#undef SFX
#undef IS_F32
