/*
 * ar_hip.h -- C-ABI of the MI355X (gfx950) HIP backend for the Qwen3 decode/prefill path.
 *
 * Plain C: opaque handles, POD structs, raw pointers and sizes.  Every function returns
 * AR_HIP_OK (0) or an error code; ar_hip_last_error() gives the calling thread's message.
 * A JNI bridge maps `long` handles to these pointers and turns a non-zero code into
 * HardwareException.
 *
 * Reference interfaces each group replaces are cited as path:line under
 * almostrealism/common.
 */
#ifndef AR_HIP_H
#define AR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ----------------------------------------------------------------- */
#define AR_HIP_OK 0
#define AR_HIP_ERR_INVALID 1   /* bad argument (IllegalArgumentException in the reference) */
#define AR_HIP_ERR_HIP 2       /* HIP runtime error (HardwareException) */
#define AR_HIP_ERR_NO_DEVICE 3 /* no usable GPU: driver init fails (Hardware.java:771-777) */
#define AR_HIP_ERR_STATE 4     /* call out of order (missing weight, position past capacity) */
#define AR_HIP_ERR_NOT_FOUND 5 /* unknown weight key / allocation not owned by this provider */

/* ---- element types ---------------------------------------------------------------- */
#define AR_DTYPE_F32 0
#define AR_DTYPE_BF16 1
#define AR_DTYPE_F16 2   /* KV-cache storage option (ar_qwen3_cfg.kv_dtype) */

/* ---- QK-norm grouping ------------------------------------------------------------- */
#define AR_QK_NORM_WHOLE 0    /* one RMS over the whole q / k vector (AttentionFeatures.java:840-845, :886-891) */
#define AR_QK_NORM_PER_HEAD 1 /* one RMS per head (HF Qwen3) */

typedef struct ar_hip_ctx ar_hip_ctx;
typedef struct ar_qwen3 ar_qwen3;

/* Thread-local message for the last failing call on this thread ("" if none). */
const char *ar_hip_last_error(void);
/* Library version string. */
const char *ar_hip_version(void);

/* ---- data context / compute context ------------------------------------------------
 * Replaces DataContext.init/destroy/getComputeContexts
 * (base/code/src/main/java/io/almostrealism/code/DataContext.java:81-88) and
 * ComputeContext (base/code/src/main/java/io/almostrealism/code/ComputeContext.java:89,133)
 * for the HIP driver: one context per GPU, one in-order HIP stream per context. */
int ar_hip_device_count(int *count);
/* device < 0 selects the device the environment variable AR_HIP_DEVICE names (default 0), as the
 * reference selects its hardware from AR_* variables (Hardware.java:526,684 via SystemUtils).
 * AR_HIP_LOG=1 additionally writes every error message to stderr as it is set. */
int ar_hip_init(int device, ar_hip_ctx **out);
int ar_hip_destroy(ar_hip_ctx *ctx);
int ar_hip_synchronize(ar_hip_ctx *ctx);
/* Number of compute units and HBM bytes of the context's device. */
int ar_hip_device_info(ar_hip_ctx *ctx, int *num_cus, size_t *hbm_bytes, char *name, int name_len);

/* ---- memory provider -----------------------------------------------------------------
 * Replaces MemoryProvider.allocate / deallocate / setMem / getMem
 * (base/code/src/main/java/io/almostrealism/code/MemoryProvider.java:60,70,158,188) and the
 * JNI provider's malloc/free (base/hardware/src/main/java/org/almostrealism/nio/NativeMemoryProvider.java).
 * Sizes are bytes; copies are ordered on the context's stream and complete on return. */
int ar_hip_alloc(ar_hip_ctx *ctx, size_t bytes, void **device_ptr);
int ar_hip_free(ar_hip_ctx *ctx, void *device_ptr);
int ar_hip_host_alloc(ar_hip_ctx *ctx, size_t bytes, void **pinned_ptr); /* pinned staging */
int ar_hip_host_free(ar_hip_ctx *ctx, void *pinned_ptr);
int ar_hip_memcpy_h2d(ar_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int ar_hip_memcpy_d2h(ar_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int ar_hip_memcpy_d2d(ar_hip_ctx *ctx, void *dst, const void *src, size_t bytes);
int ar_hip_memset(ar_hip_ctx *ctx, void *dst, int value, size_t bytes);
/* Bytes currently held by the provider. */
int ar_hip_allocated_bytes(ar_hip_ctx *ctx, size_t *bytes);

/* ---- operators (device pointers, fp32 activations) --------------------------------
 * Each runs on the context's stream and returns after enqueueing; call
 * ar_hip_synchronize before reading results on the host. */

/* rmsnorm over the last axis: y = (w * x) / sqrt(mean(x^2) + eps), `rows` vectors of n.
 * NormalizationLayerFeatures.rmsnorm (domain/graph/.../layers/NormalizationLayerFeatures.java:574-604). */
int ar_hip_rmsnorm(ar_hip_ctx *ctx, const float *x, const float *w, float *y, int rows, int n, float eps);

/* dense: y[b] = W x[b] (+ bias) for W (rows x cols) row-major, fp32 or bf16, batch <= 8.
 * If norm_w is non-null the input is first RMS-normalised with that gain (fused prologue).
 * LayerFeatures.dense (domain/graph/.../layers/LayerFeatures.java:785-830) ->
 * MatrixFeatures.matmul (compute/algebra/.../MatrixFeatures.java:182-337). */
int ar_hip_dense(ar_hip_ctx *ctx, const void *W, int w_dtype, const float *bias, const float *x,
                 const float *norm_w, float eps, float *y, int rows, int cols, int batch);

/* SwiGLU feed-forward hidden: y[b] = (Wup h) * silu(Wgate h), h = rmsnorm(x[b]; norm_w) when
 * norm_w is non-null.  FeedForwardFeatures.feedForward (engine/ml/.../FeedForwardFeatures.java:140-157),
 * silu (domain/graph/.../ActivationFeatures.java:263-265). */
int ar_hip_swiglu(ar_hip_ctx *ctx, const void *W_gate, const void *W_up, int w_dtype, const float *x,
                  const float *norm_w, float eps, float *y, int rows, int cols, int batch);

/* Split-half RoPE in place on `rows` flat vectors of heads*head_dim at position pos.
 * reshapeToSplitHalfRope -> ropeRotation -> reshapeFromSplitHalfRope
 * (engine/ml/.../AttentionFeatures.java:195-237; engine/ml/.../RotationFeatures.java:124-208). */
int ar_hip_rope(ar_hip_ctx *ctx, float *x, int heads, int head_dim, int pos, double theta, int rows);

/* First index of the maximum of each of `rows` vectors of n (ties -> lowest index).
 * AggregationFeatures.indexOfMax (compute/algebra/.../AggregationFeatures.java:111-121). */
int ar_hip_index_of_max(ar_hip_ctx *ctx, const float *x, int rows, int n, int32_t *out_device);

/* Decode-step GQA attention block core for one position: QK-norm of the raw q and k
 * projections, split-half RoPE, cache write of k and v at row `pos`, causal attention over
 * rows 0..pos with a split-context online softmax.
 *   q (heads*hd), k, v (kv_heads*hd): raw projections (fp32, device)
 *   k_cache, v_cache: (kv_heads, max_seq, hd) fp32, device; row pos is overwritten
 *   out: (heads*hd) fp32, device
 * AttentionFeatures.attentionImpl (engine/ml/.../AttentionFeatures.java:785-929): the block
 * between the projections and the o_proj dense. */
int ar_hip_attention_decode(ar_hip_ctx *ctx, const float *q, const float *k, const float *v,
                            const float *q_norm, const float *k_norm, float qk_eps, int qk_norm_mode,
                            float *k_cache, float *v_cache, int max_seq, int pos, int heads,
                            int kv_heads, int head_dim, double rope_theta, float *out);

/* ar_hip_attention_decode without any allocation: no counterpart in the reference.  For callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, kernels and results; the split partials go to a fixed
 * per-device scratch array of 2^18 floats (1 MiB, held by each GPU the library runs on until the
 * process ends) instead of memory the library allocates.  Rejects (AR_HIP_ERR_INVALID) shapes whose
 * partials, heads x splits x (head_dim + 2) floats, exceed it (16 heads x hd 128 caches up to
 * ~32k rows fit).  Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (several streams, or several host threads) race. */
int ar_hip_attention_decode_noalloc(ar_hip_ctx *ctx, const float *q, const float *k, const float *v,
                                    const float *q_norm, const float *k_norm, float qk_eps, int qk_norm_mode,
                                    float *k_cache, float *v_cache, int max_seq, int pos, int heads,
                                    int kv_heads, int head_dim, double rope_theta, float *out);

/* Token sampling, one draw per row of `rows` logit vectors of n (device, fp32), in double:
 *   AR_SAMPLE_TOKEN: AutoregressiveModel.sampleToken(logits, n, temperature, top_p, random)
 *     (engine/ml/.../AutoregressiveModel.java:323-386): softmax of logits / temperature, nucleus
 *     filtering when top_p < 1 (shortest prefix in descending order, ties by index, whose sum
 *     reaches top_p; renormalised), then the first index whose running sum exceeds
 *     r = random.nextDouble();
 *   AR_SAMPLE_MODEL: the sample function AutoregressiveModel.of installs (:413-425): logits /
 *     temperature, DistributionFeatures.softmax (compute/stats/.../DistributionFeatures.java:129-141;
 *     a value equal to 0 stays 0), then sampleToken(probabilities, n, 1.0, 1.0, random); top_p unused.
 * rng_state (device, rows entries) holds java.util.Random states, (seed ^ 0x5DEECE66D) mod 2^48 for
 * new Random(seed), and is advanced by the draw; out (device) receives the indices.  Greedy
 * temperatures (sampleToken: <= 0; the model's function: == 0) take the first maximum
 * (AggregationFeatures.indexOfMax) and draw nothing, as the reference does. */
#define AR_SAMPLE_MODEL 0
#define AR_SAMPLE_TOKEN 1
int ar_hip_sample(ar_hip_ctx *ctx, const float *logits, int rows, int n, int mode, double temperature, double top_p,
                  uint64_t *rng_state, int32_t *out);

/* Multi-token projection on the MFMA units: C[M x N] = A[M x K] . W[N x K]^T, A and W bf16
 * (raw uint16 bits, K contiguous), fp32 accumulation.  N % 128 == 0, K % 64 == 0.
 *   AR_GEMM_STORE:    C (fp32, [M][N]) = result (+ bias[N] if non-null)
 *   AR_GEMM_RESIDUAL: C += result
 *   AR_GEMM_SWIGLU:   O (bf16, [M][N]) = (A.W2^T) * silu(A.W^T)
 * The stacked-row form of LayerFeatures.dense (domain/graph/.../LayerFeatures.java:785-830) for
 * prompt rows, which the reference feeds one per step (AutoregressiveModel.java:295-308). */
#define AR_GEMM_STORE 0
#define AR_GEMM_RESIDUAL 1
#define AR_GEMM_SWIGLU 2
int ar_hip_gemm_bf16(ar_hip_ctx *ctx, const uint16_t *A, const uint16_t *W, const uint16_t *W2, const float *bias,
                     float *C, uint16_t *O, int M, int N, int K, int epilogue);
/* The same product with fp32 operands and accumulation on the fp32 MFMA units
 * (v_mfma_f32_32x32x2_f32), the prompt projections of an fp32-weight model: C (fp32, [M][N]);
 * AR_GEMM_SWIGLU writes (A.W2^T) * silu(A.W^T) to C in fp32.  N % 64 == 0, K % 32 == 0. */
int ar_hip_gemm_f32(ar_hip_ctx *ctx, const float *A, const float *W, const float *W2, const float *bias, float *C,
                    int M, int N, int K, int epilogue);

/* ---- Qwen3 model -------------------------------------------------------------------
 * Replaces Qwen3.model + CompiledModel.forward + AutoregressiveModel
 * (engine/ml/.../qwen3/Qwen3.java:334-415, domain/graph/.../model/CompiledModel.java:189-197,
 * engine/ml/.../AutoregressiveModel.java:295-308,405-434) with one fused decode-step plan. */
typedef struct ar_qwen3_cfg {
    int32_t dim;           /* TransformerConfig.dim */
    int32_t hidden_dim;    /* FFN width */
    int32_t layer_count;
    int32_t head_count;
    int32_t kv_head_count;
    int32_t head_size;     /* explicit; the reference derives dim/headCount (TransformerConfig.java:79) */
    int32_t vocab_size;
    int32_t seq_len;       /* KV-cache capacity in positions */
    int32_t max_batch;     /* independent sequences decoded together (1..8) */
    int32_t weight_dtype;  /* AR_DTYPE_F32 or AR_DTYPE_BF16 (fp32 accumulation either way) */
    int32_t qk_norm_mode;  /* AR_QK_NORM_WHOLE (reference) or AR_QK_NORM_PER_HEAD */
    int32_t shared_weights;/* tied embeddings: logits use model.embed_tokens.weight */
    int32_t qkv_bias;      /* q/k/v projection biases present */
    int32_t kv_dtype;      /* KV-cache storage: AR_DTYPE_F32 (0, default: the reference keeps the cache at
                              the context precision) or AR_DTYPE_F16 (half the per-step cache bytes of
                              long-context decode; scores and softmax stay fp32) */
    double rope_theta;
    double epsilon;        /* RMSNorm eps (1e-6, Qwen3.java:397,402); QK-norm uses the same */
} ar_qwen3_cfg;

int ar_hip_qwen3_create(ar_hip_ctx *ctx, const ar_qwen3_cfg *cfg, ar_qwen3 **out);
int ar_hip_qwen3_destroy(ar_qwen3 *m);

/* Uploads one tensor by its HF state-dict key, as StateDictionary.get supplies them to
 * Qwen3.model (engine/ml/.../StateDictionary.java; Qwen3.java:338-384).  src is host memory
 * holding n_elems values of src_dtype in the HF (out, in) row-major layout.
 * Key AR_ROPE_TABLE_KEY takes a RoPE table of fp32 (cos, sin) pairs, (positions >= seq_len,
 * head_size / 2, 2), that replaces the one computed from rope_theta: the freqCis a model built
 * from a checkpoint supplies (Llama2Weights.java freqCis, Llama2.java model()). */
#define AR_ROPE_TABLE_KEY "freq_cis"
int ar_hip_qwen3_set_weight(ar_qwen3 *m, const char *key, const void *src, int src_dtype, int64_t n_elems);
/* Checks every required tensor is present and builds the decode plan. */
int ar_hip_qwen3_finalize(ar_qwen3 *m);

/* AutoregressiveModel.reset (AutoregressiveModel.java:203-207): position 0. */
int ar_hip_qwen3_reset(ar_qwen3 *m);
/* AutoregressiveModel.setPrompt (AutoregressiveModel.java:272-275): prompt ids for sequence `seq`.
 * All sequences of a batch share one prompt length: a prompt whose length differs from the
 * batch's current one becomes the new length and drops the other sequences' prompts, which must
 * then be set again (at that length) before the next step.  reset() keeps the prompts, as the
 * reference's reset keeps its prompt. */
int ar_hip_qwen3_set_prompt(ar_qwen3 *m, int seq, const int32_t *ids, int n);
/* AutoregressiveModel.next (AutoregressiveModel.java:295-308) for every sequence: feeds the
 * prompt token or the greedy choice from the previous step's logits, runs one forward pass
 * and advances.  tokens_out[b] receives the token fed at this step; logits_out (optional,
 * batch x vocab floats, host) receives this step's logits. */
int ar_hip_qwen3_next(ar_qwen3 *m, int32_t *tokens_out, float *logits_out);
/* `steps` calls of next() enqueued back to back without host synchronisation (the token
 * loop stays on the device); tokens_out is batch x steps (row-major by sequence). */
int ar_hip_qwen3_run(ar_qwen3 *m, int steps, int32_t *tokens_out);
/* Whole-prompt prefill from position 0: the prompt rows of every sequence run together (bf16
 * weights: fp16 MFMA GEMMs + causal flash attention; fp32 weights: fp32 MFMA GEMMs + fp32 causal
 * attention, or the decode step per token when dim, the q+k+v rows or the FFN width is not a
 * multiple of 64).  Leaves
 * the model exactly where prompt_len calls of next() would: position = prompt length, KV cache
 * rows 0..prompt_len-1 written, and the next next() feeds the greedy token of the last prompt
 * row.  logits_out (optional, batch x vocab, host) receives the last prompt row's logits.
 * AutoregressiveModel.next over the prompt (AutoregressiveModel.java:295-299), batched.
 * The bf16 path stores its MFMA operands as fp16; when any value stored that way (a weight, a
 * normalised row, a rotated query or key, a value row, a SwiGLU output) lies outside the fp16 range
 * (|v| >= 65520), the batched pass is discarded before the logits and the sampler run, and the
 * prompt goes through the decode step instead (fp32 activations; slower, same result as next()). */
int ar_hip_qwen3_prefill(ar_qwen3 *m, float *logits_out);
/* Number of ar_hip_qwen3_prefill calls on this model that went through the decode step (fp32
 * weights, or a value outside the fp16 range on the bf16 path). */
int ar_hip_qwen3_prefill_by_steps(ar_qwen3 *m, int *count);
/* Which kernels run the bf16 path's prefill products (the QKV, O, gate/up and down projections of
 * every prompt row).  No counterpart in the reference (its prompt goes through the decode step, see
 * above); a throughput option only.  AR_PREFILL_GEMM_ROCBLAS (default): rocBLAS gemm_ex on the fp16
 * operands with fp32 accumulation, the residual adds as beta = 1 on the fp32 rows, gate/up as one
 * fp16 product over the stacked gate and up rows and a SwiGLU pass (a QKV projection with a bias
 * stays on the library's kernel).  AR_PREFILL_GEMM_OWN: the library's MFMA kernels (gemm.hip, the
 * epilogues fused, O and down split over k where that fills more CUs).  Both round to the same
 * fp16 operands; results agree within float rounding.  Rejects other values (AR_HIP_ERR_INVALID). */
#define AR_PREFILL_GEMM_OWN 0
#define AR_PREFILL_GEMM_ROCBLAS 1
int ar_hip_qwen3_prefill_gemm(ar_qwen3 *m, int backend);
int ar_hip_qwen3_prefill_gemm_backend(ar_qwen3 *m, int *backend);
/* Token selection of next / run / prefill.  Default: AR_SAMPLE_MODEL at temperature 0, i.e. greedy,
 * as a new AutoregressiveModel starts.  AR_SAMPLE_MODEL with another temperature is
 * AutoregressiveModel.setTemperature (AutoregressiveModel.java:258-260) with the sample function of
 * AutoregressiveModel.of; AR_SAMPLE_TOKEN applies sampleToken(logits, V, temperature, top_p, random)
 * instead (see ar_hip_sample).  seeds (host, max_batch values, or NULL to keep the generators) seed
 * one java.util.Random per sequence; a draw happens only for steps past the prompt, so each
 * sequence's draws match a reference model driven with new Random(seed).  Tokens sampled on the
 * device are fed without a host round trip, like the greedy ones. */
int ar_hip_qwen3_set_sampling(ar_qwen3 *m, int mode, double temperature, double top_p, const int64_t *seeds);
/* Current position (AutoregressiveModel.getCurrentStep). */
int ar_hip_qwen3_position(ar_qwen3 *m, int *pos);
/* Residual-stream vector after the last step (batch x dim floats, host) for activation checks. */
int ar_hip_qwen3_hidden(ar_qwen3 *m, float *out);

/* Kernel timing probe: when enabled, HIP events bracket every launch of kernel class `which`
 * (AR_KT_*) on the model's stream; ar_hip_qwen3_kernel_time returns the summed milliseconds and
 * the launch count since the last enable. */
#define AR_KT_NONE 0
#define AR_KT_LOGITS 1      /* final RMSNorm + logits GEMV + argmax */
#define AR_KT_GATE_UP 2     /* RMSNorm + gate/up GEMV + SwiGLU */
#define AR_KT_QKV 3
#define AR_KT_ATTENTION 4
#define AR_KT_DOWN 5
#define AR_KT_O 6
#define AR_KT_LAYERS 7      /* the persistent decode kernel (layers + logits of the step in one launch) */
/* Timing one of the classes 1..6 runs the step as separate launches; AR_KT_LAYERS times the
 * persistent kernel when it runs the step (ar_hip_qwen3_persistent). */
int ar_hip_qwen3_kernel_timing(ar_qwen3 *m, int which);
int ar_hip_qwen3_kernel_time(ar_qwen3 *m, double *ms, int *launches);
/* Loop probe of one decode kernel class (AR_KT_QKV, AR_KT_O, AR_KT_GATE_UP, AR_KT_DOWN or
 * AR_KT_LOGITS): `reps` launches of that class exactly as the decode step issues them, cycling
 * through the layers' weights (so the weights stream from HBM as in the step), captured into one
 * HIP graph and replayed between two events (with graphs off, ar_hip_qwen3_use_graph(m, 0): the
 * launches back to back between the two events); *us_per_launch receives the average launch
 * duration (no event inside any dispatch).  A measurement aid of the benchmark, like
 * ar_hip_qwen3_kernel_timing: the launches overwrite the step's activations (the residual classes
 * add into the residual stream), so the model must be reset before its next step. */
int ar_hip_qwen3_kernel_loop(ar_qwen3 *m, int which, int reps, double *us_per_launch);
/* Use a captured HIP graph per decode step (1, default) or plain launches (0). */
int ar_hip_qwen3_use_graph(ar_qwen3 *m, int enable);
/* Fragment-ordered decode GEMVs.  For batches of 3..8 with bf16 weights (and dims that split into
 * 16 x 32 fragments, at least one per wavefront of a two-wavefront-per-CU grid), finalize also stores
 * each layer's O, gate/up and down matrices in MFMA fragment order (16 x 32 blocks of 1 KB; as many
 * bytes again as those weights), and those projections of the decode step read that copy, split
 * evenly over every wavefront of the GPU, instead of the row-major weights; the O projection then
 * also publishes per-16-row sums of squares of the residual stream for the gate/up RMSNorm.  No
 * counterpart in the reference (a weight layout of this backend); results match the row-major
 * GEMVs within float rounding.  enable 1 (default) or 0; ar_hip_qwen3_fragment_gemv reports whether
 * the steps use it. */
int ar_hip_qwen3_use_fragment_gemv(ar_qwen3 *m, int enable);
int ar_hip_qwen3_fragment_gemv(ar_qwen3 *m, int *active);
/* Persistent decode step.  For batch 1 with an fp32 or fp16 KV cache, on the instantiated shapes
 *   dim 1024 / FFN 3072 / 16 Q, 8 KV heads / head size 128 with fp32 weights (Qwen3-0.6B),
 *   dim 2048 / FFN 6144 / 16 Q, 8 KV heads / head size 128 with bf16 weights (Qwen3-1.7B), and
 *   dim 768 / FFN 2048 / 12 Q = KV heads / head size 64 with fp32 weights (llama2.c stories110M),
 * on a device that holds one 512-thread block per CU on 256 CUs at once, the layers and the logits of
 * each decode step run as one launch whose stages exchange data through device-scope words tagged
 * with an epoch, instead of five launches per layer and one for the logits; the step-begin kernel
 * stays separate, and the two launches are enqueued directly (a graph replay of them measured
 * slower).  No counterpart in the reference (its backend runs the compiled operation list); a
 * throughput option only: results match the multi-launch step within float rounding.  enable 1
 * (default) or 0; ar_hip_qwen3_persistent reports whether the next steps use it.
 * The launch needs every block resident at once.  If another kernel or process holds CUs, the
 * blocks that run abandon their waits after a bounded number of polls (about 0.3 s) and the launch
 * drains with invalid results; ar_hip_qwen3_next / run then recompute the steps of that call as
 * separate launches before returning (same tokens, logits and sampler draws as an undisturbed call)
 * and switch the model to separate launches (ar_hip_qwen3_persistent reports 0) until
 * ar_hip_qwen3_use_persistent(m, 1). */
int ar_hip_qwen3_use_persistent(ar_qwen3 *m, int enable);
int ar_hip_qwen3_persistent(ar_qwen3 *m, int *active);
/* Steps recomputed as separate launches after a timed-out persistent launch, over the model's life. */
int ar_hip_qwen3_persistent_recomputed(ar_qwen3 *m, int *steps);
/* Polls of one cross-block wait of the persistent kernel before it is abandoned (0: the default,
 * 2^18).  A test and diagnostic knob: a small limit makes the waits time out while every block of the
 * launch still runs to its end, which exercises the recompute above without any other load on the
 * device. */
int ar_hip_qwen3_persistent_wait_limit(ar_qwen3 *m, unsigned polls);

/* Debug pointer check.  With AR_HIP_CHECK_PTRS=1 in the environment (read once per process), the
 * decode-path launches (step begin, GEMVs, attention + split combine, persistent decode step) first
 * check every device pointer argument, with the extent its kernel reads or writes, against the HIP
 * allocation holding it (hipMemGetAddressRange), and refuse the launch with AR_HIP_ERR_INVALID when
 * a range leaves its allocation.  *checked receives the number of ranges checked so far in the
 * process (0 while the flag is off).  No counterpart in the reference (its generated C has no
 * error channel); a diagnostic only. */
int ar_hip_pointer_checks(unsigned long long *checked);

#ifdef __cplusplus
}
#endif

#endif /* AR_HIP_H */
