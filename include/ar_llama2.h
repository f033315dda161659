/*
 * ar_llama2.h -- the Llama2 model family on the HIP decoder: llama2.c checkpoints, their
 * configuration header, and the score-driven BPE tokenizer that goes with them.
 *
 * Replaces, on the reference side (engine/ml/src/main/java/org/almostrealism/ml/):
 *   TransformerConfig(ByteBuffer)   TransformerConfig.java:69-80   -> ar_hip_llama2_parse_config
 *   Llama2Weights(config, buffer)   llama2/Llama2Weights.java:90-113 -> ar_hip_llama2_open / _tensor
 *   Llama2.model(...)               llama2/Llama2.java:173-201     -> ar_hip_llama2_create_model
 *   tokenizer read in Llama2(...)   llama2/Llama2.java:130-146     -> ar_hip_bpe_load
 *   BPE.lookup / BPE.encode         BPE.java:33-101                -> ar_hip_bpe_lookup / _encode
 *
 * The model built here is an ar_qwen3 decoder handle (include/ar_hip.h): the reference builds
 * Llama2 from the same AttentionFeatures.transformer blocks as Qwen3 (AttentionFeatures.java:
 * 1607-1618 -> 1688-1708), with no QK-norm, no biases, RMSNorm eps 1e-5 and the checkpoint's
 * RoPE table, so every token-loop, sampling and prefill entry point of ar_hip.h applies to it.
 *
 * Status codes, thread-local error text and dtype constants are those of ar_hip.h.
 */
#ifndef AR_LLAMA2_H
#define AR_LLAMA2_H

#include <stddef.h>
#include <stdint.h>

#include "ar_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* TransformerConfig as read from a checkpoint header (TransformerConfig.java:69-80): seven
 * little-endian int32 (dim, hiddenDim, layerCount, headCount, kvHeadCount, vocabSize, seqLen);
 * a negative vocabSize means the classifier is stored separately (sharedWeights false);
 * headSize = dim / headCount. */
typedef struct ar_llama2_cfg {
    int32_t dim;
    int32_t hidden_dim;
    int32_t layer_count;
    int32_t head_count;
    int32_t kv_head_count; /* read but not used by the model: Llama2Weights reads wk / wv as dim x dim
                              and Llama2.model builds heads == kvHeads (Llama2.java:181-192) */
    int32_t vocab_size;    /* |header value| */
    int32_t seq_len;
    int32_t shared_weights;
    int32_t head_size;
} ar_llama2_cfg;

#define AR_LLAMA2_HEADER_BYTES 28

/* Parses a checkpoint header from n >= 28 bytes. */
int ar_hip_llama2_parse_config(const void *header, size_t n, ar_llama2_cfg *out);

/* A mapped llama2.c checkpoint: header + fp32 tensors in Llama2Weights order (tokenEmbeddings,
 * rmsAttWeights, wq, wk, wv, wo, rmsFfn, w1, w2, w3, rmsFinalWeight, the RoPE real and imaginary
 * planes (seqLen x headSize/2 each), then wcls unless shared).  A file shorter than that layout is
 * rejected (the reference fails reading past the end); bytes after it are ignored. */
typedef struct ar_llama2_ckpt ar_llama2_ckpt;

int ar_hip_llama2_open(const char *path, ar_llama2_ckpt **out);
int ar_hip_llama2_close(ar_llama2_ckpt *ck);
int ar_hip_llama2_config(const ar_llama2_ckpt *ck, ar_llama2_cfg *out);

/* A whole tensor by its Llama2Weights field name ("tokenEmbeddings", "rmsAttWeights", "wq", "wk",
 * "wv", "wo", "rmsFfn", "w1", "w2", "w3", "rmsFinalWeight", "freqCis", "wcls"); layer-stacked
 * tensors are returned whole.  freqCis is (seqLen, headSize/2, 2): the two planes interleaved
 * element by element as Llama2Weights.stage does with two sources (Llama2Weights.java:108-109,
 * 143-173); wcls is tokenEmbeddings when the weights are shared.  The pointer stays valid until
 * ar_hip_llama2_close. */
int ar_hip_llama2_tensor(const ar_llama2_ckpt *ck, const char *name, const float **data, int64_t *n_elems);

/* Llama2.model (Llama2.java:173-201): a decoder on ctx with the checkpoint's weights (uploaded from
 * the mapping), kv_heads = heads, eps 1e-5 (the transformer overload of AttentionFeatures.java:
 * 1607-1618 and the default of NormalizationLayerFeatures.java:557-561), the checkpoint's freqCis as
 * the RoPE table and a KV cache of seqLen positions.  max_batch 1..8 sequences; weight_dtype
 * AR_DTYPE_F32 (the checkpoint's values) or AR_DTYPE_BF16 (rounded once on upload); kv_dtype
 * AR_DTYPE_F32 or AR_DTYPE_F16.  The model is finalized and reset; destroy it with
 * ar_hip_qwen3_destroy.  The checkpoint may be closed afterwards. */
int ar_hip_llama2_create_model(ar_hip_ctx *ctx, const ar_llama2_ckpt *ck, int max_batch, int weight_dtype,
                               int kv_dtype, ar_qwen3 **out);

/* ---- the score-driven BPE tokenizer of llama2.c checkpoints ------------------------------ */

typedef struct ar_bpe ar_bpe;

/* Reads tokenizer.bin as the Llama2 constructor does (Llama2.java:130-146): an int32 max token
 * length (skipped), then vocab_size entries of (float32 score, int32 length, bytes); each entry's
 * bytes are decoded as UTF-8 with U+FFFD for malformed input (new String(bytes)). */
int ar_hip_bpe_load(const char *path, int vocab_size, ar_bpe **out);
/* The same from memory: n UTF-8 strings and their scores. */
int ar_hip_bpe_create(const char *const *vocab, const float *scores, int n, ar_bpe **out);
int ar_hip_bpe_destroy(ar_bpe *t);
int ar_hip_bpe_vocab_size(const ar_bpe *t, int *n);
/* vocab[id] as UTF-8 (pointer valid until destroy) and its score. */
int ar_hip_bpe_token(const ar_bpe *t, int id, const char **utf8, int *len, float *score);
/* BPE.lookup (BPE.java:33-41): the first id whose string equals the text, or -1. */
int ar_hip_bpe_lookup(const ar_bpe *t, const char *utf8, int len, int *id);
/* BPE.encode (BPE.java:57-101): every UTF-16 unit of the text becomes its one-character
 * token (a unit with no such token is an error, as the reference throws); then, while some
 * adjacent pair concatenates to a token, the pair whose token has the highest score (the first
 * pair on ties, scores compared against a floor of -1e10) is merged.  At most cap tokens. */
int ar_hip_bpe_encode(const ar_bpe *t, const char *utf8, int len, int32_t *tokens, int cap, int *n);

#ifdef __cplusplus
}
#endif

#endif /* AR_LLAMA2_H */
