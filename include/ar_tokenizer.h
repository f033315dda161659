/*
 * ar_tokenizer.h -- the Qwen3 byte-level BPE tokenizer on the host (no GPU needed).
 *
 * Replaces Qwen3Tokenizer (engine/ml/src/main/java/org/almostrealism/ml/qwen3/Qwen3Tokenizer.java)
 * with its base ByteLevelBPETokenizer, RegexPreTokenizer and ByteLevelEncoder
 * (engine/ml/src/main/java/org/almostrealism/ml/tokenization/).  Text crosses the boundary as
 * UTF-8 bytes (Java strings are UTF-16; the same code points either way).  Every function returns
 * AR_HIP_OK (0) or an AR_HIP_ERR_* code with a message in ar_hip_last_error().
 */
#ifndef AR_TOKENIZER_H
#define AR_TOKENIZER_H

#include <stddef.h>
#include <stdint.h>

#include "ar_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define AR_QWEN3_BOS_TOKEN 151643 /* Qwen3Tokenizer.BOS_TOKEN (also PAD_TOKEN) */
#define AR_QWEN3_EOS_TOKEN 151645 /* Qwen3Tokenizer.EOS_TOKEN */
#define AR_QWEN3_UNK_TOKEN 128244 /* Qwen3Tokenizer.UNK_TOKEN: id of a token missing from the vocabulary */

typedef struct ar_tokenizer ar_tokenizer;

/* Qwen3Tokenizer(String tokenizerPath) (Qwen3Tokenizer.java:99-148): the binary vocabulary
 * (little-endian int32 count, then per token float32 score, int32 byte length, UTF-8 bytes) and,
 * when the path names a directory part, the merges.txt beside it (loadMergesFromFile, :150-199:
 * "#" and blank lines skipped, "first second" split at the first space, a merge whose parts or
 * concatenation are not in the vocabulary is dropped but still takes its priority number).
 * Missing file -> AR_HIP_ERR_NOT_FOUND; truncated file -> AR_HIP_ERR_INVALID. */
int ar_hip_tokenizer_load(const char *tokenizer_path, ar_tokenizer **out);
/* Qwen3Tokenizer(String[] vocab, float[] vocabScores) (:201-217): no merges.  vocab[i] holds
 * lens[i] UTF-8 bytes (lens may be NULL for NUL-terminated strings). */
int ar_hip_tokenizer_from_vocab(const char *const *vocab, const int32_t *lens, const float *scores, int n,
                                ar_tokenizer **out);
/* Reads merges in the merges.txt format into an existing tokenizer, numbering priorities from 0. */
int ar_hip_tokenizer_load_merges(ar_tokenizer *t, const char *merges_path);
int ar_hip_tokenizer_destroy(ar_tokenizer *t);

/* getVocabSize; the number of merges kept; one vocabulary entry (UTF-8, valid until destroy). */
int ar_hip_tokenizer_vocab_size(const ar_tokenizer *t, int *n);
int ar_hip_tokenizer_merge_count(const ar_tokenizer *t, int *n);
int ar_hip_tokenizer_token(const ar_tokenizer *t, int id, const char **utf8, int *len, float *score);

/* Qwen3Tokenizer.encode(text, addBos, addEos) (:271-296) over ByteLevelBPETokenizer.encode
 * (ByteLevelBPETokenizer.java): pre-tokenisation with the reference's pattern, byte-level
 * mapping, BPE merging one adjacent pair at a time (the lowest priority, leftmost on ties), ids by
 * exact string lookup (AR_QWEN3_UNK_TOKEN when absent).  *count receives the number of ids; out
 * (capacity entries, may be NULL to ask for the count) receives them; a count above capacity
 * returns AR_HIP_ERR_INVALID with *count set.  Text that is not valid UTF-8 -> AR_HIP_ERR_INVALID. */
int ar_hip_tokenizer_encode(const ar_tokenizer *t, const char *text, int64_t text_len, int add_bos, int add_eos,
                            int32_t *out, int capacity, int *count);
/* ByteLevelBPETokenizer.decode: ids in range and not BOS/EOS/PAD/UNK are concatenated and mapped
 * back to bytes; malformed UTF-8 in the result becomes U+FFFD per maximal subpart, as Java's
 * decoder does.  *length receives the byte length (without a terminator); out (capacity bytes,
 * may be NULL) receives the bytes and a terminating NUL when there is room.  A character outside
 * the byte-level alphabet -> AR_HIP_ERR_INVALID (IllegalArgumentException in ByteLevelEncoder). */
int ar_hip_tokenizer_decode(const ar_tokenizer *t, const int32_t *ids, int n, char *out, int64_t capacity,
                            int64_t *length);
/* RegexPreTokenizer.preTokenize (RegexPreTokenizer.java:89-116): the segments of `text`, as
 * byte offsets: segment k is [offsets[2k], offsets[2k+1]).  Same buffer rules as encode (capacity
 * counts segments). */
int ar_hip_tokenizer_pretokenize(const char *text, int64_t text_len, int64_t *offsets, int capacity, int *count);

#ifdef __cplusplus
}
#endif

#endif /* AR_TOKENIZER_H */
