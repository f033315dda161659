/*
 * ar_state_dict.h -- weight I/O in the reference's protobuf format (host only, no GPU needed).
 *
 * The reference stores model weights as serialized `CollectionLibraryData` messages
 * (engine/ml/src/main/proto/collections.proto:1-27): a list of (key, CollectionData) entries,
 * CollectionData = { TraversalPolicyData{dims, traversal_axis}, repeated double data,
 * repeated float data_32 }.  A weights directory holds several such files (one per layer
 * group, engine/ml/qwen/tools/extract_qwen3_weights.py:108-170), read by StateDictionary
 * (engine/ml/src/main/java/org/almostrealism/ml/StateDictionary.java).
 *
 * This is a self-contained reader/writer of that wire format: files are memory-mapped and
 * packed fp32 payloads are handed to the device upload without a host copy.  Every function
 * returns AR_HIP_OK (0) or an AR_HIP_ERR_* code with a message in ar_hip_last_error().
 */
#ifndef AR_STATE_DICT_H
#define AR_STATE_DICT_H

#include <stddef.h>
#include <stdint.h>

#include "ar_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define AR_DTYPE_F64 3       /* CollectionData.data (repeated double) */
#define AR_SD_MAX_DIMS 8     /* dims per tensor accepted by this library */

typedef struct ar_state_dict ar_state_dict;

/* StateDictionary(String weightsDirectory) (StateDictionary.java constructor + loadWeights):
 * `path` is a directory (every regular file whose name does not start with '.', in name order)
 * or a single file.  Each file is parsed as CollectionLibraryData (StateDictionary.java:119-150):
 * a file that is not a valid message is skipped whole with a warning on stderr (parseFrom fails
 * before any entry is stored); entries are then stored in order, and one that cannot be decoded
 * (a non-positive dimension, or a value count other than the shape's size) stops that file with
 * a warning, the entries before it kept (the per-file try/catch).  An entry whose shape has no
 * dimensions is dropped (CollectionEncoder.decode returns null for it).  A key seen again
 * replaces the earlier entry (HashMap.put).  Errors: path missing or unreadable ->
 * AR_HIP_ERR_NOT_FOUND. */
int ar_hip_state_dict_open(const char *path, ar_state_dict **out);
/* StateDictionary(Map) with an empty map: an in-memory dictionary to fill with _put. */
int ar_hip_state_dict_create(ar_state_dict **out);
/* StateDictionary.destroy: releases the mapped files and owned tensors. */
int ar_hip_state_dict_destroy(ar_state_dict *sd);

/* StateDictionary.size / keySet (keys in byte order; *key stays valid until the dictionary
 * is modified or destroyed) / containsKey. */
int ar_hip_state_dict_size(const ar_state_dict *sd, int *count);
int ar_hip_state_dict_key(const ar_state_dict *sd, int index, const char **key);
int ar_hip_state_dict_contains(const ar_state_dict *sd, const char *key, int *found);
/* Files read by _open: parsed completely, and skipped after a parse failure. */
int ar_hip_state_dict_files(const ar_state_dict *sd, int *loaded, int *failed);

/* Shape and storage of one tensor: dims[0..*ndims-1] (dims must hold AR_SD_MAX_DIMS),
 * TraversalPolicyData.traversal_axis, the stored element type (AR_DTYPE_F64 when the entry
 * carries `data`, else AR_DTYPE_F32 for `data_32`: CollectionDataMemory.valueAt prefers data)
 * and the element count.  Unknown key -> AR_HIP_ERR_NOT_FOUND. */
int ar_hip_state_dict_info(const ar_state_dict *sd, const char *key, int *ndims, int32_t *dims,
                           int *traversal_axis, int *stored_dtype, int64_t *count);
/* StateDictionary.get(key) values, converted to `dtype` (AR_DTYPE_F32 rounds doubles to
 * nearest; AR_DTYPE_F64 widens floats exactly) into host memory of `count` elements
 * (count must equal the tensor's element count). */
int ar_hip_state_dict_read(const ar_state_dict *sd, const char *key, int dtype, void *out, int64_t count);

/* StateDictionary.put(key, collection): copies `count` values of `dtype` (AR_DTYPE_F32 or
 * AR_DTYPE_F64) with shape dims[0..ndims-1] (product must equal count). */
int ar_hip_state_dict_put(ar_state_dict *sd, const char *key, const int32_t *dims, int ndims, int traversal_axis,
                          const void *data, int dtype, int64_t count);
/* StateDictionary.save(Path, Precision) (StateDictionary.java save/encode; CollectionEncoder.encode):
 * one CollectionLibraryData file holding every entry, values written as data_32 (precision
 * AR_DTYPE_F32) or data (AR_DTYPE_F64). */
int ar_hip_state_dict_save(const ar_state_dict *sd, const char *path, int precision);

/* Qwen3.inferConfigFromWeights (engine/ml/.../qwen3/Qwen3.java:197-239): vocab and dim from
 * model.embed_tokens.weight, layer count from consecutive input_layernorm keys, heads and KV
 * heads from the first dimension of the layer-0 q_norm / k_norm gains, FFN width from
 * gate_proj, seq_len 131072, rope theta 1e6, tied embeddings unless lm_head.weight is present.
 * head_size is q_norm's second dimension when it has two (the reference's (heads, head_size)
 * gains), else dim / heads (TransformerConfig.java:79); QK-norm over the whole vector (the
 * reference graph, AttentionFeatures.java:840-845).
 * Fields the reference leaves to the caller (max_batch, weight_dtype, kv_dtype) are set to 1,
 * AR_DTYPE_F32, AR_DTYPE_F32; epsilon 1e-6 (Qwen3.java:397,402). */
int ar_hip_qwen3_infer_config(const ar_state_dict *sd, ar_qwen3_cfg *cfg);
/* Sets every tensor of the dictionary that the model has a slot for (keys the model does not
 * use are ignored, as Qwen3.model only asks for the ones it needs); the model still needs
 * ar_hip_qwen3_finalize.  Packed fp32 payloads go from the mapped file to the device. */
int ar_hip_qwen3_load_state_dict(ar_qwen3 *m, const ar_state_dict *sd);

#ifdef __cplusplus
}
#endif

#endif /* AR_STATE_DICT_H */
