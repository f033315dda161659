/*
 * JNI bridge: the natives of org.almostrealism.hardware.hip.HIP (java/ beside this file) onto the
 * C-ABI of libar_hip.so (include/ar_hip.h, include/ar_state_dict.h, include/ar_tokenizer.h,
 * include/ar_llama2.h).
 *
 * Not compiled in this repository: the build image has no JDK, so there is no jni.h.  A maintainer
 * builds it next to the library:
 *
 *   cc -O2 -shared -fPIC -I$JAVA_HOME/include -I$JAVA_HOME/include/linux -Iinclude \
 *      common_amd/jni/ar_hip_jni.c -Lcommon_amd/lib -lar_hip -Wl,-rpath,'$ORIGIN' \
 *      -o common_amd/lib/libar_hip_jni.so   (System.loadLibrary("ar_hip_jni") loads libar_hip_jni.so)
 *
 * The pattern is the one of the reference's hand-written Metal bridge
 * (base/hardware/src/main/cpp/MTL.cpp:37-536): jlong handles, array pinning around each native
 * call, and a Java exception for every failed call.  Status mapping: AR_HIP_ERR_INVALID ->
 * IllegalArgumentException, every other error -> org.almostrealism.hardware.HardwareException,
 * both carrying ar_hip_last_error().  A native that throws returns 0 / NULL; Java sees only the
 * exception.
 *
 * Array pinning: GetPrimitiveArrayCritical is used only around calls that copy (host <-> device
 * copies, weight uploads); calls that run model steps pin with Get<Type>ArrayElements, since they
 * may block on the GPU for milliseconds and a critical region would stall the garbage collector.
 */
#include <jni.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ar_hip.h"
#include "ar_llama2.h"
#include "ar_state_dict.h"
#include "ar_tokenizer.h"

#define HIP_CLASS(name) Java_org_almostrealism_hardware_hip_HIP_##name

/* The model handle Java holds: the library's model plus the two sizes its arrays need. */
typedef struct jqwen3 {
    ar_qwen3 *m;
    int max_batch;
    int vocab;
} jqwen3;

enum { QWEN3_INTS = 14, QWEN3_DOUBLES = 2 };

static void throw_status(JNIEnv *env, int rc) {
    const char *cls = rc == AR_HIP_ERR_INVALID ? "java/lang/IllegalArgumentException"
                                               : "org/almostrealism/hardware/HardwareException";
    char msg[1200];
    snprintf(msg, sizeof msg, "ar_hip error %d: %s", rc, ar_hip_last_error());
    jclass c = (*env)->FindClass(env, cls);
    if (c) (*env)->ThrowNew(env, c, msg);
}

static void throw_arg(JNIEnv *env, const char *msg) {
    jclass c = (*env)->FindClass(env, "java/lang/IllegalArgumentException");
    if (c) (*env)->ThrowNew(env, c, msg);
}

static void throw_oom(JNIEnv *env) {
    jclass c = (*env)->FindClass(env, "java/lang/OutOfMemoryError");
    if (c) (*env)->ThrowNew(env, c, "ar_hip_jni: host allocation failed");
}

/* 1 when rc failed (exception pending), else 0 */
static int failed(JNIEnv *env, int rc) {
    if (rc == AR_HIP_OK) return 0;
    throw_status(env, rc);
    return 1;
}

static ar_hip_ctx *CTX(jlong h) { return (ar_hip_ctx *)(intptr_t)h; }
static jqwen3 *QM(jlong h) { return (jqwen3 *)(intptr_t)h; }

/* [off, off + len) inside an array of n elements */
static int in_bounds(JNIEnv *env, jsize n, jint off, jint len) {
    if (off < 0 || len < 0 || (jlong)off + len > n) {
        throw_arg(env, "array range out of bounds");
        return 0;
    }
    return 1;
}

/* ---- context and memory ------------------------------------------------------------ */

JNIEXPORT jint JNICALL HIP_CLASS(deviceCount)(JNIEnv *env, jclass c) {
    int n = 0;
    const int rc = ar_hip_device_count(&n);
    /* no driver is "zero devices" for selection, as the reference probes drivers and warns */
    return rc == AR_HIP_OK ? n : 0;
}

JNIEXPORT jlong JNICALL HIP_CLASS(init)(JNIEnv *env, jclass c, jint device) {
    ar_hip_ctx *ctx = NULL;
    if (failed(env, ar_hip_init(device, &ctx))) return 0;
    return (jlong)(intptr_t)ctx;
}

JNIEXPORT void JNICALL HIP_CLASS(destroy)(JNIEnv *env, jclass c, jlong ctx) {
    failed(env, ar_hip_destroy(CTX(ctx)));
}

JNIEXPORT void JNICALL HIP_CLASS(synchronize)(JNIEnv *env, jclass c, jlong ctx) {
    failed(env, ar_hip_synchronize(CTX(ctx)));
}

JNIEXPORT jint JNICALL HIP_CLASS(computeUnits)(JNIEnv *env, jclass c, jlong ctx) {
    int cus = 0;
    if (failed(env, ar_hip_device_info(CTX(ctx), &cus, NULL, NULL, 0))) return 0;
    return cus;
}

JNIEXPORT jlong JNICALL HIP_CLASS(hbmBytes)(JNIEnv *env, jclass c, jlong ctx) {
    size_t bytes = 0;
    if (failed(env, ar_hip_device_info(CTX(ctx), NULL, &bytes, NULL, 0))) return 0;
    return (jlong)bytes;
}

JNIEXPORT jstring JNICALL HIP_CLASS(deviceName)(JNIEnv *env, jclass c, jlong ctx) {
    char name[256];
    if (failed(env, ar_hip_device_info(CTX(ctx), NULL, NULL, name, (int)sizeof name))) return NULL;
    return (*env)->NewStringUTF(env, name);
}

JNIEXPORT jlong JNICALL HIP_CLASS(alloc)(JNIEnv *env, jclass c, jlong ctx, jlong bytes) {
    void *p = NULL;
    if (bytes <= 0) {
        throw_arg(env, "allocation size must be positive");
        return 0;
    }
    if (failed(env, ar_hip_alloc(CTX(ctx), (size_t)bytes, &p))) return 0;
    return (jlong)(intptr_t)p;
}

JNIEXPORT void JNICALL HIP_CLASS(free)(JNIEnv *env, jclass c, jlong ctx, jlong ptr) {
    failed(env, ar_hip_free(CTX(ctx), (void *)(intptr_t)ptr));
}

JNIEXPORT jlong JNICALL HIP_CLASS(allocatedBytes)(JNIEnv *env, jclass c, jlong ctx) {
    size_t bytes = 0;
    if (failed(env, ar_hip_allocated_bytes(CTX(ctx), &bytes))) return 0;
    return (jlong)bytes;
}

JNIEXPORT void JNICALL HIP_CLASS(setMem)(JNIEnv *env, jclass c, jlong ctx, jlong dst, jlong dst_off, jfloatArray src,
                                         jint src_off, jint len) {
    if (!in_bounds(env, (*env)->GetArrayLength(env, src), src_off, len) || len == 0) return;
    jfloat *p = (*env)->GetPrimitiveArrayCritical(env, src, NULL);
    if (!p) { throw_oom(env); return; }
    const int rc = ar_hip_memcpy_h2d(CTX(ctx), (char *)(intptr_t)dst + dst_off, p + src_off, (size_t)len * sizeof(float));
    (*env)->ReleasePrimitiveArrayCritical(env, src, p, JNI_ABORT);  /* read only: no copy back */
    failed(env, rc);
}

JNIEXPORT void JNICALL HIP_CLASS(getMem)(JNIEnv *env, jclass c, jlong ctx, jlong src, jlong src_off, jfloatArray dst,
                                         jint dst_off, jint len) {
    if (!in_bounds(env, (*env)->GetArrayLength(env, dst), dst_off, len) || len == 0) return;
    jfloat *p = (*env)->GetPrimitiveArrayCritical(env, dst, NULL);
    if (!p) { throw_oom(env); return; }
    const int rc = ar_hip_memcpy_d2h(CTX(ctx), p + dst_off, (const char *)(intptr_t)src + src_off, (size_t)len * sizeof(float));
    (*env)->ReleasePrimitiveArrayCritical(env, dst, p, 0);
    failed(env, rc);
}

JNIEXPORT void JNICALL HIP_CLASS(copy)(JNIEnv *env, jclass c, jlong ctx, jlong dst, jlong src, jlong bytes) {
    if (bytes < 0) { throw_arg(env, "negative copy size"); return; }
    failed(env, ar_hip_memcpy_d2d(CTX(ctx), (void *)(intptr_t)dst, (const void *)(intptr_t)src, (size_t)bytes));
}

/* ---- stand-alone decode attention ---------------------------------------------------- */

#define ATTN_ARGS                                                                                     \
    CTX(ctx), (const float *)(intptr_t)q, (const float *)(intptr_t)k, (const float *)(intptr_t)v,   \
        (const float *)(intptr_t)qn, (const float *)(intptr_t)kn, eps, mode, (float *)(intptr_t)kc,  \
        (float *)(intptr_t)vc, max_seq, pos, heads, kv_heads, hd, theta, (float *)(intptr_t)out

JNIEXPORT void JNICALL HIP_CLASS(attentionDecode)(JNIEnv *env, jclass c, jlong ctx, jlong q, jlong k, jlong v, jlong qn,
                                                  jlong kn, jfloat eps, jint mode, jlong kc, jlong vc, jint max_seq,
                                                  jint pos, jint heads, jint kv_heads, jint hd, jdouble theta,
                                                  jlong out) {
    failed(env, ar_hip_attention_decode(ATTN_ARGS));
}

JNIEXPORT void JNICALL HIP_CLASS(attentionDecodeNoAlloc)(JNIEnv *env, jclass c, jlong ctx, jlong q, jlong k, jlong v,
                                                         jlong qn, jlong kn, jfloat eps, jint mode, jlong kc, jlong vc,
                                                         jint max_seq, jint pos, jint heads, jint kv_heads, jint hd,
                                                         jdouble theta, jlong out) {
    failed(env, ar_hip_attention_decode_noalloc(ATTN_ARGS));
}
#undef ATTN_ARGS

/* ---- Qwen3 model ------------------------------------------------------------------- */

static int read_cfg(JNIEnv *env, jintArray ints, jdoubleArray doubles, ar_qwen3_cfg *cfg) {
    if ((*env)->GetArrayLength(env, ints) != QWEN3_INTS || (*env)->GetArrayLength(env, doubles) != QWEN3_DOUBLES) {
        throw_arg(env, "qwen3 config: 14 ints and 2 doubles expected");
        return 0;
    }
    jint v[QWEN3_INTS];
    jdouble d[QWEN3_DOUBLES];
    (*env)->GetIntArrayRegion(env, ints, 0, QWEN3_INTS, v);
    (*env)->GetDoubleArrayRegion(env, doubles, 0, QWEN3_DOUBLES, d);
    memset(cfg, 0, sizeof *cfg);
    cfg->dim = v[0]; cfg->hidden_dim = v[1]; cfg->layer_count = v[2]; cfg->head_count = v[3];
    cfg->kv_head_count = v[4]; cfg->head_size = v[5]; cfg->vocab_size = v[6]; cfg->seq_len = v[7];
    cfg->max_batch = v[8]; cfg->weight_dtype = v[9]; cfg->qk_norm_mode = v[10]; cfg->shared_weights = v[11];
    cfg->qkv_bias = v[12]; cfg->kv_dtype = v[13];
    cfg->rope_theta = d[0]; cfg->epsilon = d[1];
    return 1;
}

static void write_cfg(JNIEnv *env, const ar_qwen3_cfg *cfg, jintArray ints, jdoubleArray doubles) {
    const jint v[QWEN3_INTS] = {cfg->dim, cfg->hidden_dim, cfg->layer_count, cfg->head_count, cfg->kv_head_count,
                                cfg->head_size, cfg->vocab_size, cfg->seq_len, cfg->max_batch, cfg->weight_dtype,
                                cfg->qk_norm_mode, cfg->shared_weights, cfg->qkv_bias, cfg->kv_dtype};
    const jdouble d[QWEN3_DOUBLES] = {cfg->rope_theta, cfg->epsilon};
    (*env)->SetIntArrayRegion(env, ints, 0, QWEN3_INTS, v);
    (*env)->SetDoubleArrayRegion(env, doubles, 0, QWEN3_DOUBLES, d);
}

JNIEXPORT jlong JNICALL HIP_CLASS(qwen3Create)(JNIEnv *env, jclass c, jlong ctx, jintArray ints, jdoubleArray doubles) {
    ar_qwen3_cfg cfg;
    if (!read_cfg(env, ints, doubles, &cfg)) return 0;
    jqwen3 *h = calloc(1, sizeof *h);
    if (!h) { throw_oom(env); return 0; }
    if (failed(env, ar_hip_qwen3_create(CTX(ctx), &cfg, &h->m))) {
        free(h);
        return 0;
    }
    h->max_batch = cfg.max_batch;
    h->vocab = cfg.vocab_size;
    return (jlong)(intptr_t)h;
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3SetWeight)(JNIEnv *env, jclass c, jlong m, jstring key, jfloatArray data) {
    const char *k = (*env)->GetStringUTFChars(env, key, NULL);
    if (!k) return;  /* OutOfMemoryError pending */
    const jsize n = (*env)->GetArrayLength(env, data);
    jfloat *p = (*env)->GetPrimitiveArrayCritical(env, data, NULL);
    if (!p) { (*env)->ReleaseStringUTFChars(env, key, k); throw_oom(env); return; }
    const int rc = ar_hip_qwen3_set_weight(QM(m)->m, k, p, AR_DTYPE_F32, (int64_t)n);
    (*env)->ReleasePrimitiveArrayCritical(env, data, p, JNI_ABORT);
    (*env)->ReleaseStringUTFChars(env, key, k);
    failed(env, rc);
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3SetWeightBf16)(JNIEnv *env, jclass c, jlong m, jstring key, jshortArray data) {
    const char *k = (*env)->GetStringUTFChars(env, key, NULL);
    if (!k) return;
    const jsize n = (*env)->GetArrayLength(env, data);
    jshort *p = (*env)->GetPrimitiveArrayCritical(env, data, NULL);
    if (!p) { (*env)->ReleaseStringUTFChars(env, key, k); throw_oom(env); return; }
    const int rc = ar_hip_qwen3_set_weight(QM(m)->m, k, p, AR_DTYPE_BF16, (int64_t)n);
    (*env)->ReleasePrimitiveArrayCritical(env, data, p, JNI_ABORT);
    (*env)->ReleaseStringUTFChars(env, key, k);
    failed(env, rc);
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3Finalize)(JNIEnv *env, jclass c, jlong m) {
    failed(env, ar_hip_qwen3_finalize(QM(m)->m));
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3Reset)(JNIEnv *env, jclass c, jlong m) {
    failed(env, ar_hip_qwen3_reset(QM(m)->m));
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3SetPrompt)(JNIEnv *env, jclass c, jlong m, jint seq, jintArray ids) {
    const jsize n = (*env)->GetArrayLength(env, ids);
    jint *p = (*env)->GetIntArrayElements(env, ids, NULL);
    if (!p) { throw_oom(env); return; }
    const int rc = ar_hip_qwen3_set_prompt(QM(m)->m, seq, (const int32_t *)p, (int)n);
    (*env)->ReleaseIntArrayElements(env, ids, p, JNI_ABORT);
    failed(env, rc);
}

/* logits (optional) must hold max_batch x vocab floats */
static jfloat *logits_elements(JNIEnv *env, const jqwen3 *h, jfloatArray logits, int *ok) {
    *ok = 1;
    if (!logits) return NULL;
    if ((*env)->GetArrayLength(env, logits) != (jsize)((jlong)h->max_batch * h->vocab)) {
        throw_arg(env, "logits array must hold maxBatch x vocabSize floats");
        *ok = 0;
        return NULL;
    }
    jfloat *p = (*env)->GetFloatArrayElements(env, logits, NULL);
    if (!p) { throw_oom(env); *ok = 0; }
    return p;
}

JNIEXPORT jintArray JNICALL HIP_CLASS(qwen3Next)(JNIEnv *env, jclass c, jlong m, jfloatArray logits) {
    jqwen3 *h = QM(m);
    int ok;
    jfloat *lp = logits_elements(env, h, logits, &ok);
    if (!ok) return NULL;
    int32_t toks[64];  /* max_batch <= 8 (ar_qwen3_cfg) */
    const int rc = ar_hip_qwen3_next(h->m, toks, lp);
    if (lp) (*env)->ReleaseFloatArrayElements(env, logits, lp, rc == AR_HIP_OK ? 0 : JNI_ABORT);
    if (failed(env, rc)) return NULL;
    jintArray out = (*env)->NewIntArray(env, h->max_batch);  /* one token per sequence */
    if (out) (*env)->SetIntArrayRegion(env, out, 0, h->max_batch, (const jint *)toks);
    return out;
}

JNIEXPORT jintArray JNICALL HIP_CLASS(qwen3Run)(JNIEnv *env, jclass c, jlong m, jint steps) {
    jqwen3 *h = QM(m);
    if (steps < 0) { throw_arg(env, "steps must be >= 0"); return NULL; }
    const jlong n = (jlong)h->max_batch * steps;
    if (n > 0x7fffffffL) { throw_arg(env, "maxBatch x steps exceeds an int array"); return NULL; }
    int32_t *toks = malloc((size_t)(n > 0 ? n : 1) * sizeof(int32_t));
    if (!toks) { throw_oom(env); return NULL; }
    const int rc = steps > 0 ? ar_hip_qwen3_run(h->m, steps, toks) : AR_HIP_OK;
    jintArray out = NULL;
    if (!failed(env, rc)) {
        out = (*env)->NewIntArray(env, (jsize)n);
        if (out) (*env)->SetIntArrayRegion(env, out, 0, (jsize)n, (const jint *)toks);
    }
    free(toks);
    return out;
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3Prefill)(JNIEnv *env, jclass c, jlong m, jfloatArray logits) {
    jqwen3 *h = QM(m);
    int ok;
    jfloat *lp = logits_elements(env, h, logits, &ok);
    if (!ok) return;
    const int rc = ar_hip_qwen3_prefill(h->m, lp);
    if (lp) (*env)->ReleaseFloatArrayElements(env, logits, lp, rc == AR_HIP_OK ? 0 : JNI_ABORT);
    failed(env, rc);
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3SetSampling)(JNIEnv *env, jclass c, jlong m, jint mode, jdouble temperature,
                                                   jdouble top_p, jlongArray seeds) {
    jqwen3 *h = QM(m);
    int64_t s[64];
    if (seeds) {
        if ((*env)->GetArrayLength(env, seeds) != h->max_batch) {
            throw_arg(env, "seeds must hold one value per sequence (maxBatch)");
            return;
        }
        jlong tmp[64];
        (*env)->GetLongArrayRegion(env, seeds, 0, h->max_batch, tmp);
        for (int i = 0; i < h->max_batch; i++) s[i] = (int64_t)tmp[i];
    }
    failed(env, ar_hip_qwen3_set_sampling(h->m, mode, temperature, top_p, seeds ? s : NULL));
}

JNIEXPORT jint JNICALL HIP_CLASS(qwen3Position)(JNIEnv *env, jclass c, jlong m) {
    int pos = 0;
    if (failed(env, ar_hip_qwen3_position(QM(m)->m, &pos))) return 0;
    return pos;
}

JNIEXPORT jint JNICALL HIP_CLASS(qwen3MaxBatch)(JNIEnv *env, jclass c, jlong m) { return QM(m)->max_batch; }

JNIEXPORT jint JNICALL HIP_CLASS(qwen3VocabSize)(JNIEnv *env, jclass c, jlong m) { return QM(m)->vocab; }

JNIEXPORT void JNICALL HIP_CLASS(qwen3KernelTiming)(JNIEnv *env, jclass c, jlong m, jint which) {
    failed(env, ar_hip_qwen3_kernel_timing(QM(m)->m, which));
}

JNIEXPORT jdoubleArray JNICALL HIP_CLASS(qwen3KernelTime)(JNIEnv *env, jclass c, jlong m) {
    double ms = 0.0;
    int launches = 0;
    if (failed(env, ar_hip_qwen3_kernel_time(QM(m)->m, &ms, &launches))) return NULL;
    const jdouble v[2] = {ms, (jdouble)launches};
    jdoubleArray out = (*env)->NewDoubleArray(env, 2);
    if (out) (*env)->SetDoubleArrayRegion(env, out, 0, 2, v);
    return out;
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3UsePersistent)(JNIEnv *env, jclass c, jlong m, jboolean enable) {
    failed(env, ar_hip_qwen3_use_persistent(QM(m)->m, enable ? 1 : 0));
}

JNIEXPORT jboolean JNICALL HIP_CLASS(qwen3Persistent)(JNIEnv *env, jclass c, jlong m) {
    int active = 0;
    if (failed(env, ar_hip_qwen3_persistent(QM(m)->m, &active))) return JNI_FALSE;
    return active ? JNI_TRUE : JNI_FALSE;
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3PrefillGemm)(JNIEnv *env, jclass c, jlong m, jint backend) {
    failed(env, ar_hip_qwen3_prefill_gemm(QM(m)->m, backend));
}

JNIEXPORT jint JNICALL HIP_CLASS(qwen3PrefillGemmBackend)(JNIEnv *env, jclass c, jlong m) {
    int backend = 0;
    if (failed(env, ar_hip_qwen3_prefill_gemm_backend(QM(m)->m, &backend))) return -1;
    return backend;
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3Destroy)(JNIEnv *env, jclass c, jlong m) {
    jqwen3 *h = QM(m);
    if (!h) return;
    const int rc = ar_hip_qwen3_destroy(h->m);
    free(h);
    failed(env, rc);
}

/* ---- protobuf weights -------------------------------------------------------------- */

JNIEXPORT jlong JNICALL HIP_CLASS(stateDictOpen)(JNIEnv *env, jclass c, jstring path) {
    const char *p = (*env)->GetStringUTFChars(env, path, NULL);
    if (!p) return 0;
    ar_state_dict *sd = NULL;
    const int rc = ar_hip_state_dict_open(p, &sd);
    (*env)->ReleaseStringUTFChars(env, path, p);
    if (failed(env, rc)) return 0;
    return (jlong)(intptr_t)sd;
}

JNIEXPORT void JNICALL HIP_CLASS(stateDictDestroy)(JNIEnv *env, jclass c, jlong sd) {
    failed(env, ar_hip_state_dict_destroy((ar_state_dict *)(intptr_t)sd));
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3InferConfig)(JNIEnv *env, jclass c, jlong sd, jintArray ints, jdoubleArray doubles) {
    if ((*env)->GetArrayLength(env, ints) != QWEN3_INTS || (*env)->GetArrayLength(env, doubles) != QWEN3_DOUBLES) {
        throw_arg(env, "qwen3 config: 14 ints and 2 doubles expected");
        return;
    }
    ar_qwen3_cfg cfg;
    if (failed(env, ar_hip_qwen3_infer_config((const ar_state_dict *)(intptr_t)sd, &cfg))) return;
    write_cfg(env, &cfg, ints, doubles);
}

JNIEXPORT void JNICALL HIP_CLASS(qwen3LoadStateDict)(JNIEnv *env, jclass c, jlong m, jlong sd) {
    failed(env, ar_hip_qwen3_load_state_dict(QM(m)->m, (const ar_state_dict *)(intptr_t)sd));
}

/* ---- llama2.c checkpoints ------------------------------------------------------------ */

JNIEXPORT jlong JNICALL HIP_CLASS(llama2Open)(JNIEnv *env, jclass c, jstring path) {
    const char *p = (*env)->GetStringUTFChars(env, path, NULL);
    if (!p) return 0;
    ar_llama2_ckpt *ck = NULL;
    const int rc = ar_hip_llama2_open(p, &ck);
    (*env)->ReleaseStringUTFChars(env, path, p);
    if (failed(env, rc)) return 0;
    return (jlong)(intptr_t)ck;
}

JNIEXPORT jintArray JNICALL HIP_CLASS(llama2Config)(JNIEnv *env, jclass c, jlong ck) {
    ar_llama2_cfg cfg;
    if (failed(env, ar_hip_llama2_config((const ar_llama2_ckpt *)(intptr_t)ck, &cfg))) return NULL;
    const jint v[9] = {cfg.dim, cfg.hidden_dim, cfg.layer_count, cfg.head_count, cfg.kv_head_count,
                       cfg.vocab_size, cfg.seq_len, cfg.shared_weights, cfg.head_size};
    jintArray out = (*env)->NewIntArray(env, 9);
    if (out) (*env)->SetIntArrayRegion(env, out, 0, 9, v);
    return out;
}

JNIEXPORT jlong JNICALL HIP_CLASS(llama2CreateModel)(JNIEnv *env, jclass c, jlong ctx, jlong ck, jint batch,
                                                     jint wdtype, jint kvdtype) {
    ar_llama2_cfg cfg;
    if (failed(env, ar_hip_llama2_config((const ar_llama2_ckpt *)(intptr_t)ck, &cfg))) return 0;
    jqwen3 *h = calloc(1, sizeof *h);
    if (!h) { throw_oom(env); return 0; }
    if (failed(env, ar_hip_llama2_create_model(CTX(ctx), (const ar_llama2_ckpt *)(intptr_t)ck, batch, wdtype, kvdtype,
                                               &h->m))) {
        free(h);
        return 0;
    }
    h->max_batch = batch;
    h->vocab = cfg.vocab_size;
    return (jlong)(intptr_t)h;
}

JNIEXPORT void JNICALL HIP_CLASS(llama2Close)(JNIEnv *env, jclass c, jlong ck) {
    failed(env, ar_hip_llama2_close((ar_llama2_ckpt *)(intptr_t)ck));
}

JNIEXPORT jlong JNICALL HIP_CLASS(bpeLoad)(JNIEnv *env, jclass c, jstring path, jint vocab_size) {
    const char *p = (*env)->GetStringUTFChars(env, path, NULL);
    if (!p) return 0;
    ar_bpe *t = NULL;
    const int rc = ar_hip_bpe_load(p, vocab_size, &t);
    (*env)->ReleaseStringUTFChars(env, path, p);
    if (failed(env, rc)) return 0;
    return (jlong)(intptr_t)t;
}

JNIEXPORT jintArray JNICALL HIP_CLASS(bpeEncode)(JNIEnv *env, jclass c, jlong bpe, jbyteArray utf8) {
    const jsize n = (*env)->GetArrayLength(env, utf8);
    jbyte *text = (*env)->GetByteArrayElements(env, utf8, NULL);
    if (!text) { throw_oom(env); return NULL; }
    /* one token per UTF-16 unit before merging, and a UTF-8 text has at least as many bytes */
    int32_t *toks = malloc((size_t)(n > 0 ? n : 1) * sizeof(int32_t));
    if (!toks) {
        (*env)->ReleaseByteArrayElements(env, utf8, text, JNI_ABORT);
        throw_oom(env);
        return NULL;
    }
    int count = 0;
    const int rc = ar_hip_bpe_encode((const ar_bpe *)(intptr_t)bpe, (const char *)text, (int)n, toks, (int)n, &count);
    (*env)->ReleaseByteArrayElements(env, utf8, text, JNI_ABORT);
    jintArray out = NULL;
    if (!failed(env, rc)) {
        out = (*env)->NewIntArray(env, count);
        if (out && count > 0) (*env)->SetIntArrayRegion(env, out, 0, count, (const jint *)toks);
    }
    free(toks);
    return out;
}

JNIEXPORT jbyteArray JNICALL HIP_CLASS(bpeToken)(JNIEnv *env, jclass c, jlong bpe, jint id) {
    const char *s = NULL;
    int len = 0;
    float score = 0.f;
    if (failed(env, ar_hip_bpe_token((const ar_bpe *)(intptr_t)bpe, id, &s, &len, &score))) return NULL;
    jbyteArray out = (*env)->NewByteArray(env, len);
    if (out && len > 0) (*env)->SetByteArrayRegion(env, out, 0, len, (const jbyte *)s);
    return out;
}

JNIEXPORT void JNICALL HIP_CLASS(bpeDestroy)(JNIEnv *env, jclass c, jlong bpe) {
    failed(env, ar_hip_bpe_destroy((ar_bpe *)(intptr_t)bpe));
}

/* ---- tokenizer ---------------------------------------------------------------------- */

JNIEXPORT jlong JNICALL HIP_CLASS(tokenizerLoad)(JNIEnv *env, jclass c, jstring path) {
    const char *p = (*env)->GetStringUTFChars(env, path, NULL);
    if (!p) return 0;
    ar_tokenizer *t = NULL;
    const int rc = ar_hip_tokenizer_load(p, &t);
    (*env)->ReleaseStringUTFChars(env, path, p);
    if (failed(env, rc)) return 0;
    return (jlong)(intptr_t)t;
}

JNIEXPORT jintArray JNICALL HIP_CLASS(tokenizerEncode)(JNIEnv *env, jclass c, jlong tok, jbyteArray utf8, jboolean bos,
                                                       jboolean eos) {
    const ar_tokenizer *t = (const ar_tokenizer *)(intptr_t)tok;
    const jsize n = (*env)->GetArrayLength(env, utf8);
    jbyte *text = (*env)->GetByteArrayElements(env, utf8, NULL);
    if (!text) { throw_oom(env); return NULL; }
    int count = 0;
    /* first call sizes the output (out = NULL), the second fills it */
    int rc = ar_hip_tokenizer_encode(t, (const char *)text, n, bos, eos, NULL, 0, &count);
    int32_t *ids = NULL;
    if (rc == AR_HIP_OK && count > 0) {
        ids = malloc((size_t)count * sizeof(int32_t));
        if (!ids) {
            (*env)->ReleaseByteArrayElements(env, utf8, text, JNI_ABORT);
            throw_oom(env);
            return NULL;
        }
        rc = ar_hip_tokenizer_encode(t, (const char *)text, n, bos, eos, ids, count, &count);
    }
    (*env)->ReleaseByteArrayElements(env, utf8, text, JNI_ABORT);
    jintArray out = NULL;
    if (!failed(env, rc)) {
        out = (*env)->NewIntArray(env, count);
        if (out && count > 0) (*env)->SetIntArrayRegion(env, out, 0, count, (const jint *)ids);
    }
    free(ids);
    return out;
}

JNIEXPORT jbyteArray JNICALL HIP_CLASS(tokenizerDecode)(JNIEnv *env, jclass c, jlong tok, jintArray ids) {
    const ar_tokenizer *t = (const ar_tokenizer *)(intptr_t)tok;
    const jsize n = (*env)->GetArrayLength(env, ids);
    jint *p = (*env)->GetIntArrayElements(env, ids, NULL);
    if (!p) { throw_oom(env); return NULL; }
    int64_t len = 0;
    int rc = ar_hip_tokenizer_decode(t, (const int32_t *)p, (int)n, NULL, 0, &len);
    char *buf = NULL;
    if (rc == AR_HIP_OK) {
        buf = malloc((size_t)len + 1);
        if (!buf) {
            (*env)->ReleaseIntArrayElements(env, ids, p, JNI_ABORT);
            throw_oom(env);
            return NULL;
        }
        rc = ar_hip_tokenizer_decode(t, (const int32_t *)p, (int)n, buf, len + 1, &len);
    }
    (*env)->ReleaseIntArrayElements(env, ids, p, JNI_ABORT);
    jbyteArray out = NULL;
    if (!failed(env, rc)) {
        if (len > 0x7fffffffL) {
            throw_arg(env, "decoded text exceeds a byte array");
        } else {
            out = (*env)->NewByteArray(env, (jsize)len);
            if (out && len > 0) (*env)->SetByteArrayRegion(env, out, 0, (jsize)len, (const jbyte *)buf);
        }
    }
    free(buf);
    return out;
}

JNIEXPORT void JNICALL HIP_CLASS(tokenizerDestroy)(JNIEnv *env, jclass c, jlong tok) {
    failed(env, ar_hip_tokenizer_destroy((ar_tokenizer *)(intptr_t)tok));
}
