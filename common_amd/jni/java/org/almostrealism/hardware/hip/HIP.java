/*
 * Native entry points of libar_hip.so, bound through libar_hip_jni.so (ar_hip_jni.c beside this
 * source tree).  Handles are opaque native pointers carried as long; every native throws
 * org.almostrealism.hardware.HardwareException (HIP / driver failures) or IllegalArgumentException
 * (invalid arguments) with the library's own message when the C call does not return AR_HIP_OK.
 *
 * Not compiled in this repository (the build image has no JDK); the Python ctypes binding
 * (common_amd/hardware.py, common_amd/qwen3.py) binds the same C symbols and is what the tests run.
 *
 * Reference counterparts: the Metal bridge's native class (base/hardware/src/main/java/org/
 * almostrealism/hardware/metal/MTL.java) and its C++ side (base/hardware/src/main/cpp/MTL.cpp:37-536).
 */
package org.almostrealism.hardware.hip;

final class HIP {
	static {
		System.loadLibrary("ar_hip_jni");
	}

	private HIP() { }

	/* AR_DTYPE_* / AR_QK_NORM_* / AR_SAMPLE_* of include/ar_hip.h */
	static final int DTYPE_F32 = 0;
	static final int DTYPE_BF16 = 1;
	static final int DTYPE_F16 = 2;
	static final int QK_NORM_WHOLE = 0;
	static final int QK_NORM_PER_HEAD = 1;
	static final int SAMPLE_MODEL = 0;
	static final int SAMPLE_TOKEN = 1;
	// kernel classes of the decode step (AR_KT_* of include/ar_hip.h)
	static final int KT_NONE = 0, KT_LOGITS = 1, KT_GATE_UP = 2, KT_QKV = 3, KT_ATTENTION = 4, KT_DOWN = 5, KT_O = 6,
			KT_LAYERS = 7;
	// prefill product backends (AR_PREFILL_GEMM_* of include/ar_hip.h)
	static final int PREFILL_GEMM_OWN = 0, PREFILL_GEMM_ROCBLAS = 1;

	/* ---- data / compute context and memory (DataContext, ComputeContext, MemoryProvider) ---- */
	static native int deviceCount();                                   // ar_hip_device_count
	static native long init(int device);                               // ar_hip_init (-1: AR_HIP_DEVICE)
	static native void destroy(long ctx);                              // ar_hip_destroy
	static native void synchronize(long ctx);                          // ar_hip_synchronize
	static native int computeUnits(long ctx);                          // ar_hip_device_info
	static native long hbmBytes(long ctx);                             // ar_hip_device_info
	static native String deviceName(long ctx);                         // ar_hip_device_info
	static native long alloc(long ctx, long bytes);                    // ar_hip_alloc
	static native void free(long ctx, long ptr);                       // ar_hip_free
	static native long allocatedBytes(long ctx);                       // ar_hip_allocated_bytes
	/** Host floats -> device: writes length floats at dst + dstByteOffset. */
	static native void setMem(long ctx, long dst, long dstByteOffset, float[] src, int srcOffset, int length);
	/** Device -> host floats: reads length floats at src + srcByteOffset. */
	static native void getMem(long ctx, long src, long srcByteOffset, float[] dst, int dstOffset, int length);
	/** Device -> device copy of bytes, ordered on the context's stream. */
	static native void copy(long ctx, long dst, long src, long bytes);  // ar_hip_memcpy_d2d

	/* ---- stand-alone decode attention (AttentionFeatures.attentionImpl), device pointers ---- */
	static native void attentionDecode(long ctx, long q, long k, long v, long qNorm, long kNorm, float eps,
									   int qkNormMode, long kCache, long vCache, int maxSeq, int pos, int heads,
									   int kvHeads, int headDim, double ropeTheta, long out);  // ar_hip_attention_decode
	/** The same without any allocation (no reference counterpart): for callers that cannot allocate. */
	static native void attentionDecodeNoAlloc(long ctx, long q, long k, long v, long qNorm, long kNorm, float eps,
											  int qkNormMode, long kCache, long vCache, int maxSeq, int pos,
											  int heads, int kvHeads, int headDim, double ropeTheta,
											  long out);  // ar_hip_attention_decode_noalloc

	/* ---- Qwen3 model (Qwen3.model + CompiledModel.forward + AutoregressiveModel) ---- */
	/**
	 * ints: dim, hiddenDim, layerCount, headCount, kvHeadCount, headSize, vocabSize, seqLen, maxBatch,
	 * weightDtype, qkNormMode, sharedWeights, qkvBias, kvDtype; doubles: ropeTheta, epsilon
	 * (the fields of ar_qwen3_cfg in that order).
	 */
	static native long qwen3Create(long ctx, int[] ints, double[] doubles);     // ar_hip_qwen3_create
	static native void qwen3SetWeight(long model, String key, float[] data);     // ar_hip_qwen3_set_weight (fp32)
	static native void qwen3SetWeightBf16(long model, String key, short[] data); // ar_hip_qwen3_set_weight (bf16 bits)
	static native void qwen3Finalize(long model);                                // ar_hip_qwen3_finalize
	static native void qwen3Reset(long model);                                   // ar_hip_qwen3_reset
	static native void qwen3SetPrompt(long model, int seq, int[] ids);           // ar_hip_qwen3_set_prompt
	/** One step of every sequence: maxBatch tokens; logits (maxBatch x vocab) filled when not null. */
	static native int[] qwen3Next(long model, float[] logitsOrNull);             // ar_hip_qwen3_next
	/** steps steps of every sequence: maxBatch x steps tokens, row-major by sequence. */
	static native int[] qwen3Run(long model, int steps);                         // ar_hip_qwen3_run
	static native void qwen3Prefill(long model, float[] logitsOrNull);           // ar_hip_qwen3_prefill
	static native void qwen3SetSampling(long model, int mode, double temperature, double topP,
										long[] seedsOrNull);                     // ar_hip_qwen3_set_sampling
	static native int qwen3Position(long model);                                 // ar_hip_qwen3_position
	static native int qwen3MaxBatch(long model);                                 // kept by the shim
	static native int qwen3VocabSize(long model);                                // kept by the shim
	static native void qwen3Destroy(long model);                                 // ar_hip_qwen3_destroy
	static native void qwen3KernelTiming(long model, int which);                 // ar_hip_qwen3_kernel_timing
	static native double[] qwen3KernelTime(long model);                          // ar_hip_qwen3_kernel_time: {ms, launches}
	static native void qwen3UsePersistent(long model, boolean enable);           // ar_hip_qwen3_use_persistent
	static native boolean qwen3Persistent(long model);                           // ar_hip_qwen3_persistent
	static native void qwen3PrefillGemm(long model, int backend);                // ar_hip_qwen3_prefill_gemm
	static native int qwen3PrefillGemmBackend(long model);                       // ar_hip_qwen3_prefill_gemm_backend

	/* ---- protobuf weights (StateDictionary) ---- */
	static native long stateDictOpen(String weightsDirectory);                   // ar_hip_state_dict_open
	static native void stateDictDestroy(long dict);                              // ar_hip_state_dict_destroy
	/** Qwen3.inferConfigFromWeights: ints / doubles in qwen3Create's order. */
	static native void qwen3InferConfig(long dict, int[] ints, double[] doubles); // ar_hip_qwen3_infer_config
	static native void qwen3LoadStateDict(long model, long dict);                // ar_hip_qwen3_load_state_dict

	/* ---- llama2.c checkpoints and their BPE tokenizer (Llama2, Llama2Weights, BPE) ---- */
	static native long llama2Open(String checkpoint);                            // ar_hip_llama2_open
	/** dim, hiddenDim, layerCount, headCount, kvHeadCount, vocabSize, seqLen, sharedWeights, headSize */
	static native int[] llama2Config(long ckpt);                                 // ar_hip_llama2_config
	/** Llama2.model on ctx: a model handle of the same kind as qwen3Create's. */
	static native long llama2CreateModel(long ctx, long ckpt, int maxBatch, int weightDtype, int kvDtype);
	static native void llama2Close(long ckpt);                                   // ar_hip_llama2_close
	static native long bpeLoad(String tokenizerPath, int vocabSize);             // ar_hip_bpe_load
	static native int[] bpeEncode(long bpe, byte[] utf8);                        // ar_hip_bpe_encode
	static native byte[] bpeToken(long bpe, int id);                             // ar_hip_bpe_token
	static native void bpeDestroy(long bpe);                                     // ar_hip_bpe_destroy

	/* ---- tokenizer (Qwen3Tokenizer) ---- */
	static native long tokenizerLoad(String tokenizerPath);                      // ar_hip_tokenizer_load
	static native int[] tokenizerEncode(long tok, byte[] utf8, boolean addBos, boolean addEos); // ar_hip_tokenizer_encode
	static native byte[] tokenizerDecode(long tok, int[] ids);                   // ar_hip_tokenizer_decode
	static native void tokenizerDestroy(long tok);                               // ar_hip_tokenizer_destroy
}
