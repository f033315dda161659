/*
 * The Qwen3 decode / prefill step on a HIP GPU, with AutoregressiveModel's contract
 * (engine/ml/src/main/java/org/almostrealism/ml/AutoregressiveModel.java:194-308): reset, setPrompt,
 * next, getCurrentStep, get/setTemperature, plus the batched forms of this backend (one handle
 * decodes up to 8 independent sequences; next() of a batch returns one token per sequence).
 *
 * Qwen3.model (engine/ml/src/main/java/org/almostrealism/ml/qwen3/Qwen3.java:334-415) builds it
 * instead of the compiled graph when the local hardware has a HipDataContext:
 *
 *   HipQwen3 m = HipQwen3.fromWeights(hip, weightsDirectory, 1, HIP.DTYPE_F32, HIP.DTYPE_F32, seqLen);
 *   m.setPrompt(promptTokens, promptTokens.length);
 *   m.prefill();                     // optional: the whole prompt at once, same state as the next() calls
 *   for (...) token = m.next();
 *
 * Not compiled in this repository (no JDK in the build image).
 */
package org.almostrealism.hardware.hip;

import io.almostrealism.profile.OperationProfileNode;

import java.util.ArrayList;
import java.util.HashMap;
import java.util.List;
import java.util.Map;

public class HipQwen3 implements AutoCloseable {
	private final HipDataContext context;
	private long model;
	private final int maxBatch;
	private final int vocabSize;
	private double temperature;
	private Integer currentToken;

	private HipQwen3(HipDataContext context, long model) {
		this.context = context;
		this.model = model;
		this.maxBatch = HIP.qwen3MaxBatch(model);
		this.vocabSize = HIP.qwen3VocabSize(model);
	}

	/**
	 * A model from a StateDictionary directory (protobuf CollectionLibraryData files), its
	 * configuration inferred as Qwen3.inferConfigFromWeights does (Qwen3.java:197-239), then the
	 * fields the reference leaves to the caller: sequences decoded together, weight storage
	 * (DTYPE_F32 as the reference computes, or DTYPE_BF16), KV-cache storage and capacity.
	 */
	public static HipQwen3 fromWeights(HipDataContext context, String weightsDirectory, int maxBatch, int weightDtype,
									   int kvDtype, int seqLen) {
		long dict = HIP.stateDictOpen(weightsDirectory);
		try {
			int[] ints = new int[14];
			double[] doubles = new double[2];
			HIP.qwen3InferConfig(dict, ints, doubles);
			ints[7] = seqLen;
			ints[8] = maxBatch;
			ints[9] = weightDtype;
			ints[13] = kvDtype;
			long m = HIP.qwen3Create(context.getHandle(), ints, doubles);
			try {
				HIP.qwen3LoadStateDict(m, dict);
				HIP.qwen3Finalize(m);
			} catch (RuntimeException e) {
				HIP.qwen3Destroy(m);
				throw e;
			}
			return new HipQwen3(context, m);
		} finally {
			HIP.stateDictDestroy(dict);
		}
	}

	/**
	 * Llama2.model over a llama2.c checkpoint (engine/ml/src/main/java/org/almostrealism/ml/llama2/
	 * Llama2.java:173-201): the same decoder with the checkpoint's weights and RoPE table.
	 */
	public static HipQwen3 fromLlama2(HipDataContext context, String checkpoint, int maxBatch, int weightDtype,
									  int kvDtype) {
		long ck = HIP.llama2Open(checkpoint);
		try {
			return new HipQwen3(context, HIP.llama2CreateModel(context.getHandle(), ck, maxBatch, weightDtype, kvDtype));
		} finally {
			HIP.llama2Close(ck);
		}
	}

	public int getMaxBatch() { return maxBatch; }

	public int getVocabSize() { return vocabSize; }

	private long handle() {
		if (model == 0) throw new IllegalStateException("model destroyed");
		return model;
	}

	/** AutoregressiveModel.getCurrentStep: the position of the next step. */
	public int getCurrentStep() { return HIP.qwen3Position(handle()); }

	/** AutoregressiveModel.reset: position 0; the prompts are kept. */
	public void reset() {
		HIP.qwen3Reset(handle());
		currentToken = null;
	}

	/** AutoregressiveModel.setPrompt for sequence 0 (batch 1). */
	public void setPrompt(Integer[] promptTokens, int length) {
		int[] ids = new int[length];
		for (int i = 0; i < length; i++) ids[i] = promptTokens[i];
		setPrompt(0, ids);
	}

	/** The prompt of sequence seq; all sequences of a batch share one prompt length. */
	public void setPrompt(int seq, int[] ids) { HIP.qwen3SetPrompt(handle(), seq, ids); }

	public Integer getCurrentToken() { return currentToken; }

	public double getTemperature() { return temperature; }

	/** AutoregressiveModel.setTemperature: 0 is greedy (indexOfMax), else the model's sampler. */
	public void setTemperature(double temperature) {
		HIP.qwen3SetSampling(handle(), HIP.SAMPLE_MODEL, temperature, 1.0, null);
		this.temperature = temperature;
	}

	/** One java.util.Random seed per sequence for the sampler (the reference's is unseeded). */
	public void setSeeds(long[] seeds) {
		HIP.qwen3SetSampling(handle(), HIP.SAMPLE_MODEL, temperature, 1.0, seeds);
	}

	/** AutoregressiveModel.next (batch 1): the token fed at this step. */
	public Integer next() {
		if (maxBatch != 1) throw new IllegalStateException("batch of " + maxBatch + ": use nextAll()");
		currentToken = HIP.qwen3Next(handle(), null)[0];
		return currentToken;
	}

	/** next() of every sequence: maxBatch tokens. */
	public int[] nextAll() { return HIP.qwen3Next(handle(), null); }

	/** next() of every sequence with this step's logits copied into logits (maxBatch x vocab). */
	public int[] nextAll(float[] logits) { return HIP.qwen3Next(handle(), logits); }

	/** steps calls of next() enqueued back to back: maxBatch x steps tokens, row-major by sequence. */
	public int[] run(int steps) { return HIP.qwen3Run(handle(), steps); }

	/** The whole prompt at once; leaves the model where prompt-length calls of next() would. */
	public void prefill() { HIP.qwen3Prefill(handle(), null); }

	/** Which kernels run the bf16 prefill's projections: HIP.PREFILL_GEMM_ROCBLAS, the default, or
	 *  HIP.PREFILL_GEMM_OWN, the library's fused MFMA kernels; results agree within float rounding. */
	public void setPrefillGemm(int backend) { HIP.qwen3PrefillGemm(handle(), backend); }

	public int getPrefillGemm() { return HIP.qwen3PrefillGemmBackend(handle()); }

	// the separate-launch step's classes in step order, and their node names (common_amd/profile.py
	// builds the same tree from Python)
	private static final int[] STEP_CLASSES = {HIP.KT_QKV, HIP.KT_ATTENTION, HIP.KT_O, HIP.KT_GATE_UP, HIP.KT_DOWN,
			HIP.KT_LOGITS};
	private static final String[] STEP_NAMES = {"rmsnorm + dense qkv", "qk-norm + rope + attention",
			"dense o + residual", "rmsnorm + dense gate/up + swiglu", "dense down + residual",
			"rmsnorm + logits + indexOfMax"};

	/**
	 * The decode step as a profile tree in the reference's format (io.almostrealism.profile
	 * .OperationProfileNode, base/code/src/main/java/io/almostrealism/profile/OperationProfileNode.java:
	 * 188-460, which Qwen3.java:189-190 installs on the compiled model): steps decode steps timed per
	 * kernel class, each node's metric holding the class's summed seconds and launch count.  Under the
	 * root, the persistent launch (when the model runs it) and the step as separate launches, one node
	 * per class.  The model advances steps x 7 positions (x 6 without the persistent launch); save()
	 * writes the tree as the reference's XML.
	 */
	public OperationProfileNode profile(int steps) {
		if (steps < 1) throw new IllegalArgumentException("steps must be >= 1");
		List<OperationProfileNode> children = new ArrayList<>();
		boolean persistent = HIP.qwen3Persistent(handle());
		try {
			if (persistent) {
				children.add(timed(HIP.KT_LAYERS, "decode_persistent (layers + final norm + logits + argmax keys)",
						steps));
				HIP.qwen3UsePersistent(handle(), false);
			}
			List<OperationProfileNode> classes = new ArrayList<>();
			for (int i = 0; i < STEP_CLASSES.length; i++) classes.add(timed(STEP_CLASSES[i], STEP_NAMES[i], steps));
			OperationProfileNode separate = new OperationProfileNode("separate launches per stage");
			separate.setChildren(classes);
			children.add(separate);
		} finally {
			if (persistent) HIP.qwen3UsePersistent(handle(), true);
		}
		OperationProfileNode root = new OperationProfileNode("decode: " + steps + " steps per class");
		root.setChildren(children);
		return root;
	}

	private OperationProfileNode timed(int which, String name, int steps) {
		double[] t;
		HIP.qwen3KernelTiming(handle(), which);
		try {
			HIP.qwen3Run(handle(), steps);
			t = HIP.qwen3KernelTime(handle());
		} finally {
			HIP.qwen3KernelTiming(handle(), HIP.KT_NONE);
		}
		OperationProfileNode n = new OperationProfileNode(name);
		n.setMetricEntries(new HashMap<>(Map.of(name, t[0] / 1000.0)));
		n.setMetricCounts(new HashMap<>(Map.of(name, (int) t[1])));
		return n;
	}

	@Override
	public void close() {
		if (model != 0) {
			HIP.qwen3Destroy(model);
			model = 0;
		}
	}
}
