"""Qwen3 model runtime on the HIP backend, mirroring the reference's model API.

``Qwen3(config, state_dict)`` builds the device model from HF-named tensors as
``Qwen3.model`` does (engine/ml/src/main/java/org/almostrealism/ml/qwen3/Qwen3.java:334-415),
and ``Qwen3.model`` returns an ``AutoregressiveModel`` with the reference's
``reset`` / ``set_prompt`` / ``next`` token loop
(engine/ml/src/main/java/org/almostrealism/ml/AutoregressiveModel.java:203-220,295-308).
All work happens in the native library (include/ar_hip.h).
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

from . import hardware as hw
from .config import DTYPE_BF16, Qwen3Config

KT_NONE, KT_LOGITS, KT_GATE_UP, KT_QKV, KT_ATTENTION, KT_DOWN, KT_O, KT_LAYERS = range(8)
# ar_hip_qwen3_prefill_gemm backends: the library's MFMA kernels, or rocBLAS gemm_ex
PREFILL_GEMM_OWN, PREFILL_GEMM_ROCBLAS = 0, 1


class _Cfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "dim", "hidden_dim", "layer_count", "head_count", "kv_head_count", "head_size", "vocab_size", "seq_len",
        "max_batch", "weight_dtype", "qk_norm_mode", "shared_weights", "qkv_bias", "kv_dtype")] + [
        ("rope_theta", ctypes.c_double), ("epsilon", ctypes.c_double)]


def native_cfg(c: Qwen3Config) -> _Cfg:
    return _Cfg(c.dim, c.hidden_dim, c.layer_count, c.head_count, c.kv_head_count, c.head_size, c.vocab_size,
                c.seq_len, c.max_batch, c.weight_dtype, c.qk_norm_mode, int(c.shared_weights), int(c.qkv_bias), c.kv_dtype,
                c.rope_theta, c.epsilon)


class AutoregressiveModel:
    """Token loop over the device model: prompt tokens are fed one per step, then the greedy
    choice from the previous step's logits (AutoregressiveModel.next, :295-308)."""

    def __init__(self, qwen: "Qwen3"):
        self.qwen = qwen
        self.batch = qwen.config.max_batch

    @property
    def handle(self):
        return self.qwen.handle

    def reset(self):
        hw.check(hw.lib().ar_hip_qwen3_reset(self.handle))

    def set_prompt(self, ids, seq: int = 0):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        hw.check(hw.lib().ar_hip_qwen3_set_prompt(self.handle, seq, ids.ctypes.data, ids.size))

    def next(self, return_logits: bool = False):
        toks = np.empty(self.batch, dtype=np.int32)
        logits = np.empty((self.batch, self.qwen.config.vocab_size), dtype=np.float32) if return_logits else None
        hw.check(hw.lib().ar_hip_qwen3_next(self.handle, toks.ctypes.data,
                                            logits.ctypes.data if return_logits else None))
        return (toks, logits) if return_logits else toks

    def prefill(self, return_logits: bool = False):
        """The whole prompt at once (MFMA path for bf16 weights); afterwards the model is where
        prompt-length next() calls would leave it.  Optionally returns the last prompt row's logits."""
        logits = np.empty((self.batch, self.qwen.config.vocab_size), dtype=np.float32) if return_logits else None
        hw.check(hw.lib().ar_hip_qwen3_prefill(self.handle, logits.ctypes.data if return_logits else None))
        return logits

    def run(self, steps: int) -> np.ndarray:
        """``steps`` calls of next() without host synchronisation; returns (batch, steps) tokens."""
        out = np.empty((self.batch, steps), dtype=np.int32)
        hw.check(hw.lib().ar_hip_qwen3_run(self.handle, steps, out.ctypes.data))
        return out

    def prefill_by_steps(self) -> int:
        """Prefill calls of this model that went through the decode step (fp32 weights, or a value
        outside the fp16 range of the bf16 path's MFMA operands)."""
        v = ctypes.c_int()
        hw.check(hw.lib().ar_hip_qwen3_prefill_by_steps(self.handle, ctypes.byref(v)))
        return v.value

    def get_current_step(self) -> int:
        v = ctypes.c_int()
        hw.check(hw.lib().ar_hip_qwen3_position(self.handle, ctypes.byref(v)))
        return v.value

    def hidden(self) -> np.ndarray:
        out = np.empty((self.batch, self.qwen.config.dim), dtype=np.float32)
        hw.check(hw.lib().ar_hip_qwen3_hidden(self.handle, out.ctypes.data))
        return out

    def set_temperature(self, temperature: float):
        """AutoregressiveModel.setTemperature (AutoregressiveModel.java:258-260): 0 is greedy, any
        other value samples with the sample function of AutoregressiveModel.of (:413-425)."""
        hw.check(hw.lib().ar_hip_qwen3_set_sampling(self.handle, hw.SAMPLE_MODEL, float(temperature), 1.0, None))

    def set_sampling(self, mode: int, temperature: float, top_p: float = 1.0, seeds=None):
        """Token selection: hw.SAMPLE_MODEL (the reference model's sample function) or
        hw.SAMPLE_TOKEN (AutoregressiveModel.sampleToken with top_p); ``seeds`` (one per sequence)
        reseed the per-sequence java.util.Random generators."""
        sd = None
        if seeds is not None:
            sd = np.ascontiguousarray(np.broadcast_to(np.asarray(seeds, dtype=np.int64), (self.batch,)))
        hw.check(hw.lib().ar_hip_qwen3_set_sampling(self.handle, int(mode), float(temperature), float(top_p),
                                                    sd.ctypes.data if sd is not None else None))

    def use_graph(self, enable: bool):
        hw.check(hw.lib().ar_hip_qwen3_use_graph(self.handle, int(enable)))

    def use_fragment_gemv(self, enable: bool):
        """Batches of 3..8 with bf16 weights: the decode step's O, gate/up and down GEMVs read copies
        of those matrices in MFMA fragment order made at finalize (default on), split evenly over
        every wavefront, or (False) the row-major weights."""
        hw.check(hw.lib().ar_hip_qwen3_use_fragment_gemv(self.handle, int(enable)))

    @property
    def fragment_gemv(self) -> bool:
        """Whether the decode steps use the fragment-ordered GEMVs."""
        a = ctypes.c_int()
        hw.check(hw.lib().ar_hip_qwen3_fragment_gemv(self.handle, ctypes.byref(a)))
        return bool(a.value)

    def use_persistent(self, enable: bool):
        """Run the layers of each decode step as one persistent launch when the model qualifies
        (default on) or as separate launches.  It qualifies at batch 1 with an fp32 or fp16 KV cache
        on the three instantiated shapes: d1024/F3072, 16/8 heads of 128, fp32 weights (Qwen3-0.6B),
        d2048/F6144, 16/8 heads of 128, bf16 weights (Qwen3-1.7B) and d768/F2048, 12/12 heads of 64,
        fp32 weights (llama2.c stories110M).  A call whose persistent launch
        timed out (blocks not resident together) is recomputed as separate launches and switches
        the model to them until this is called with True again."""
        hw.check(hw.lib().ar_hip_qwen3_use_persistent(self.handle, int(enable)))

    @property
    def persistent_recomputed(self) -> int:
        """Steps recomputed as separate launches after a timed-out persistent launch."""
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_qwen3_persistent_recomputed(self.handle, ctypes.byref(n)))
        return n.value

    def persistent_wait_limit(self, polls: int):
        """Polls of one cross-block wait of the persistent kernel before it is abandoned (0: the
        default).  A test knob: a tiny limit makes the waits time out while every block still runs
        to its end."""
        hw.check(hw.lib().ar_hip_qwen3_persistent_wait_limit(self.handle, int(polls)))

    @property
    def persistent(self) -> bool:
        """Whether the next decode steps run their layers in the persistent kernel."""
        a = ctypes.c_int()
        hw.check(hw.lib().ar_hip_qwen3_persistent(self.handle, ctypes.byref(a)))
        return bool(a.value)

    @property
    def prefill_gemm(self) -> int:
        """Which kernels run the bf16 prefill's projections: PREFILL_GEMM_ROCBLAS (default) or
        PREFILL_GEMM_OWN (the library's fused MFMA kernels)."""
        a = ctypes.c_int()
        hw.check(hw.lib().ar_hip_qwen3_prefill_gemm_backend(self.handle, ctypes.byref(a)))
        return a.value

    @prefill_gemm.setter
    def prefill_gemm(self, backend: int):
        hw.check(hw.lib().ar_hip_qwen3_prefill_gemm(self.handle, int(backend)))

    def kernel_timing(self, which: int):
        hw.check(hw.lib().ar_hip_qwen3_kernel_timing(self.handle, which))

    def kernel_time(self):
        ms = ctypes.c_double()
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_qwen3_kernel_time(self.handle, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def kernel_loop(self, which: int, reps: int) -> float:
        """Average launch duration (µs) of kernel class `which` over `reps` graph-replayed launches
        cycling through the layers (ar_hip_qwen3_kernel_loop); call reset() before the next step."""
        us = ctypes.c_double()
        hw.check(hw.lib().ar_hip_qwen3_kernel_loop(self.handle, which, reps, ctypes.byref(us)))
        return us.value


class Qwen3:
    """Device-resident Qwen3 built from an HF-keyed state dict (or an iterator of (key, tensor))."""

    def __init__(self, config: Qwen3Config, state_dict, ctx: hw.HipContext | None = None, tokenizer=None):
        self.config = config
        self.tokenizer = tokenizer  # a common_amd.tokenizer.Qwen3Tokenizer, for run(); optional
        self.ctx = ctx or hw.HipContext()
        self._own_ctx = ctx is None
        h = ctypes.c_void_p()
        cfg = native_cfg(config)
        hw.check(hw.lib().ar_hip_qwen3_create(self.ctx.handle, ctypes.byref(cfg), ctypes.byref(h)))
        self.handle = h.value
        from .state_dict import StateDictionary
        if isinstance(state_dict, StateDictionary):
            # protobuf weights: packed fp32 payloads go from the mapped files to the device
            hw.check(hw.lib().ar_hip_qwen3_load_state_dict(self.handle, state_dict.handle))
        else:
            items = state_dict.items() if isinstance(state_dict, dict) else state_dict
            for key, t in items:
                self.set_weight(key, t)
        hw.check(hw.lib().ar_hip_qwen3_finalize(self.handle))
        self.model = AutoregressiveModel(self)

    @classmethod
    def from_weights_directory(cls, path, tokenizer_path=None, config: Qwen3Config | None = None,
                               ctx: hw.HipContext | None = None, **config_fields) -> "Qwen3":
        """Qwen3(String weightsDirectory, tokenizerPath, config) (Qwen3.java:154-190): reads the
        protobuf weights with StateDictionary and, without a config, infers one from the weight
        shapes (Qwen3.inferConfigFromWeights); ``config_fields`` override fields of the inferred
        config (e.g. seq_len, max_batch, weight_dtype).  The tokenizer is optional, as there."""
        from .state_dict import StateDictionary
        from .tokenizer import Qwen3Tokenizer
        tok = Qwen3Tokenizer(tokenizer_path) if tokenizer_path is not None else None
        with StateDictionary(path) as sd:
            if config is None:
                config = dataclasses.replace(sd.infer_config(), **config_fields)
            return cls(config, sd, ctx, tokenizer=tok)

    def run(self, steps: int, prompt: str | None, output, prefill: bool = True) -> float:
        """Qwen3.run (Qwen3.java:426-478): encodes the prompt with BOS, feeds it and generates until
        `steps` positions or EOS, handing each token's text to ``output`` between "<|im_start|>\n"
        and "<|im_end|>"; returns the milliseconds after the first token.  The token loop is the
        device model's (greedy, or the sampling set with AutoregressiveModel.set_sampling).  With
        ``prefill`` the prompt runs as one batched prefill (the reference feeds it one token per
        step; the model ends in the same state) and its tokens are emitted as they would be."""
        import time

        from .tokenizer import BOS_TOKEN, EOS_TOKEN
        if steps <= 0 or steps > self.config.seq_len:
            steps = self.config.seq_len
        if self.tokenizer is None:
            raise RuntimeError("No tokenizer loaded. Cannot process text input.")
        ids = self.tokenizer.encode(prompt, True, False) if prompt is not None else []
        am = self.model
        am.reset()
        # setCurrentToken(BOS) + an empty prompt: the first step feeds BOS
        am.set_prompt(ids if ids else [BOS_TOKEN])
        output("<|im_start|>\n")
        start = 0.0
        if prefill and len(ids) > 1 and len(ids) < steps:
            am.prefill()
            for t in ids:
                output(self.tokenizer.decode([t]))
        while am.get_current_step() < steps:
            nxt = int(am.next()[0])
            output(self.tokenizer.decode([nxt]))
            if nxt == EOS_TOKEN:
                break
            if start == 0.0:
                start = time.perf_counter()
        output("<|im_end|>")
        return 1000.0 * (time.perf_counter() - start) if start else 0.0

    def set_weight(self, key: str, t: np.ndarray):
        t = np.ascontiguousarray(t, dtype=np.float32)
        hw.check(hw.lib().ar_hip_qwen3_set_weight(self.handle, key.encode(), t.ctypes.data, hw.DTYPE_F32, t.size))

    def close(self):
        if self.handle:
            hw.check(hw.lib().ar_hip_qwen3_destroy(self.handle))
            self.handle = None
        if self._own_ctx and self.ctx:
            self.ctx.close()
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def weight_bytes(self) -> int:
        return 2 if self.config.weight_dtype == DTYPE_BF16 else 4
