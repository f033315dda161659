"""Llama2 on the HIP decoder, mirroring the reference's Llama2 classes
(engine/ml/src/main/java/org/almostrealism/ml/llama2/): ``Llama2(checkpoint, tokenizer)`` maps a
llama2.c checkpoint (``Llama2Config`` from its header, ``Llama2Weights`` layout), builds the device
model as ``Llama2.model`` does (Llama2.java:173-201) and exposes ``setTemperature`` and
``run(steps, prompt, output)`` (Llama2.java:211-258); ``BPE`` is the score-driven tokenizer of
BPE.java.  All work happens in the native library (include/ar_llama2.h); the token loop is the
``AutoregressiveModel`` of common_amd.qwen3, which serves both families.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os
import struct
import time

import numpy as np

from . import hardware as hw
from .config import DTYPE_F32
from .qwen3 import AutoregressiveModel

BOS = 1  # llama2.c's <s>, fed at position 0 (Llama2.java:220)


class _Cfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "dim", "hidden_dim", "layer_count", "head_count", "kv_head_count", "vocab_size", "seq_len", "shared_weights",
        "head_size")]


@dataclasses.dataclass
class Llama2Config:
    """TransformerConfig as read from a checkpoint header (TransformerConfig.java:69-80)."""
    dim: int
    hidden_dim: int
    layer_count: int
    head_count: int
    kv_head_count: int
    vocab_size: int
    seq_len: int
    shared_weights: bool
    head_size: int
    max_batch: int = 1

    @classmethod
    def from_header(cls, header: bytes) -> "Llama2Config":
        c = _Cfg()
        hw.check(hw.lib().ar_hip_llama2_parse_config(bytes(header), len(header), ctypes.byref(c)))
        return cls._of(c)

    @classmethod
    def _of(cls, c: _Cfg) -> "Llama2Config":
        return cls(c.dim, c.hidden_dim, c.layer_count, c.head_count, c.kv_head_count, c.vocab_size, c.seq_len,
                   bool(c.shared_weights), c.head_size)

    # the reference's field names
    hiddenDim = property(lambda s: s.hidden_dim)  # noqa: N815
    layerCount = property(lambda s: s.layer_count)  # noqa: N815
    headCount = property(lambda s: s.head_count)  # noqa: N815
    kvHeadCount = property(lambda s: s.kv_head_count)  # noqa: N815
    vocabSize = property(lambda s: s.vocab_size)  # noqa: N815
    seqLen = property(lambda s: s.seq_len)  # noqa: N815
    sharedWeights = property(lambda s: s.shared_weights)  # noqa: N815
    headSize = property(lambda s: s.head_size)  # noqa: N815


class Llama2Checkpoint:
    """A mapped llama2.c checkpoint; ``tensor(name)`` returns a copy of a Llama2Weights field
    (``freqCis`` with its two planes interleaved, as Llama2Weights stages it)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        hw.check(hw.lib().ar_hip_llama2_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h.value
        c = _Cfg()
        hw.check(hw.lib().ar_hip_llama2_config(self.handle, ctypes.byref(c)))
        self.config = Llama2Config._of(c)

    def tensor(self, name: str) -> np.ndarray:
        p, n = ctypes.c_void_p(), ctypes.c_int64()
        hw.check(hw.lib().ar_hip_llama2_tensor(self.handle, name.encode(), ctypes.byref(p), ctypes.byref(n)))
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), shape=(n.value,)).copy()

    def close(self):
        if getattr(self, "handle", None):
            hw.check(hw.lib().ar_hip_llama2_close(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class BPE:
    """The llama2.c vocabulary with scores and BPE.encode / BPE.lookup (BPE.java:33-101).
    ``BPE(path, vocab_size)`` reads tokenizer.bin as the Llama2 constructor does
    (Llama2.java:130-146); ``BPE(vocab, scores)`` takes the strings directly."""

    def __init__(self, source, vocab_size_or_scores):
        h = ctypes.c_void_p()
        if isinstance(source, (str, os.PathLike)):
            hw.check(hw.lib().ar_hip_bpe_load(os.fsencode(source), int(vocab_size_or_scores), ctypes.byref(h)))
        else:
            vocab = [v.encode("utf-8") if isinstance(v, str) else bytes(v) for v in source]
            n = len(vocab)
            arr = (ctypes.c_char_p * max(n, 1))(*vocab)
            sc = np.ascontiguousarray(vocab_size_or_scores if n else [0.0], dtype=np.float32)
            hw.check(hw.lib().ar_hip_bpe_create(arr, sc.ctypes.data, n, ctypes.byref(h)))
        self.handle = h.value

    def vocab_size(self) -> int:
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_bpe_vocab_size(self.handle, ctypes.byref(n)))
        return n.value

    def token(self, i: int) -> str:
        p, n, sc = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_float()
        hw.check(hw.lib().ar_hip_bpe_token(self.handle, i, ctypes.byref(p), ctypes.byref(n), ctypes.byref(sc)))
        return ctypes.string_at(p, n.value).decode("utf-8")

    def score(self, i: int) -> float:
        p, n, sc = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_float()
        hw.check(hw.lib().ar_hip_bpe_token(self.handle, i, ctypes.byref(p), ctypes.byref(n), ctypes.byref(sc)))
        return sc.value

    def lookup(self, text: str) -> int:
        b = text.encode("utf-8")
        i = ctypes.c_int()
        hw.check(hw.lib().ar_hip_bpe_lookup(self.handle, b, len(b), ctypes.byref(i)))
        return i.value

    def encode(self, text: str, max_tokens: int | None = None) -> list[int]:
        b = text.encode("utf-8")
        cap = max_tokens if max_tokens is not None else len(text.encode("utf-16-le")) // 2
        out = np.empty(max(cap, 1), dtype=np.int32)
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_bpe_encode(self.handle, b, len(b), out.ctypes.data, cap, ctypes.byref(n)))
        return out[: n.value].tolist()

    def close(self):
        if getattr(self, "handle", None):
            hw.check(hw.lib().ar_hip_bpe_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Llama2:
    """Llama2(checkpoint, tokenizer) (Llama2.java:107-162): the checkpoint's config and weights on
    the device, the tokenizer read with the checkpoint's vocabulary size, and ``model`` the
    AutoregressiveModel (greedy until ``setTemperature``)."""

    def __init__(self, checkpoint, tokenizer="tokenizer.bin", ctx: hw.HipContext | None = None, max_batch: int = 1,
                 weight_dtype: int = DTYPE_F32, kv_dtype: int = DTYPE_F32):
        self.handle = None
        with Llama2Checkpoint(checkpoint) as ck:
            self.config = dataclasses.replace(ck.config, max_batch=max_batch)
            self.tokenizer = BPE(tokenizer, self.config.vocab_size) if tokenizer is not None else None
            self.ctx = ctx or hw.HipContext()
            self._own_ctx = ctx is None
            h = ctypes.c_void_p()
            try:
                hw.check(hw.lib().ar_hip_llama2_create_model(self.ctx.handle, ck.handle, max_batch, weight_dtype,
                                                             kv_dtype, ctypes.byref(h)))
            except Exception:
                self.close()
                raise
            self.handle = h.value
        self.model = AutoregressiveModel(self)

    def setTemperature(self, temperature: float):  # noqa: N802 (reference name)
        """Llama2.setTemperature -> AutoregressiveModel.setTemperature: 0 is greedy."""
        self.model.set_temperature(temperature)

    def run(self, steps: int, prompt: str | None, output) -> int:
        """Llama2.run (Llama2.java:211-258): BOS at position 0, then the BPE-encoded prompt, fed one
        token per step; every token fed after the prompt goes to ``output`` as its vocabulary string
        (its leading space dropped right after BOS), after a first "<s>\\n".  Returns the milliseconds
        from the first generated token."""
        if steps <= 0 or steps > self.config.seq_len:
            steps = self.config.seq_len
        if self.tokenizer is None:
            raise RuntimeError("Llama2.run needs a tokenizer")
        ids = [BOS]
        if prompt is not None:
            ids += self.tokenizer.encode(prompt, self.config.seq_len)
        count = len(ids)
        am = self.model
        am.reset()
        am.set_prompt(ids)
        output("<s>\n")
        start = 0.0
        token = BOS
        while am.get_current_step() < steps:
            nxt = int(am.next()[0])
            if am.get_current_step() > count:
                s = self.tokenizer.token(nxt)
                output(s[1:] if token == BOS and s.startswith(" ") else s)
            token = nxt
            if start == 0.0 and am.get_current_step() > count:
                start = time.perf_counter()
        return 0 if start == 0.0 else int(1000.0 * (time.perf_counter() - start))

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


def write_checkpoint(path, cfg: Llama2Config, weights: dict):
    """Writes a llama2.c checkpoint: the header (vocabulary size negated when the classifier is
    stored) and the fp32 tensors in Llama2Weights order.  ``weights`` holds the Llama2Weights field
    names, layer-stacked; "freqCisReal" / "freqCisImag" are the two RoPE planes (seqLen x
    headSize/2) and "wcls" is needed only when the weights are not shared."""
    names = ["tokenEmbeddings", "rmsAttWeights", "wq", "wk", "wv", "wo", "rmsFfn", "w1", "w2", "w3",
             "rmsFinalWeight", "freqCisReal", "freqCisImag"] + ([] if cfg.shared_weights else ["wcls"])
    with open(path, "wb") as f:
        v = cfg.vocab_size if cfg.shared_weights else -cfg.vocab_size
        f.write(struct.pack("<7i", cfg.dim, cfg.hidden_dim, cfg.layer_count, cfg.head_count, cfg.kv_head_count, v,
                            cfg.seq_len))
        for n in names:
            f.write(np.ascontiguousarray(weights[n], dtype="<f4").tobytes())


def write_tokenizer(path, vocab, scores, max_token_length: int | None = None):
    """Writes a llama2.c tokenizer.bin: int32 max token length, then (float32 score, int32 length,
    UTF-8 bytes) per entry."""
    enc = [v.encode("utf-8") if isinstance(v, str) else bytes(v) for v in vocab]
    with open(path, "wb") as f:
        f.write(struct.pack("<i", max_token_length if max_token_length is not None else max((len(b) for b in enc),
                                                                                            default=0)))
        for b, s in zip(enc, scores):
            f.write(struct.pack("<fi", float(s), len(b)))
            f.write(b)
