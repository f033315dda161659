"""Seeded synthetic inputs for the Qwen3 hot path.

The reference's synthetic tests draw weights from ``java.util.Random`` in row-major
order (compute/algebra/src/main/java/org/almostrealism/collect/computations/Random.java:214-220);
that stream cannot be reproduced without a JVM, so this build uses its own documented,
counter-based generator (common_amd/csrc/synth/ar_synth.c):

* tensor ``key`` under ``seed`` is stream ``crc32(key)``; element i is a pure function of
  (seed, stream, i), so values do not depend on thread count or request order;
* projection and embedding matrices are N(0, 0.02); RMSNorm and QK-norm gains are
  N(1, 0.02) (gains of N(0, 0.02) would shrink every normalised activation ~50x);
* for bf16 configurations every value is rounded to the nearest bfloat16 (ties to even)
  and returned as float32, so the GPU path and the oracle see identical numbers;
* prompt token ids are uniform in [0, vocab), stream ``0x70726f6d + row``.

Keys are the HF state-dict names ``Qwen3.model`` reads
(engine/ml/src/main/java/org/almostrealism/ml/qwen3/Qwen3.java:338-384).
"""
from __future__ import annotations

import ctypes
import zlib

import numpy as np

from . import _native
from .config import DTYPE_BF16, Qwen3Config

STD = 0.02
PROMPT_STREAM = 0x70726F6D


def _lib():
    lib = _native.load_synth()
    if not getattr(lib, "_ar_typed", False):
        lib.ar_synth_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double,
                                        ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
        lib.ar_synth_uniform_ids.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int32,
                                             ctypes.c_void_p, ctypes.c_int64]
        lib.ar_synth_bf16_round.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        lib._ar_typed = True
    return lib


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 precision (round-to-nearest-even), as float32."""
    out = np.array(a, dtype=np.float32, copy=True, order="C")
    _lib().ar_synth_bf16_round(out.ctypes.data, out.size)
    return out


def normal_tensor(key: str, shape, seed: int, mean: float = 0.0, std: float = STD,
                  bf16: bool = False) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    _lib().ar_synth_normal(seed, zlib.crc32(key.encode()), mean, std, out.ctypes.data, out.size, int(bf16))
    return out


def weight_specs(cfg: Qwen3Config):
    """(key, shape, is_gain) for every tensor of the model, in HF naming."""
    d, qd, kd, f, v, hd = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden_dim, cfg.vocab_size, cfg.head_size
    specs = [("model.embed_tokens.weight", (v, d), False), ("model.norm.weight", (d,), True)]
    if not cfg.shared_weights:
        specs.append(("lm_head.weight", (v, d), False))
    for i in range(cfg.layer_count):
        p = f"model.layers.{i}."
        specs += [
            (p + "input_layernorm.weight", (d,), True),
            (p + "self_attn.q_proj.weight", (qd, d), False),
            (p + "self_attn.k_proj.weight", (kd, d), False),
            (p + "self_attn.v_proj.weight", (kd, d), False),
            (p + "self_attn.o_proj.weight", (d, qd), False),
            (p + "self_attn.q_norm.weight", (cfg.head_count, hd), True),
            (p + "self_attn.k_norm.weight", (cfg.kv_head_count, hd), True),
            (p + "post_attention_layernorm.weight", (d,), True),
            (p + "mlp.gate_proj.weight", (f, d), False),
            (p + "mlp.up_proj.weight", (f, d), False),
            (p + "mlp.down_proj.weight", (d, f), False),
        ]
        if cfg.qkv_bias:
            specs += [(p + "self_attn.q_proj.bias", (qd,), False),
                      (p + "self_attn.k_proj.bias", (kd,), False),
                      (p + "self_attn.v_proj.bias", (kd,), False)]
    return specs


def iter_state_dict(cfg: Qwen3Config, seed: int = 0):
    """Yields (key, float32 array) one tensor at a time, so a large model never needs two
    full copies in host memory."""
    bf16 = cfg.weight_dtype == DTYPE_BF16
    for key, shape, gain in weight_specs(cfg):
        yield key, normal_tensor(key, shape, seed, mean=1.0 if gain else 0.0, bf16=bf16)


def state_dict(cfg: Qwen3Config, seed: int = 0) -> dict:
    return dict(iter_state_dict(cfg, seed))


def prompt_ids(n: int, vocab: int, seed: int = 0, batch: int = 1) -> np.ndarray:
    """Prompt token ids uniform in [0, vocab): shape (n,) for batch 1, else (batch, n)."""
    out = np.empty((batch, n), dtype=np.int32)
    for b in range(batch):
        _lib().ar_synth_uniform_ids(seed, PROMPT_STREAM + b, vocab, out[b].ctypes.data, n)
    return out[0] if batch == 1 else out
