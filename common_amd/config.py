"""Qwen3 shape contract and the five benchmark configurations.

Mirrors ``Qwen3Config`` / ``TransformerConfig``
(engine/ml/src/main/java/org/almostrealism/ml/qwen3/Qwen3Config.java:104-109,
engine/ml/src/main/java/org/almostrealism/ml/TransformerConfig.java:79,104) with the
same field names.  The reference hard-wires ``headSize = dim / headCount``; this
config carries ``head_size`` explicitly so that shapes with ``heads * headSize != dim``
(Qwen3-0.6B, Qwen3-4B) are expressible.  When ``heads * headSize == dim`` every
computation reduces to the reference graph.
"""
from __future__ import annotations

import dataclasses
import os

QK_NORM_WHOLE = 0     # one RMS over the whole q / k vector (AttentionFeatures.java:840-845, :886-891)
QK_NORM_PER_HEAD = 1  # one RMS per head (HF Qwen3 semantics)

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2  # KV-cache storage option (kv_dtype)


def default_kv_dtype() -> int:
    """KV-cache storage of a config that does not name one: AR_HIP_KV_DTYPE = "fp32" (default, the
    reference keeps its cache at the context precision) or "fp16"."""
    v = os.environ.get("AR_HIP_KV_DTYPE", "fp32").strip().lower()
    if v in ("fp32", "f32", "float32", ""):
        return DTYPE_F32
    if v in ("fp16", "f16", "float16", "half"):
        return DTYPE_F16
    raise ValueError(f"AR_HIP_KV_DTYPE={v!r}: expected fp32 or fp16")


@dataclasses.dataclass(frozen=True)
class Qwen3Config:
    dim: int
    hidden_dim: int           # FFN width (TransformerConfig.hiddenDim)
    layer_count: int
    head_count: int
    kv_head_count: int
    vocab_size: int
    seq_len: int              # KV-cache capacity in positions
    head_size: int = 0        # 0 -> dim // head_count, as TransformerConfig.java:79
    shared_weights: bool = True
    rope_theta: float = 1_000_000.0
    epsilon: float = 1e-6     # Qwen3.java:397,402
    qk_norm_mode: int = QK_NORM_WHOLE
    weight_dtype: int = DTYPE_F32
    kv_dtype: int = dataclasses.field(default_factory=lambda: default_kv_dtype())
    # KV cache storage: DTYPE_F32 (reference) or DTYPE_F16; default from AR_HIP_KV_DTYPE
    max_batch: int = 1
    qkv_bias: bool = False

    def __post_init__(self):
        if self.head_size == 0:
            object.__setattr__(self, "head_size", self.dim // self.head_count)
        self.validate()

    @property
    def q_dim(self) -> int:
        return self.head_count * self.head_size

    @property
    def kv_dim(self) -> int:
        return self.kv_head_count * self.head_size

    def validate(self):
        """Qwen3Config.validate (Qwen3Config.java:165-183), with an explicit head size."""
        if self.head_count % self.kv_head_count != 0:
            raise ValueError(f"headCount ({self.head_count}) must be divisible by "
                             f"kvHeadCount ({self.kv_head_count})")
        if min(self.layer_count, self.head_count, self.kv_head_count) <= 0:
            raise ValueError("Layer and head counts must be positive")
        if self.vocab_size <= 0 or self.seq_len <= 0:
            raise ValueError("Vocabulary size and sequence length must be positive")
        if self.head_size % 2 != 0:
            raise ValueError("head size must be even for split-half RoPE")

    def param_count(self) -> int:
        d, qd, kd, f = self.dim, self.q_dim, self.kv_dim, self.hidden_dim
        per_layer = qd * d + 2 * kd * d + d * qd + 3 * f * d + 2 * d + qd + kd
        if self.qkv_bias:
            per_layer += qd + 2 * kd
        head = 0 if self.shared_weights else self.vocab_size * d
        return self.layer_count * per_layer + self.vocab_size * d + d + head

    def layer_weight_params(self) -> int:
        d, qd, kd, f = self.dim, self.q_dim, self.kv_dim, self.hidden_dim
        return qd * d + 2 * kd * d + d * qd + 3 * f * d


# BASELINE.json configs ------------------------------------------------------------
# C1: tiny Qwen3-architecture decoder (runs on the reference's CPU path).
C1_TINY = Qwen3Config(dim=256, hidden_dim=768, layer_count=2, head_count=4, kv_head_count=2,
                      vocab_size=1024, seq_len=48, head_size=64)
C1_PROMPT, C1_DECODE = 16, 32

# C2: single-layer decode-step GQA attention op (16 Q / 8 KV heads, hd 128, cache 4096 + 1).
C2_HEADS, C2_KV_HEADS, C2_HEAD_SIZE, C2_POS = 16, 8, 128, 4096

# C3: Qwen3-0.6B shape, fp32, prompt 128 + 256 greedy decode (the north-star metric).
C3_0_6B = Qwen3Config(dim=1024, hidden_dim=3072, layer_count=28, head_count=16, kv_head_count=8,
                      vocab_size=151936, seq_len=384, head_size=128)
C3_PROMPT, C3_DECODE = 128, 256

# C4: Qwen3-1.7B shape, bf16 weights / fp32 accumulation, prefill 2048 + decode 128.
C4_1_7B = Qwen3Config(dim=2048, hidden_dim=6144, layer_count=28, head_count=16, kv_head_count=8,
                      vocab_size=151936, seq_len=2176, head_size=128, weight_dtype=DTYPE_BF16)
C4_PROMPT, C4_DECODE = 2048, 128

# C5: Qwen3-4B shape, bf16 weights, batch 8 x 8192-token context, decode 64 each.
C5_4B = Qwen3Config(dim=2560, hidden_dim=9728, layer_count=36, head_count=32, kv_head_count=8,
                    vocab_size=151936, seq_len=8256, head_size=128, weight_dtype=DTYPE_BF16,
                    max_batch=8)
C5_PROMPT, C5_DECODE, C5_BATCH = 8192, 64, 8
