"""Weights in the reference's protobuf format, mirroring ``StateDictionary``.

``StateDictionary(path)`` reads a weights directory (or one file) of serialized
``CollectionLibraryData`` messages (engine/ml/src/main/proto/collections.proto:1-27) the way
``StateDictionary.loadWeights`` does (engine/ml/src/main/java/org/almostrealism/ml/
StateDictionary.java:119-150); ``get`` / ``containsKey`` / ``keySet`` / ``size`` / ``put`` /
``save`` / ``destroy`` keep the reference's names and meaning.  Parsing, storage and writing
are in the native library (include/ar_state_dict.h): files are memory-mapped and
``Qwen3(config, StateDictionary)`` and ``Qwen3.from_weights_directory`` move packed fp32
payloads from the mapping to the device.

``save_split`` writes the layout of engine/ml/qwen/tools/extract_qwen3_weights.py:108-170
(``embeddings`` + ``layer_NN`` files), which is what ``Qwen3(weightsDirectory)`` reads.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

from . import hardware as hw
from .config import DTYPE_F32, Qwen3Config
from .qwen3 import _Cfg

DTYPE_F64 = hw.DTYPE_F64
MAX_DIMS = 8


class StateDictionary:
    """HF-keyed tensors backed by the native dictionary (StateDictionary.java)."""

    def __init__(self, source: str | os.PathLike | dict | None = None):
        h = ctypes.c_void_p()
        if source is None or isinstance(source, dict):
            hw.check(hw.lib().ar_hip_state_dict_create(ctypes.byref(h)))
            self.handle = h.value
            for k, v in (source or {}).items():
                self.put(k, v)
        else:
            hw.check(hw.lib().ar_hip_state_dict_open(os.fsencode(source), ctypes.byref(h)))
            self.handle = h.value

    # ---- StateDictionary API -----------------------------------------------------------
    def size(self) -> int:
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_state_dict_size(self._h(), ctypes.byref(n)))
        return n.value

    def keySet(self) -> list[str]:  # noqa: N802 (reference name)
        out = []
        k = ctypes.c_char_p()
        for i in range(self.size()):
            hw.check(hw.lib().ar_hip_state_dict_key(self._h(), i, ctypes.byref(k)))
            out.append(k.value.decode())
        return out

    def containsKey(self, key: str) -> bool:  # noqa: N802
        f = ctypes.c_int()
        hw.check(hw.lib().ar_hip_state_dict_contains(self._h(), key.encode(), ctypes.byref(f)))
        return bool(f.value)

    def info(self, key: str):
        """(shape, traversal_axis, stored dtype, element count) of one tensor."""
        nd, ax, dt, n = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
        dims = (ctypes.c_int32 * MAX_DIMS)()
        hw.check(hw.lib().ar_hip_state_dict_info(self._h(), key.encode(), ctypes.byref(nd), dims, ctypes.byref(ax),
                                                 ctypes.byref(dt), ctypes.byref(n)))
        return tuple(dims[i] for i in range(nd.value)), ax.value, dt.value, n.value

    def get(self, key: str, dtype=np.float32) -> np.ndarray | None:
        """The tensor's values in its shape (None for an unknown key, as Map.get)."""
        if not self.containsKey(key):
            return None
        if np.dtype(dtype) not in (np.float32, np.float64):
            raise ValueError("values are read as float32 or float64")
        shape, _, _, n = self.info(key)
        out = np.empty(n, dtype=dtype)
        code = DTYPE_F64 if out.dtype == np.float64 else DTYPE_F32
        hw.check(hw.lib().ar_hip_state_dict_read(self._h(), key.encode(), code, out.ctypes.data, n))
        return out.reshape(shape)

    def getAllWeights(self) -> dict:  # noqa: N802
        return {k: self.get(k) for k in self.keySet()}

    def put(self, key: str, value, traversal_axis: int = 0):
        a = np.asarray(value)
        if a.dtype != np.float64:
            a = a.astype(np.float32)
        a = np.ascontiguousarray(a)
        shape = a.shape if a.ndim else (1,)
        dims = (ctypes.c_int32 * len(shape))(*shape)
        code = DTYPE_F64 if a.dtype == np.float64 else DTYPE_F32
        hw.check(hw.lib().ar_hip_state_dict_put(self._h(), key.encode(), dims, len(shape), traversal_axis,
                                                a.ctypes.data, code, a.size))

    def save(self, path: str | os.PathLike, precision: int = DTYPE_F32):
        """StateDictionary.save(Path, Precision): one file, data_32 (fp32) or data (fp64)."""
        hw.check(hw.lib().ar_hip_state_dict_save(self._h(), os.fsencode(path), precision))

    def files(self) -> tuple[int, int]:
        """(files parsed, files skipped after a parse failure) of the directory that was read."""
        a, b = ctypes.c_int(), ctypes.c_int()
        hw.check(hw.lib().ar_hip_state_dict_files(self._h(), ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def infer_config(self) -> Qwen3Config:
        """Qwen3.inferConfigFromWeights (Qwen3.java:197-239)."""
        c = _Cfg()
        hw.check(hw.lib().ar_hip_qwen3_infer_config(self._h(), ctypes.byref(c)))
        return Qwen3Config(dim=c.dim, hidden_dim=c.hidden_dim, layer_count=c.layer_count, head_count=c.head_count,
                           kv_head_count=c.kv_head_count, vocab_size=c.vocab_size, seq_len=c.seq_len,
                           head_size=c.head_size, shared_weights=bool(c.shared_weights), rope_theta=c.rope_theta,
                           epsilon=c.epsilon, qk_norm_mode=c.qk_norm_mode, qkv_bias=bool(c.qkv_bias))

    def destroy(self):
        if getattr(self, "handle", None):
            hw.check(hw.lib().ar_hip_state_dict_destroy(self.handle))
            self.handle = None

    # ---- helpers -------------------------------------------------------------------------
    def _h(self):
        if not self.handle:
            raise hw.HardwareException(hw.AR_HIP_ERR_STATE, "state dictionary was destroyed")
        return self.handle

    def __contains__(self, key):
        return self.containsKey(key)

    def __len__(self):
        return self.size()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


_LAYER = re.compile(r"^model\.layers\.(\d+)\.")


def save_split(weights, directory: str | os.PathLike, precision: int = DTYPE_F32) -> list[str]:
    """Writes ``weights`` (dict or iterable of (key, array)) as extract_qwen3_weights.py lays a
    model out: ``embeddings`` (embed_tokens, final norm, lm_head) and one ``layer_NN`` file per
    transformer layer (engine/ml/qwen/tools/extract_qwen3_weights.py:108-170)."""
    os.makedirs(directory, exist_ok=True)
    groups: dict[str, StateDictionary] = {}
    items = weights.items() if isinstance(weights, dict) else weights
    for k, v in items:
        m = _LAYER.match(k)
        name = f"layer_{int(m.group(1)):02d}" if m else "embeddings"
        groups.setdefault(name, StateDictionary()).put(k, v)
    paths = []
    for name, sd in sorted(groups.items()):
        p = os.path.join(directory, name)
        sd.save(p, precision)
        sd.destroy()
        paths.append(p)
    return paths
