"""The Qwen3 byte-level BPE tokenizer, mirroring ``Qwen3Tokenizer``
(engine/ml/src/main/java/org/almostrealism/ml/qwen3/Qwen3Tokenizer.java) with the reference's
names: ``Qwen3Tokenizer(path)`` / ``Qwen3Tokenizer(vocab, scores)``, ``encode``, ``decode``,
``getVocabSize``, ``createTestTokenizer``.  The work happens in the native library
(include/ar_tokenizer.h); text is passed as UTF-8.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import hardware as hw

BOS_TOKEN = 151643
EOS_TOKEN = 151645
PAD_TOKEN = 151643
UNK_TOKEN = 128244


class Qwen3Tokenizer:
    BOS_TOKEN, EOS_TOKEN, PAD_TOKEN, UNK_TOKEN = BOS_TOKEN, EOS_TOKEN, PAD_TOKEN, UNK_TOKEN

    def __init__(self, source, scores=None):
        h = ctypes.c_void_p()
        if isinstance(source, (str, os.PathLike)):
            hw.check(hw.lib().ar_hip_tokenizer_load(os.fsencode(source), ctypes.byref(h)))
        else:
            vocab = [v.encode("utf-8") if isinstance(v, str) else bytes(v) for v in source]
            n = len(vocab)
            arr = (ctypes.c_char_p * max(n, 1))(*vocab)
            lens = np.array([len(v) for v in vocab] or [0], dtype=np.int32)
            sc = np.ascontiguousarray(scores if scores is not None else np.zeros(max(n, 1)), dtype=np.float32)
            hw.check(hw.lib().ar_hip_tokenizer_from_vocab(arr, lens.ctypes.data, sc.ctypes.data, n, ctypes.byref(h)))
        self.handle = h.value

    @classmethod
    def createTestTokenizer(cls) -> "Qwen3Tokenizer":  # noqa: N802 (reference name)
        """Qwen3Tokenizer.createTestTokenizer (Qwen3Tokenizer.java:317-346): 256 "<0xNN>" byte
        entries and a few words, no merges."""
        vocab = [f"<0x{i:02X}>" for i in range(256)]
        common = [" ", "the", "a", "an", "and", "or", "is", "in", "to", "of", "Hello", "World", "!", "?", ".", ",",
                  "\n", "Once", "upon", "time", "there", "was"]
        vocab += common
        scores = [float(i) for i in range(256)] + [256.0 + i for i in range(len(common))]
        return cls(vocab, scores)

    def load_merges(self, path):
        hw.check(hw.lib().ar_hip_tokenizer_load_merges(self.handle, os.fsencode(path)))

    def getVocabSize(self) -> int:  # noqa: N802
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_tokenizer_vocab_size(self.handle, ctypes.byref(n)))
        return n.value

    def merge_count(self) -> int:
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_tokenizer_merge_count(self.handle, ctypes.byref(n)))
        return n.value

    def token(self, i: int) -> str:
        p, n, sc = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_float()
        hw.check(hw.lib().ar_hip_tokenizer_token(self.handle, i, ctypes.byref(p), ctypes.byref(n), ctypes.byref(sc)))
        return ctypes.string_at(p, n.value).decode("utf-8")

    def encode(self, text: str, add_bos: bool | None = None, add_eos: bool | None = None) -> list[int]:
        """encode(text, addBos, addEos); encode(text) adds both, as Qwen3Tokenizer.encode(String)."""
        if add_bos is None and add_eos is None:
            add_bos = add_eos = True
        b = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        n = ctypes.c_int()
        hw.check(hw.lib().ar_hip_tokenizer_encode(self.handle, b, len(b), int(bool(add_bos)), int(bool(add_eos)),
                                                  None, 0, ctypes.byref(n)))
        out = np.empty(max(n.value, 1), dtype=np.int32)
        hw.check(hw.lib().ar_hip_tokenizer_encode(self.handle, b, len(b), int(bool(add_bos)), int(bool(add_eos)),
                                                  out.ctypes.data, n.value, ctypes.byref(n)))
        return out[: n.value].tolist()

    def decode(self, ids) -> str:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        ln = ctypes.c_int64()
        hw.check(hw.lib().ar_hip_tokenizer_decode(self.handle, a.ctypes.data, a.size, None, 0, ctypes.byref(ln)))
        buf = ctypes.create_string_buffer(ln.value + 1)
        hw.check(hw.lib().ar_hip_tokenizer_decode(self.handle, a.ctypes.data, a.size, buf, ln.value + 1,
                                                  ctypes.byref(ln)))
        return buf.raw[: ln.value].decode("utf-8")

    def close(self):
        if getattr(self, "handle", None):
            hw.check(hw.lib().ar_hip_tokenizer_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pretokenize(text: str) -> list[str]:
    """RegexPreTokenizer.preTokenize (RegexPreTokenizer.java:89-116) through the native scanner."""
    b = text.encode("utf-8")
    n = ctypes.c_int()
    hw.check(hw.lib().ar_hip_tokenizer_pretokenize(b, len(b), None, 0, ctypes.byref(n)))
    offs = np.empty(max(2 * n.value, 2), dtype=np.int64)
    hw.check(hw.lib().ar_hip_tokenizer_pretokenize(b, len(b), offs.ctypes.data, n.value, ctypes.byref(n)))
    return [b[offs[2 * k]:offs[2 * k + 1]].decode("utf-8") for k in range(n.value)]


def write_tokenizer(path, vocab, scores=None, merges=None):
    """Writes the reference's binary vocabulary (int32 count; per token float32 score, int32 length,
    UTF-8 bytes; little-endian: extract_qwen3_weights.py's tokenizer.bin) and, when given, a
    merges.txt beside it ("first second" per line)."""
    import struct
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(vocab)))
        for i, v in enumerate(vocab):
            b = v.encode("utf-8")
            f.write(struct.pack("<fi", float(scores[i]) if scores is not None else 0.0, len(b)))
            f.write(b)
    if merges is not None:
        with open(os.path.join(os.path.dirname(os.path.abspath(path)), "merges.txt"), "w", encoding="utf-8") as f:
            f.write("#version: 0.2\n")
            for a, b in merges:
                f.write(f"{a} {b}\n")
