"""TEST INFRASTRUCTURE ONLY: a plain-Python restatement of the reference tokenizer, the checker
for the native ones (common_amd/csrc/tokenizer.cpp, common_amd/csrc/bpe.cpp).  Only tests/ import it.

  * pre-tokenisation: the reference's pattern (RegexPreTokenizer.java:89-98) run by the `regex`
    package's backtracking engine, with Java's ASCII meaning of \\s / \\S written out (Python's
    \\s is Unicode whitespace);
  * byte-level mapping (ByteLevelEncoder.java): GPT-2's byte-to-character table;
  * BPE (ByteLevelBPETokenizer.applyBPEMerges): merge the lowest-priority adjacent pair, the
    leftmost on ties, one at a time;
  * Qwen3Tokenizer.encode(text, addBos, addEos) / decode (Qwen3Tokenizer.java:271-296,
    ByteLevelBPETokenizer.decode), merges.txt parsing (loadMergesFromFile, :150-199);
  * llama2.c's score-driven BPE (BPE.java:33-101): llama2_bpe_encode.
"""
from __future__ import annotations

import regex

BOS, EOS, PAD, UNK = 151643, 151645, 151643, 128244

_JS = r"[ \t\n\x0B\f\r]"       # Java \s
_JNS = r"[^ \t\n\x0B\f\r]"     # Java \S
PATTERN = regex.compile(
    r"'s|'t|'re|'ve|'m|'ll|'d"
    r"|[^\r\n\p{L}\p{N}]?\p{L}+"
    r"|\p{N}"
    r"| ?[^ \t\n\x0B\f\r\p{L}\p{N}]+[\r\n]*"
    r"|" + _JS + r"*[\r\n]+"
    r"|" + _JS + r"+(?!" + _JNS + r")"
    r"|" + _JS + r"+")


def pretokenize(text: str) -> list[str]:
    return [m.group(0) for m in PATTERN.finditer(text) if m.group(0)]


def byte_to_char() -> dict[int, str]:
    table, n = {}, 0
    for b in range(256):
        if ord("!") <= b <= ord("~") or 161 <= b <= 172 or 174 <= b <= 255:
            table[b] = chr(b)
        else:
            table[b] = chr(256 + n)
            n += 1
    return table


_B2C = byte_to_char()
_TRIM = "".join(chr(c) for c in range(0x21))
_C2B = {c: b for b, c in _B2C.items()}


class Tokenizer:
    def __init__(self, vocab: list[str], merges_lines: list[str] | None = None):
        self.vocab = list(vocab)
        self.ids = {}
        for i, v in enumerate(self.vocab):
            self.ids[v] = i
        self.merges = {}
        if merges_lines is not None:
            priority = 0
            for line in merges_lines:
                if line.startswith("#") or not line.strip(_TRIM):  # String.trim: chars <= U+0020
                    continue
                if " " not in line:
                    continue
                a, b = line.split(" ", 1)
                if a not in self.ids or b not in self.ids or (a + b) not in self.ids:
                    priority += 1
                    continue
                self.merges[a + " " + b] = (a + b, priority)
                priority += 1

    def bpe(self, tokens: list[str]) -> list[str]:
        if len(tokens) <= 1 or not self.merges:
            return tokens
        while True:
            best, best_pri, best_m = -1, None, None
            for i in range(len(tokens) - 1):
                m = self.merges.get(tokens[i] + " " + tokens[i + 1])
                if m is not None and (best_pri is None or m[1] < best_pri):
                    best, best_pri, best_m = i, m[1], m[0]
            if best < 0:
                return tokens
            tokens = tokens[:best] + [best_m] + tokens[best + 2:]

    def encode(self, text: str, add_bos: bool, add_eos: bool) -> list[int]:
        special = add_bos or add_eos
        ids = [BOS] if special else []
        for seg in pretokenize(text):
            chars = [_B2C[b] for b in seg.encode("utf-8")]
            ids += [self.ids.get(t, UNK) for t in self.bpe(chars)]
        if special:
            ids.append(EOS)
            if not add_bos and ids and ids[0] == BOS:
                ids = ids[1:]
            if not add_eos and ids and ids[-1] == EOS:
                ids = ids[:-1]
        return ids

    def decode(self, ids) -> str:
        s = "".join(self.vocab[i] for i in ids if i not in (BOS, EOS, PAD, UNK) and 0 <= i < len(self.vocab))
        return bytes(_C2B[c] for c in s).decode("utf-8", errors="replace")


# ---- llama2.c score-driven BPE (engine/ml/.../BPE.java) ---------------------------------------

def llama2_bpe_encode(text: str, vocab: list[str], scores) -> list[int]:
    """BPE.encode (BPE.java:57-101) with BPE.lookup's linear scan for the first equal entry
    (:33-41).  Java strings are UTF-16: the text is split into UTF-16 units, so a supplementary
    character becomes two lone surrogates that no entry equals (the reference throws; so does this).
    Scores compare as float32 against a floor of -1e10f."""
    import numpy as np
    raw = text.encode("utf-16-le", "surrogatepass")
    units = [raw[i:i + 2].decode("utf-16-le", "surrogatepass") for i in range(0, len(raw), 2)]

    def lookup(s):
        for i, v in enumerate(vocab):
            if v == s:
                return i
        return -1

    tokens = []
    for u in units:
        i = lookup(u)
        if i == -1:
            raise ValueError(f"no token for {u!r}")
        tokens.append(i)
    while True:
        best_score, best_id, best_index = np.float32(-1e10), -1, -1
        for i in range(len(tokens) - 1):
            j = lookup(vocab[tokens[i]] + vocab[tokens[i + 1]])
            if j != -1 and np.float32(scores[j]) > best_score:
                best_score, best_id, best_index = np.float32(scores[j]), j, i
        if best_index == -1:
            return tokens
        tokens[best_index] = best_id
        del tokens[best_index + 1]
