"""Llama2 checkpoints and tokenizer (include/ar_llama2.h) on the CPU, and the oracle's RoPE-table
input that the Llama2 GPU parity tests rely on.  No GPU.

  * header parsing: the reference's own cases (Llama2ConfigTest: shared / non-shared / GQA
    headers);
  * checkpoint layout: tensors read back from files written here in Llama2Weights order, the
    freqCis interleave on the reference's values (Llama2WeightsTest.testStageInterleaving:
    planes 1..4 and 0.1..0.4 -> 1, 0.1, 2, 0.2, ...), wcls aliasing, short and long files;
  * BPE: hand-worked merges, the reference's first-entry lookup and its errors, and random
    texts against the plain-Python restatement of BPE.java (oracle/tokenizer_oracle.py);
  * oracle: a freqCis table equal to computeRopeFreqs(theta) (rounded to fp32, as a checkpoint
    stores it) gives the theta path's tokens and logits to fp32 rounding; a table shifted by one
    position leaves them unchanged (RoPE scores depend on position differences only) and one with
    two rows swapped changes every step that attends to more than one row.
"""
import random
import struct

import numpy as np
import pytest

import oracle
from common_amd import config as C
from common_amd import hardware as hw
from common_amd.llama2 import BPE, Llama2Checkpoint, Llama2Config, write_checkpoint, write_tokenizer
from oracle import tokenizer_oracle as O


def header(*v):
    return struct.pack("<7i", *v)


def test_parse_header_reference_cases():
    c = Llama2Config.from_header(header(768, 2048, 12, 12, 12, 32000, 1024))
    assert (c.dim, c.hiddenDim, c.layerCount, c.headCount, c.kvHeadCount, c.vocabSize, c.seqLen) == \
        (768, 2048, 12, 12, 12, 32000, 1024)
    assert c.sharedWeights and c.headSize == 64
    c = Llama2Config.from_header(header(512, 1024, 6, 8, 8, -32000, 512))
    assert c.vocabSize == 32000 and not c.sharedWeights and c.headSize == 64
    c = Llama2Config.from_header(header(4096, 11008, 32, 32, 8, 32000, 2048))
    assert c.headCount == 32 and c.kvHeadCount == 8 and c.headSize == 128
    with pytest.raises(hw.HardwareException):
        Llama2Config.from_header(header(1, 2, 3, 4, 5, 6, 7)[:20])


def small_cfg(shared=True, S=3, dim=8, heads=2, F=12, L=2, V=5):
    return Llama2Config(dim, F, L, heads, heads, V, S, shared, dim // heads)


def random_weights(cfg, seed=0):
    rng = np.random.default_rng(seed)
    d, F, L, V, S, hh = cfg.dim, cfg.hidden_dim, cfg.layer_count, cfg.vocab_size, cfg.seq_len, cfg.head_size // 2
    shapes = {"tokenEmbeddings": V * d, "rmsAttWeights": L * d, "wq": L * d * d, "wk": L * d * d, "wv": L * d * d,
              "wo": L * d * d, "rmsFfn": L * d, "w1": L * F * d, "w2": L * d * F, "w3": L * F * d,
              "rmsFinalWeight": d, "freqCisReal": S * hh, "freqCisImag": S * hh, "wcls": V * d}
    return {k: rng.standard_normal(n).astype(np.float32) for k, n in shapes.items()}


@pytest.mark.parametrize("shared", [True, False])
def test_checkpoint_tensors_round_trip(tmp_path, shared):
    cfg = small_cfg(shared)
    w = random_weights(cfg)
    p = tmp_path / "m.bin"
    write_checkpoint(p, cfg, w)
    with Llama2Checkpoint(p) as ck:
        assert ck.config.dim == cfg.dim and ck.config.shared_weights == shared
        for k in ("tokenEmbeddings", "rmsAttWeights", "wq", "wk", "wv", "wo", "rmsFfn", "w1", "w2", "w3",
                  "rmsFinalWeight"):
            np.testing.assert_array_equal(ck.tensor(k), w[k], err_msg=k)
        fc = ck.tensor("freqCis").reshape(cfg.seq_len, cfg.head_size // 2, 2)
        np.testing.assert_array_equal(fc[..., 0].ravel(), w["freqCisReal"])
        np.testing.assert_array_equal(fc[..., 1].ravel(), w["freqCisImag"])
        np.testing.assert_array_equal(ck.tensor("wcls"), w["tokenEmbeddings"] if shared else w["wcls"])
        with pytest.raises(hw.HardwareException) as e:
            ck.tensor("nope")
        assert e.value.code == hw.AR_HIP_ERR_NOT_FOUND


def test_freq_cis_interleave_reference_values(tmp_path):
    # Llama2WeightsTest.testStageInterleaving: stage((2, 2, 2), take(4), take(4)) over
    # 1, 2, 3, 4, 0.1, 0.2, 0.3, 0.4 -> 1, 0.1, 2, 0.2, 3, 0.3, 4, 0.4
    cfg = small_cfg(True, S=2, dim=4, heads=1)
    w = random_weights(cfg)
    w["freqCisReal"] = np.array([1, 2, 3, 4], np.float32)
    w["freqCisImag"] = np.array([0.1, 0.2, 0.3, 0.4], np.float32)
    write_checkpoint(tmp_path / "m.bin", cfg, w)
    with Llama2Checkpoint(tmp_path / "m.bin") as ck:
        np.testing.assert_array_equal(ck.tensor("freqCis"),
                                      np.array([1, 0.1, 2, 0.2, 3, 0.3, 4, 0.4], np.float32))


def test_checkpoint_size_rules(tmp_path):
    cfg = small_cfg(False)
    w = random_weights(cfg)
    p = tmp_path / "m.bin"
    write_checkpoint(p, cfg, w)
    data = p.read_bytes()
    (tmp_path / "short.bin").write_bytes(data[:-4])
    with pytest.raises(hw.HardwareException, match="describes"):
        Llama2Checkpoint(tmp_path / "short.bin")
    (tmp_path / "long.bin").write_bytes(data + b"\0" * 12)  # trailing bytes are never read
    with Llama2Checkpoint(tmp_path / "long.bin") as ck:
        np.testing.assert_array_equal(ck.tensor("wcls"), w["wcls"])
    with pytest.raises(hw.HardwareException) as e:
        Llama2Checkpoint(tmp_path / "missing.bin")
    assert e.value.code == hw.AR_HIP_ERR_NOT_FOUND
    (tmp_path / "bad.bin").write_bytes(header(10, 4, 1, 3, 3, 5, 2) + b"\0" * 4096)  # 10 % 3 != 0
    with pytest.raises(hw.HardwareException, match="bad header"):
        Llama2Checkpoint(tmp_path / "bad.bin")


def test_checkpoint_header_overflow_is_rejected(tmp_path):
    """Header fields whose tensor sizes overflow 64 bits, or describe far more floats than the file
    holds, are rejected before any tensor offset is used (no wrapped total can pass the length
    check)."""
    big = 2 ** 31 - 1
    cases = {
        # L * F * d = (2^31-1)^3 overflows int64
        "mul.bin": header(big - 1, big, big, 1, 1, 5, 2),
        # every product fits, the sum of the tensors is ~2^62.5 floats: far past the file
        "sum.bin": header(2 ** 30, 2 ** 30, 2 ** 2, 2 ** 10, 2 ** 10, 2 ** 30, 2),
        # a negative vocabulary (separate wcls) with a sum past the file
        "wcls.bin": header(1 << 20, 4, 1, 1 << 10, 1 << 10, -(2 ** 31 - 1), 2),
    }
    for name, h in cases.items():
        (tmp_path / name).write_bytes(h + b"\0" * 4096)
        with pytest.raises(hw.HardwareException, match="describes") as e:
            Llama2Checkpoint(tmp_path / name)
        assert e.value.code == hw.AR_HIP_ERR_INVALID, name


# ---- BPE ---------------------------------------------------------------------------------------

VOCAB = ["a", "b", "c", " ", "ab", "bc", "abc", " a", "é", "ab", "日", "日本", "本"]
SCORES = [0, 0, 0, 0, 1.0, 2.0, 0.5, 3.0, 0, 9.0, 0, 1.0, 0]


def test_bpe_hand_worked():
    t = BPE(VOCAB, SCORES)
    assert t.vocab_size() == len(VOCAB)
    # lookup takes the first equal entry: "ab" is 4 although entry 9 also holds it (with score 9)
    assert t.lookup("ab") == 4 and t.lookup("zz") == -1
    # "abc": pairs ab (id 4, score 1 -- the first "ab", not entry 9's score 9) and bc (id 5, score
    # 2) -> bc first; then "a"+"bc" is entry 6 -> [abc]
    assert t.encode("abc") == [6]
    # "cab": ca is no entry, ab (1.0) -> [c, ab]; "c"+"ab" is no entry
    assert t.encode("cab") == [2, 4]
    # " ab": " a" (3.0) beats "ab" (1.0); then " a"+"b" is no entry -> [" a", "b"]
    assert t.encode(" ab") == [7, 1]
    assert t.encode("日本") == [11]
    assert t.encode("") == []
    assert t.encode("ba") == [1, 0]
    # the plain-Python restatement on the same hand-worked cases
    for text, want in (("abc", [6]), ("cab", [2, 4]), (" ab", [7, 1]), ("日本", [11]), ("", []), ("ba", [1, 0])):
        assert O.llama2_bpe_encode(text, VOCAB, np.float32(SCORES)) == want, text
    with pytest.raises(hw.HardwareException, match="no token"):
        t.encode("x")
    with pytest.raises(hw.HardwareException, match="no token"):
        t.encode("a\U0001F600")  # two UTF-16 units, neither an entry
    with pytest.raises(hw.HardwareException, match="buffer"):
        t.encode("abc", max_tokens=2)
    assert t.token(8) == "é" and t.score(7) == 3.0


def test_bpe_ties_and_score_floor():
    # equal scores: the leftmost pair merges first
    t = BPE(["a", "aa"], [0, 1])
    assert t.encode("aaa") == [1, 0] == O.llama2_bpe_encode("aaa", ["a", "aa"], [0, 1])
    # ... and a merged token can merge again: [aa, a] -> aaa
    t = BPE(["a", "aa", "aaa"], [0, 1, 5])
    assert t.encode("aaa") == [2]
    # a merge whose score does not exceed -1e10 never happens
    t = BPE(["a", "b", "ab"], [0, 0, -2e10])
    assert t.encode("ab") == [0, 1]
    t = BPE(["a", "b", "ab"], [0, 0, float("nan")])
    assert t.encode("ab") == [0, 1]


def _random_vocab(rng, n_merges=120):
    chars = list("abcde xyzé日本")
    vocab, scores = list(chars), [rng.uniform(-5, 5) for _ in chars]
    for _ in range(n_merges):
        s = rng.choice(vocab) + rng.choice(vocab)
        if len(s) > 6:
            continue
        vocab.append(s)  # duplicates allowed: lookup takes the first
        scores.append(rng.choice([rng.uniform(-5, 5), 1.0, 1.0]))
    return vocab, scores


def test_bpe_random_against_restatement():
    rng = random.Random(11)
    for trial in range(6):
        vocab, scores = _random_vocab(rng)
        t = BPE(vocab, scores)
        alpha = list("abcde xyzé日本")
        for _ in range(150):
            text = "".join(rng.choice(alpha) for _ in range(rng.randint(0, 24)))
            assert t.encode(text) == O.llama2_bpe_encode(text, vocab, np.float32(scores)), (trial, text)


def test_bpe_file(tmp_path):
    vocab = ["<unk>", "<s>", "</s>"] + VOCAB + ["�"]
    write_tokenizer(tmp_path / "tokenizer.bin", vocab, [0, 0, 0] + SCORES + [0])
    t = BPE(tmp_path / "tokenizer.bin", len(vocab))
    assert [t.token(i) for i in range(len(vocab))] == vocab
    assert t.encode(" abc") == O.llama2_bpe_encode(" abc", vocab, np.float32([0, 0, 0] + SCORES + [0]))
    # a shorter vocabulary size reads only that many entries; a longer one runs off the end
    assert BPE(tmp_path / "tokenizer.bin", 5).vocab_size() == 5
    with pytest.raises(hw.HardwareException, match="ends at entry"):
        BPE(tmp_path / "tokenizer.bin", len(vocab) + 1)
    # a negative entry length is rejected; a zero-entry vocabulary has no token for any character
    with open(tmp_path / "neg.bin", "wb") as f:
        f.write(struct.pack("<i", 4) + struct.pack("<fi", 0.0, -1))
    with pytest.raises(hw.HardwareException, match="length"):
        BPE(tmp_path / "neg.bin", 1)
    empty = BPE(tmp_path / "tokenizer.bin", 0)
    assert empty.vocab_size() == 0 and empty.encode("") == [] and empty.lookup("a") == -1
    with pytest.raises(hw.HardwareException, match="no token"):
        empty.encode("a")
    with pytest.raises(hw.HardwareException):
        BPE(tmp_path / "missing.bin", 3)
    # entry bytes that are not UTF-8 decode to U+FFFD, as new String(bytes) does
    with open(tmp_path / "bad.bin", "wb") as f:
        f.write(struct.pack("<i", 4) + struct.pack("<fi", 0.0, 3) + b"a\xffb")
    assert BPE(tmp_path / "bad.bin", 1).token(0) == "a�b"


# ---- the oracle's RoPE-table input -------------------------------------------------------------

def _tiny_llama_style_cfg():
    return C.Qwen3Config(dim=64, hidden_dim=96, layer_count=2, head_count=2, kv_head_count=2, head_size=32,
                         vocab_size=50, seq_len=8, qk_norm_mode=C.QK_NORM_WHOLE, shared_weights=True,
                         rope_theta=10000.0, epsilon=1e-5)


def _tiny_sd(cfg, seed=0):
    rng = np.random.default_rng(seed)
    d, F, V = cfg.dim, cfg.hidden_dim, cfg.vocab_size
    sd = {"model.embed_tokens.weight": rng.normal(0, 0.3, (V, d)), "model.norm.weight": 1 + rng.normal(0, .02, d)}
    for l in range(cfg.layer_count):
        p = f"model.layers.{l}."
        sd[p + "input_layernorm.weight"] = 1 + rng.normal(0, .02, d)
        sd[p + "post_attention_layernorm.weight"] = 1 + rng.normal(0, .02, d)
        for k in ("q_proj", "k_proj", "v_proj", "o_proj"):
            sd[p + f"self_attn.{k}.weight"] = rng.normal(0, 0.2, (d, d))
        sd[p + "mlp.gate_proj.weight"] = rng.normal(0, 0.2, (F, d))
        sd[p + "mlp.up_proj.weight"] = rng.normal(0, 0.2, (F, d))
        sd[p + "mlp.down_proj.weight"] = rng.normal(0, 0.2, (d, F))
    return {k: np.asarray(v, np.float32) for k, v in sd.items()}


def test_oracle_rope_table_matches_theta_path():
    cfg = _tiny_llama_style_cfg()
    sd = _tiny_sd(cfg)
    hd, S = cfg.head_size, cfg.seq_len
    # computeRopeFreqs in double, rounded to the fp32 a checkpoint stores; the theta path of the
    # FP32 oracle evaluates the same expressions in float, so compare in FP64 against a table
    # built the way the FP64 oracle builds it
    f = np.arange(hd // 2)
    invf = np.exp(f * (-2.0 * np.log(cfg.rope_theta) / hd))
    ang = np.arange(S)[:, None] * invf[None, :]
    tab64 = np.stack([np.cos(ang), np.sin(ang)], axis=-1)
    prompt = [3, 7, 1, 9]
    a = oracle.OracleQwen3(cfg, sd, precision="fp64")
    fed_a, lg_a = a.generate(prompt, 3)
    # the table goes in as fp32 (a checkpoint's values): compare against the theta path fed with the
    # same rounding, i.e. a table built from float32 cos / sin of the double angles
    b = oracle.OracleQwen3(cfg, dict(sd, freq_cis=tab64.astype(np.float32)), precision="fp64")
    fed_b, lg_b = b.generate(prompt, 3)
    assert list(fed_a) == list(fed_b)
    assert np.abs(np.asarray(lg_a) - np.asarray(lg_b)).max() < 1e-5  # fp32 rounding of the table only
    # RoPE scores depend on position differences only: a table whose row p holds angle p + 1
    # rotates every query and key one step further and leaves the logits unchanged (to the fp32
    # rounding of the table) -- as long as each position reads its own row for q and k
    shifted = np.concatenate([tab64[1:], tab64[-1:]], axis=0).astype(np.float32)
    c = oracle.OracleQwen3(cfg, dict(sd, freq_cis=shifted), precision="fp64")
    _, lg_c = c.generate(prompt, 3)
    assert np.abs(np.asarray(lg_c) - np.asarray(lg_a)).max() < 1e-5
    # swapping rows 1 and 2 changes positions 1 and 2 relative to the others; step 0 attends to one
    # row (softmax weight 1 whatever the rotation) and stays exactly the same
    swapped = tab64.copy()
    swapped[[1, 2]] = swapped[[2, 1]]
    e = oracle.OracleQwen3(cfg, dict(sd, freq_cis=swapped.astype(np.float32)), precision="fp64")
    _, lg_e = e.generate(prompt, 3)
    assert np.array_equal(lg_e[0], lg_b[0])
    for s in range(1, len(lg_e)):
        assert np.abs(lg_e[s] - lg_b[s]).max() > 1e-3, s
    with pytest.raises(KeyError):
        oracle.OracleQwen3(cfg, dict(sd, freq_cis=np.zeros((S - 1) * hd, np.float32)), precision="fp64")
