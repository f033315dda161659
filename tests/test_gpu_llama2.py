"""Llama2 on the GPU (include/ar_llama2.h) against the CPU oracle, through the C-ABI.

The model is Llama2.model's graph (Llama2.java:173-201): AttentionFeatures.transformer with
heads == kvHeads, no QK-norm, eps 1e-5, the checkpoint's freqCis as the RoPE table, and the
classifier tied or stored.  The oracle runs the same graph from the same checkpoint tensors,
mapped to the roles Llama2.model passes them in (transformer(heads, rmsAtt, wk, wv, wq, wo,
freqCis, rmsFfn, w1, w2, w3, ...)).  Bars as for Qwen3: greedy tokens bit-exact against the FP64
oracle (up to a genuine near-tie of the oracle's own logits), logits within 1e-4 (fp32 weights)
and 2e-2 (bf16 weights) of max |logit|.  Llama2.run's text output is checked against a
restatement of its loop (Llama2.java:211-258) fed with the oracle's tokens and BPE.encode's
restatement.
"""
import random

import numpy as np
import pytest

import oracle
from common_amd import config as C
from common_amd import hardware as hw
from common_amd.llama2 import BOS, Llama2, Llama2Config, write_checkpoint, write_tokenizer
from conftest import rel_err
from oracle import tokenizer_oracle as O

pytestmark = pytest.mark.gpu
NEAR_TIE = 1e-5


def make_weights(cfg: Llama2Config, seed=0):
    rng = np.random.default_rng(seed)
    d, F, L, V, S, hd = cfg.dim, cfg.hidden_dim, cfg.layer_count, cfg.vocab_size, cfg.seq_len, cfg.head_size
    w = {"tokenEmbeddings": rng.normal(0, 0.5, (V, d)), "rmsAttWeights": 1 + rng.normal(0, 0.05, (L, d)),
         "wq": rng.normal(0, 0.06, (L, d, d)), "wk": rng.normal(0, 0.06, (L, d, d)),
         "wv": rng.normal(0, 0.06, (L, d, d)), "wo": rng.normal(0, 0.06, (L, d, d)),
         "rmsFfn": 1 + rng.normal(0, 0.05, (L, d)), "w1": rng.normal(0, 0.06, (L, F, d)),
         "w2": rng.normal(0, 0.06, (L, d, F)), "w3": rng.normal(0, 0.06, (L, F, d)),
         "rmsFinalWeight": 1 + rng.normal(0, 0.05, d), "wcls": rng.normal(0, 0.5, (V, d))}
    # the planes llama2.c's export writes: cos / sin of pos * theta^(-2f/hd), theta 10000
    invf = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    ang = np.outer(np.arange(S), invf)
    w["freqCisReal"], w["freqCisImag"] = np.cos(ang), np.sin(ang)
    return {k: np.asarray(v, np.float32) for k, v in w.items()}


def bf16_round(a):
    """fp32 -> nearest bfloat16 (ties to even), back in fp32; finite inputs."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32).reshape(np.shape(a))


def oracle_model(cfg: Llama2Config, w, precision="fp64", round_bf16=False):
    """The checkpoint tensors in the roles Llama2.model gives them, on the oracle's decoder."""
    qc = C.Qwen3Config(dim=cfg.dim, hidden_dim=cfg.hidden_dim, layer_count=cfg.layer_count,
                       head_count=cfg.head_count, kv_head_count=cfg.head_count, vocab_size=cfg.vocab_size,
                       seq_len=cfg.seq_len, head_size=cfg.head_size, shared_weights=cfg.shared_weights,
                       rope_theta=10000.0, epsilon=1e-5)
    r = bf16_round if round_bf16 else (lambda a: a)
    sd = {"model.embed_tokens.weight": r(w["tokenEmbeddings"]), "model.norm.weight": w["rmsFinalWeight"],
          "freq_cis": np.stack([w["freqCisReal"], w["freqCisImag"]], axis=-1).ravel()}
    if not cfg.shared_weights:
        sd["lm_head.weight"] = r(w["wcls"])
    for l in range(cfg.layer_count):
        p = f"model.layers.{l}."
        sd[p + "input_layernorm.weight"] = w["rmsAttWeights"][l]
        sd[p + "self_attn.q_proj.weight"] = r(w["wq"][l])
        sd[p + "self_attn.k_proj.weight"] = r(w["wk"][l])
        sd[p + "self_attn.v_proj.weight"] = r(w["wv"][l])
        sd[p + "self_attn.o_proj.weight"] = r(w["wo"][l])
        sd[p + "post_attention_layernorm.weight"] = w["rmsFfn"][l]
        sd[p + "mlp.gate_proj.weight"] = r(w["w1"][l])
        sd[p + "mlp.down_proj.weight"] = r(w["w2"][l])
        sd[p + "mlp.up_proj.weight"] = r(w["w3"][l])
    return oracle.OracleQwen3(qc, sd, precision=precision)


def gpu_generate(model, prompt, n_decode):
    am = model.model
    am.reset()
    am.set_prompt(prompt)
    fed, logits = [], []
    for _ in range(len(prompt) + n_decode):
        t, lg = am.next(return_logits=True)
        fed.append(int(t[0]))
        logits.append(lg[0])
    return fed, np.stack(logits)


def compare_tokens(gpu_fed, ref_fed, ref_logits, n_prompt):
    for s in range(n_prompt, len(ref_fed)):
        if gpu_fed[s] != ref_fed[s]:
            top2 = np.sort(ref_logits[s - 1])[-2:]
            margin = (top2[1] - top2[0]) / max(abs(top2[1]), 1e-30)
            assert margin < NEAR_TIE, f"token mismatch at step {s}: gpu {gpu_fed[s]} ref {ref_fed[s]}"
            return s
    return len(ref_fed)


CFG_SHARED = Llama2Config(256, 512, 2, 4, 4, 384, 40, True, 64)
CFG_SEPARATE = Llama2Config(256, 512, 2, 4, 4, 384, 40, False, 64)


@pytest.mark.parametrize("cfg", [CFG_SHARED, CFG_SEPARATE], ids=["shared", "separate"])
def test_llama2_tokens_and_logits_vs_fp64_oracle(ctx, tmp_path, cfg):
    w = make_weights(cfg, seed=1)
    write_checkpoint(tmp_path / "model.bin", cfg, w)
    prompt = [BOS, 17, 230, 5, 99, 301]
    n_dec = 20
    print(f"[llama2] {'shared' if cfg.shared_weights else 'separate'} classifier, {len(prompt)}+{n_dec} steps",
          flush=True)
    ref_fed, ref_logits = oracle_model(cfg, w).generate(prompt, n_dec)
    with Llama2(tmp_path / "model.bin", None, ctx) as m:
        assert m.config == cfg
        fed, logits = gpu_generate(m, prompt, n_dec)
    assert compare_tokens(fed, ref_fed, ref_logits, len(prompt)) == len(ref_fed)
    assert rel_err(logits, np.asarray(ref_logits)) <= 1e-4


def test_llama2_bf16_weights(ctx, tmp_path):
    cfg = CFG_SEPARATE
    w = make_weights(cfg, seed=2)
    write_checkpoint(tmp_path / "model.bin", cfg, w)
    prompt = [BOS, 3, 200, 71]
    ref_fed, ref_logits = oracle_model(cfg, w, round_bf16=True).generate(prompt, 8)
    with Llama2(tmp_path / "model.bin", None, ctx, weight_dtype=C.DTYPE_BF16) as m:
        am = m.model
        am.reset()
        am.set_prompt(ref_fed)  # the oracle's tokens, so both see the same inputs
        logits = np.stack([am.next(return_logits=True)[1][0] for _ in range(len(ref_fed))])
    assert rel_err(logits, np.asarray(ref_logits)) <= 2e-2


def test_llama2_bf16_prefill_matches_token_by_token(ctx, tmp_path):
    """A bf16 Llama2 model's batched prefill (MFMA GEMMs + causal flash attention with the checkpoint's
    RoPE table, head size 64) leaves the model where feeding the prompt one token per step does:
    the next step's logits agree within the bf16 bar and the greedy continuations match."""
    cfg = CFG_SHARED
    w = make_weights(cfg, seed=6)
    write_checkpoint(tmp_path / "model.bin", cfg, w)
    prompt = [BOS] + [int(x) for x in np.random.default_rng(9).integers(3, cfg.vocab_size, 30)]
    with Llama2(tmp_path / "model.bin", None, ctx, weight_dtype=C.DTYPE_BF16) as m:
        am = m.model
        am.reset()
        am.set_prompt(prompt)
        last = am.prefill(return_logits=True)[0]
        assert am.get_current_step() == len(prompt)
        cont_pf = [int(am.next()[0]) for _ in range(6)]
        am.reset()
        am.set_prompt(prompt)
        for _ in range(len(prompt)):
            _, lg = am.next(return_logits=True)
        ref_last = lg[0]
        cont_tt = [int(am.next()[0]) for _ in range(6)]
    assert rel_err(last, ref_last) <= 2e-2
    # the token chosen from those logits, fed at the first step after the prompt (unless the two paths'
    # fp16 / fp32 activations could swap a near-tie)
    top2 = np.sort(ref_last)[-2:]
    if (top2[1] - top2[0]) > 2e-2 * np.abs(ref_last).max():
        assert cont_pf[0] == cont_tt[0]


def _vocab(V, rng):
    """A llama2.c-style vocabulary: specials, single characters, then merged strings with scores."""
    chars = list("abcdefghij klmno.")
    vocab, scores = ["<unk>", "<s>", "</s>"] + chars, [0.0, 0.0, 0.0] + [rng.uniform(-9, -5) for _ in chars]
    while len(vocab) < V:
        s = rng.choice(vocab[3:]) + rng.choice(vocab[3:])
        if len(s) <= 5 and s not in vocab:
            vocab.append(s)
            scores.append(rng.uniform(-5, 5))
    return vocab, scores


@pytest.mark.parametrize("prompt", [None, "ab cd.ef klmn"])
def test_llama2_run_text(ctx, tmp_path, prompt):
    cfg = CFG_SHARED
    w = make_weights(cfg, seed=3)
    write_checkpoint(tmp_path / "model.bin", cfg, w)
    vocab, scores = _vocab(cfg.vocab_size, random.Random(5))
    write_tokenizer(tmp_path / "tokenizer.bin", vocab, scores)
    steps = 24
    got = []
    with Llama2(tmp_path / "model.bin", tmp_path / "tokenizer.bin", ctx) as m:
        m.setTemperature(0.0)
        m.run(steps, prompt, got.append)
    # Llama2.run restated over the oracle's tokens
    ids = [BOS] + (O.llama2_bpe_encode(prompt, vocab, np.float32(scores)) if prompt is not None else [])
    ref_fed, _ = oracle_model(cfg, w).generate(ids, steps - len(ids), want_logits=False)
    want, token = ["<s>\n"], BOS
    for step, nxt in enumerate(ref_fed, start=1):
        if step > len(ids):
            s = vocab[nxt]
            want.append(s[1:] if token == BOS and s.startswith(" ") else s)
        token = nxt
    assert got == want


def test_llama2_temperature_samples_with_the_model_function(ctx, tmp_path):
    """setTemperature(T) != 0 installs AutoregressiveModel.of's sample function (a java.util.Random
    per sequence, seeded 0): the tokens equal the FP64 oracle model driven by that function until a
    draw lands within 1e-7 of a cumulative boundary."""
    cfg = CFG_SHARED
    w = make_weights(cfg, seed=4)
    write_checkpoint(tmp_path / "model.bin", cfg, w)
    prompt = [BOS, 10, 20]
    n_dec = 16
    with Llama2(tmp_path / "model.bin", None, ctx) as m:
        m.setTemperature(0.9)
        fed, _ = gpu_generate(m, prompt, n_dec)
    g = oracle.JavaRandom(0)
    margins = []

    def sampler(lg):
        k, _, mg = oracle.model_sample(lg, 0.9, g)
        margins.append(mg)
        return k

    rf, _ = oracle_model(cfg, w).generate(prompt, n_dec, want_logits=False, sampler=sampler)
    compared = 0
    for s in range(len(prompt), len(rf)):
        if margins[s - len(prompt)] < 1e-7:
            break
        assert fed[s] == rf[s], f"step {s}"
        compared += 1
    assert compared >= 6


def test_llama2_unsupported_shapes(ctx, tmp_path):
    cfg = Llama2Config(96, 128, 1, 2, 2, 64, 8, True, 48)  # head size 48: no attention kernel
    write_checkpoint(tmp_path / "model.bin", cfg, make_weights(cfg))
    with pytest.raises(hw.HardwareException, match="head size"):
        Llama2(tmp_path / "model.bin", None, ctx)


def test_llama2_stories_shape_persistent_vs_oracle_and_multi_launch(ctx, tmp_path):
    """The persistent decode step at the llama2.c stories110M layer shape (d 768, 12 heads of 64 =
    KV heads, F 2048, fp32, no QK-norm gains; 2 layers and a 1000-word tied head here): QKV rows on
    144 of the 256 blocks, O / down rows on 96, 12 x 16 attention blocks.  A short prompt fed one
    token per step against the FP64 oracle (tokens exact, logits 1e-4); then a 600-token prompt
    through the batched fp32 prefill and 12 persistent steps (16 splits of 38-39 rows) against the
    same steps as separate launches (logits 1e-5, tokens equal) and against the oracle's prompt pass."""
    cfg = Llama2Config(768, 2048, 2, 12, 12, 1000, 1024, True, 64)
    w = make_weights(cfg, seed=5)
    write_checkpoint(tmp_path / "model.bin", cfg, w)
    prompt = [BOS, 17, 230, 5, 99, 301]
    ref = oracle_model(cfg, w)
    ref_fed, ref_logits = ref.generate(prompt, 20)
    rng = np.random.default_rng(6)
    long = [BOS] + [int(t) for t in rng.integers(3, cfg.vocab_size, 599)]
    lref_fed, lref_logits = oracle_model(cfg, w, precision="fp32").generate_prefilled(long, 12)
    with Llama2(tmp_path / "model.bin", None, ctx) as m:
        am = m.model
        assert am.persistent, "the stories110M shape should run the persistent decode kernel"
        fed, logits = gpu_generate(m, prompt, 20)
        assert compare_tokens(fed, ref_fed, ref_logits, len(prompt)) == len(ref_fed)
        assert rel_err(logits, np.asarray(ref_logits)) <= 1e-4
        runs = {}
        for persistent in (True, False):
            am.use_persistent(persistent)
            assert am.persistent == persistent
            am.reset()
            am.set_prompt(long)
            lp = am.prefill(return_logits=True)
            toks, lgs = [], []
            for _ in range(12):
                t, lg = am.next(return_logits=True)
                toks.append(int(t[0]))
                lgs.append(lg[0])
            runs[persistent] = (lp[0], toks, np.stack(lgs))
        am.use_persistent(True)
    (lp_p, toks_p, lgs_p), (lp_m, toks_m, lgs_m) = runs[True], runs[False]
    assert toks_p == toks_m, (toks_p, toks_m)
    assert rel_err(lgs_p, lgs_m) <= 1e-5, rel_err(lgs_p, lgs_m)
    assert rel_err(lp_p, lref_logits[0]) <= 1e-4
    n_eq = len(toks_p)
    for s in range(len(toks_p)):  # token s was chosen from lref_logits[s] (the prompt's last row for s = 0)
        if toks_p[s] != lref_fed[s]:
            top2 = np.sort(lref_logits[s])[-2:]
            assert (top2[1] - top2[0]) / max(abs(top2[1]), 1e-30) < NEAR_TIE, (s, toks_p[s], lref_fed[s])
            n_eq = s
            break
    for s in range(n_eq):
        assert rel_err(lgs_p[s], lref_logits[s + 1]) <= 1e-4, (s, rel_err(lgs_p[s], lref_logits[s + 1]))
    print(f"[llama2] stories shape: persistent == separate launches over 12 steps at 600-611 rows, "
          f"{n_eq} of 12 decisions equal to the oracle", flush=True)
