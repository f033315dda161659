"""Pins the CPU oracle (test infrastructure) before it is trusted as the GPU checker.

Each check is a known answer from the reference's own tests, a closed form, an invariant or a
brute-force restatement in a different formulation, chosen so that a plausible mistake (a
swapped half, a wrong head index, a dropped term, a transposed operand) fails one of them.
"""
import dataclasses
import math

import numpy as np
import pytest

import oracle
from common_amd import config as C
from common_amd import synthetic

PRECS = ["fp64", "fp32"]


# ---- SplitHalfRopeReshapeTest (engine/ml/src/test/.../SplitHalfRopeReshapeTest.java:48-124) ----
@pytest.mark.parametrize("prec", PRECS)
def test_split_half_kat(prec):
    H, HD, FD = 3, 4, 2
    out = oracle.split_half(np.arange(H * HD), H, HD, prec)
    for h in range(H):
        for f in range(FD):
            assert out[h * FD * 2 + f * 2] == h * HD + f
            assert out[h * FD * 2 + f * 2 + 1] == h * HD + FD + f
    back = oracle.unsplit_half(np.arange(H * HD), H, HD, prec)
    for h in range(H):
        for f in range(FD):
            assert back[h * HD + f] == h * FD * 2 + f * 2
            assert back[h * HD + FD + f] == h * FD * 2 + f * 2 + 1
    np.testing.assert_array_equal(oracle.unsplit_half(oracle.split_half(np.arange(12), H, HD, prec), H, HD, prec),
                                  np.arange(12))


# ---- GQAExpandTest (engine/ml/src/test/.../qwen3/GQAExpandTest.java:48-100) ---------------------
def test_gqa_expand_kat():
    heads, kv, hd = 14, 2, 64
    idx = np.arange(kv * hd)
    inp = (idx // hd) * 1000 + idx % hd
    out = oracle.gqa_expand(inp, kv, heads, hd)
    for h in range(heads):
        kvh = h // (heads // kv)
        np.testing.assert_array_equal(out[h * hd:h * hd + hd], kvh * 1000 + np.arange(hd))


# ---- CausalMaskIsolationTest (engine/ml/src/test/.../CausalMaskIsolationTest.java:24-169) ------
def test_causal_mask_kat():
    m0 = oracle.causal_mask(8, 0)
    assert m0[0] == 0 and m0[1] == -10000
    m2 = oracle.causal_mask(8, 2)
    assert list(m2[:3]) == [0, 0, 0] and m2[3] == -10000
    for pos in range(5):
        m = oracle.causal_mask(5, pos)
        for i in range(5):
            assert m[i] == (0.0 if i <= pos else -10000.0)


# ---- RopePositionTest (engine/ml/src/test/.../qwen3/RopePositionTest.java:45-147) --------------
@pytest.mark.parametrize("prec", PRECS)
def test_rope_freqs_kat(prec):
    heads, hd, seq = 2, 4, 10
    fc = oracle.rope_freqs(10000.0, hd, seq, prec)
    # position 0: (cos 0, sin 0) = (1, 0) for every frequency
    np.testing.assert_array_equal(fc[0], [[1, 0], [1, 0]])
    # position 3: angle = 3 / 10000^(2f/hd)
    tol = 1e-12 if prec == "fp64" else 1e-6
    for f in range(hd // 2):
        ang = 3.0 / 10000.0 ** (2.0 * f / hd)
        assert abs(fc[3, f, 0] - math.cos(ang)) < tol
        assert abs(fc[3, f, 1] - math.sin(ang)) < tol
    # the rotation layer on input (1, 0) pairs reproduces (cos, sin), and pos 0 is the identity
    x = np.tile([1.0, 0.0], heads * hd // 2)
    r0 = oracle.rope_rotate_split(x, heads, hd, fc[0].reshape(-1), prec)
    np.testing.assert_array_equal(r0, x)
    r3 = oracle.rope_rotate_split(x, heads, hd, fc[3].reshape(-1), prec)
    np.testing.assert_allclose(r3.reshape(heads, hd // 2, 2), np.broadcast_to(fc[3], (heads, hd // 2, 2)), atol=tol)


@pytest.mark.parametrize("prec", PRECS)
def test_rope_flat_properties(prec):
    """Split-half RoPE: norm of every (f, f+hd/2) pair is preserved; rotating by p then by -p
    (via the conjugate) returns the input; it matches a complex-number formulation."""
    heads, hd, pos, theta = 4, 64, 37, 1e6
    r = np.random.default_rng(0)
    x = r.standard_normal(heads * hd)
    y = oracle.rope_flat(x, heads, hd, pos, theta, prec).astype(np.float64)
    xz = x.reshape(heads, 2, hd // 2)
    z = xz[:, 0] + 1j * xz[:, 1]
    f = np.arange(hd // 2)
    rot = z * np.exp(1j * pos * theta ** (-2.0 * f / hd))
    ref = np.stack([rot.real, rot.imag], axis=1).reshape(-1)
    tol = 1e-12 if prec == "fp64" else 2e-6
    np.testing.assert_allclose(y, ref, atol=tol * 10)
    yz = y.reshape(heads, 2, hd // 2)
    np.testing.assert_allclose(np.hypot(yz[:, 0], yz[:, 1]), np.abs(z), rtol=tol * 10)


# ---- indexOfMax (compute/algebra/.../AggregationFeatures.java:111-121; CollectionComputationTests
#      .indexOfMax2d: [[5,3],[7,10]] -> [0,1]) ----------------------------------------------------
def test_index_of_max_kat():
    np.testing.assert_array_equal(oracle.index_of_max(np.array([[5, 3], [7, 10]], float)), [0, 1])
    np.testing.assert_array_equal(oracle.index_of_max(np.array([[1, 9, 9, 2]], float)), [1])  # first max wins
    np.testing.assert_array_equal(oracle.index_of_max(np.ones((1, 7))), [0])


# ---- rmsnorm closed form + invariants (NormalizationLayerFeatures.java:584-595) -------------------
@pytest.mark.parametrize("prec", PRECS)
def test_rmsnorm_properties(prec):
    x = np.array([3.0, 4.0, 0.0, 0.0])
    # unit gains: y = x / sqrt(mean(x^2) + eps) -> rms(y) ~= 1; here mean(x^2) = 6.25
    y = oracle.rmsnorm(x, np.ones(4), 0.0, prec)
    np.testing.assert_allclose(y, x / 2.5, rtol=1e-7)
    w = np.array([2.0, -1.0, 5.0, 0.5])
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 0.0, prec), w * x / 2.5, rtol=1e-7)
    # scale invariance (eps = 0) and eps entering under the root
    r = np.random.default_rng(1).standard_normal(256)
    np.testing.assert_allclose(oracle.rmsnorm(7 * r, np.ones(256), 0.0, prec), oracle.rmsnorm(r, np.ones(256), 0.0, prec),
                               rtol=1e-6)
    z = oracle.rmsnorm(np.full(4, 1e-3), np.ones(4), 1e-6, prec)
    np.testing.assert_allclose(z, 1e-3 / math.sqrt(1e-6 + 1e-6), rtol=1e-6)
    # grouped (per-head) form equals the whole-vector form applied per group
    g = oracle.rmsnorm(np.concatenate([r, 3 * r]), np.ones(512), 1e-6, prec, group=256)
    np.testing.assert_allclose(g[:256], oracle.rmsnorm(r, np.ones(256), 1e-6, prec), rtol=1e-12 if prec == "fp64" else 1e-6)


# ---- softmax closed form (ActivationFeatures.java:135-143) --------------------------------------
def test_softmax_properties():
    s = oracle.softmax(np.array([[0.0, math.log(3.0)]]))
    np.testing.assert_allclose(s, [[0.25, 0.75]], rtol=1e-14)
    r = np.random.default_rng(2).standard_normal((3, 50)) * 10
    s = oracle.softmax(r)
    np.testing.assert_allclose(s.sum(axis=1), 1.0, rtol=1e-13)
    np.testing.assert_allclose(oracle.softmax(r + 1234.5), s, rtol=1e-9)  # shift invariance
    # masked entries (-10000) get exactly zero weight
    m = oracle.softmax(np.array([[1.0, 2.0, -10000.0 + 3.0]]))
    assert m[0, 2] == 0.0


# ---- dense against a textbook product --------------------------------------------------------------
@pytest.mark.parametrize("prec", PRECS)
def test_dense_matches_matmul(prec):
    r = np.random.default_rng(3)
    W = r.standard_normal((37, 50))
    x = r.standard_normal(50)
    b = r.standard_normal(37)
    tol = 1e-12 if prec == "fp64" else 1e-5
    np.testing.assert_allclose(oracle.dense(W, x, b, prec), W @ x + b, rtol=tol, atol=tol)
    # a transposed operand would fail this non-square case
    e = np.zeros(50)
    e[7] = 1.0
    np.testing.assert_allclose(oracle.dense(W, e, None, prec), W[:, 7], rtol=tol)


# ---- attention: AttentionTests.attentionKeys/attentionValues brute force
#      (engine/ml/src/test/.../AttentionTests.java:51-153) and independent formulations ----------
def test_attention_brute_force_expanded_cache():
    """Scores q.K[t]/sqrt(hd) over t <= pos and values sum_t a[t] V[t], written against a
    GQA-expanded (seq, heads, hd) cache as the reference stores it, with explicit loops."""
    r = np.random.default_rng(4)
    heads, kv, hd, seq, pos = 6, 2, 16, 20, 13
    q = r.standard_normal(heads * hd)
    kc = r.standard_normal((seq, kv, hd))
    vc = r.standard_normal((seq, kv, hd))
    got = oracle.attention(q, kc, vc, heads, kv, hd, pos, seq)
    got_full = oracle.attention(q, kc, vc, heads, kv, hd, pos, seq, full_seq=True)
    np.testing.assert_array_equal(got, got_full)
    kexp = np.repeat(kc, heads // kv, axis=1)  # (seq, heads, hd), as gqaExpand writes it
    vexp = np.repeat(vc, heads // kv, axis=1)
    ref = np.zeros(heads * hd)
    for h in range(heads):
        s = np.array([sum(q[h * hd + i] * kexp[t, h, i] for i in range(hd)) / math.sqrt(hd) for t in range(pos + 1)])
        a = np.exp(s - s.max())
        a /= a.sum()
        for i in range(hd):
            ref[h * hd + i] = sum(a[t] * vexp[t, h, i] for t in range(pos + 1))
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-13)


def test_attention_block_cache_write_and_norm_modes():
    r = np.random.default_rng(5)
    heads, kv, hd, seq, pos, theta = 4, 2, 8, 6, 3, 1e6
    q, k, v = r.standard_normal(heads * hd), r.standard_normal(kv * hd), r.standard_normal(kv * hd)
    qn, kn = 1 + 0.1 * r.standard_normal(heads * hd), 1 + 0.1 * r.standard_normal(kv * hd)
    kc = np.zeros((seq, kv, hd))
    vc = np.zeros((seq, kv, hd))
    out = oracle.attention_block(q, k, v, qn, kn, kc, vc, heads, kv, hd, pos, theta)
    # cache row pos holds rope(rmsnorm(k)) and raw v; other rows untouched
    knorm = oracle.rmsnorm(k, kn, 1e-6)
    np.testing.assert_allclose(kc[pos].reshape(-1), oracle.rope_flat(knorm, kv, hd, pos, theta), rtol=1e-14)
    np.testing.assert_array_equal(vc[pos].reshape(-1), v)
    assert not kc[:pos].any() and not kc[pos + 1:].any()
    # whole-vector QK-norm (reference) differs from the per-head form unless per-head RMS agree
    kc2, vc2 = np.zeros_like(kc), np.zeros_like(vc)
    out_ph = oracle.attention_block(q, k, v, qn, kn, kc2, vc2, heads, kv, hd, pos, theta, per_head_norm=True)
    assert not np.allclose(out, out_ph)
    same = np.tile(r.standard_normal(hd), heads)  # every head has the same RMS -> the forms coincide
    kc3, vc3, kc4, vc4 = (np.zeros_like(kc) for _ in range(4))
    ksame = np.tile(r.standard_normal(hd), kv)
    o1 = oracle.attention_block(same, ksame, v, qn, kn, kc3, vc3, heads, kv, hd, pos, theta)
    o2 = oracle.attention_block(same, ksame, v, qn, kn, kc4, vc4, heads, kv, hd, pos, theta, per_head_norm=True)
    np.testing.assert_allclose(o1, o2, rtol=1e-12)


# ---- whole model: independent float64 restatement on C1 ------------------------------------------
def _numpy_qwen3_reference_graph(cfg, sd, prompt, n_decode):
    """Written against the reference graph's shapes: expanded (seqLen, heads, hd) caches, a
    freqCis table indexed by position, the -10000 mask over the full seqLen, log-sum-exp
    softmax; matrix products via numpy (not sequential sums)."""
    d, H, KV, hd, V = cfg.dim, cfg.head_count, cfg.kv_head_count, cfg.head_size, cfg.vocab_size
    S, L = cfg.seq_len, cfg.layer_count
    f64 = {k: v.astype(np.float64) for k, v in sd.items()}
    fd = hd // 2
    inv = np.exp(np.arange(fd) * (-2.0 * math.log(cfg.rope_theta) / hd))
    ang = np.arange(S)[:, None] * inv[None, :]
    freq = np.stack([np.cos(ang), np.sin(ang)], axis=-1)  # (S, fd, 2)

    def rms(x, w):
        return (w * x) * (1.0 / math.sqrt((x * x).sum() / x.size + cfg.epsilon))

    def rope(x, nh, p):
        xs = x.reshape(nh, 2, fd).transpose(0, 2, 1)  # split-half -> (nh, fd, 2)
        c, s = freq[p, :, 0], freq[p, :, 1]
        o1 = xs[..., 0] * c - xs[..., 1] * s
        o2 = xs[..., 1] * c + xs[..., 0] * s
        return np.stack([o1, o2], axis=1).reshape(-1)  # back to flat halves

    kcache = np.zeros((L, S, H, hd))
    vcache = np.zeros((L, S, H, hd))
    E = f64["model.embed_tokens.weight"]
    fed, logits_all = [], []
    nxt = None
    for p in range(len(prompt) + n_decode):
        tok = int(prompt[p]) if p < len(prompt) else nxt
        fed.append(tok)
        x = E[tok].copy()
        for l in range(L):
            pre = f"model.layers.{l}."
            h = rms(x, f64[pre + "input_layernorm.weight"])
            k = f64[pre + "self_attn.k_proj.weight"] @ h
            v = f64[pre + "self_attn.v_proj.weight"] @ h
            q = f64[pre + "self_attn.q_proj.weight"] @ h
            k = rope(rms(k, f64[pre + "self_attn.k_norm.weight"].reshape(-1)), KV, p)
            q = rope(rms(q, f64[pre + "self_attn.q_norm.weight"].reshape(-1)), H, p)
            kcache[l, p] = np.repeat(k.reshape(KV, hd), H // KV, axis=0)
            vcache[l, p] = np.repeat(v.reshape(KV, hd), H // KV, axis=0)
            sc = np.einsum("hi,thi->ht", q.reshape(H, hd), kcache[l]) / math.sqrt(hd)
            sc = sc + np.where(np.arange(S) > p, -10000.0, 0.0)[None, :]
            z = sc - sc.max(axis=1, keepdims=True)
            a = np.exp(z - np.log(np.exp(z).sum(axis=1, keepdims=True)))
            o = np.einsum("ht,thi->hi", a, vcache[l]).reshape(-1)
            x = x + f64[pre + "self_attn.o_proj.weight"] @ o
            h2 = rms(x, f64[pre + "post_attention_layernorm.weight"])
            g = f64[pre + "mlp.gate_proj.weight"] @ h2
            u = f64[pre + "mlp.up_proj.weight"] @ h2
            x = x + f64[pre + "mlp.down_proj.weight"] @ (u * (g / (1.0 + np.exp(-g))))
        lg = E @ rms(x, f64["model.norm.weight"])
        logits_all.append(lg)
        nxt = int(np.argmax(lg))
    return np.array(fed), np.stack(logits_all)


def test_model_c1_matches_independent_restatement():
    cfg = C.C1_TINY
    sd = synthetic.state_dict(cfg, seed=0)
    prompt = synthetic.prompt_ids(C.C1_PROMPT, cfg.vocab_size, seed=0)
    m = oracle.OracleQwen3(cfg, sd, precision="fp64")
    fed, lg = m.generate(prompt, 12)
    rf, rl = _numpy_qwen3_reference_graph(cfg, sd, prompt, 12)
    np.testing.assert_array_equal(fed, rf)
    np.testing.assert_allclose(lg, rl, rtol=0, atol=1e-11 * np.abs(rl).max())


def test_model_c1_qdim_ne_dim_and_reset():
    """qDim = heads*hd != dim (the Qwen3-0.6B / 4B situation) and reset() replays identically."""
    import dataclasses
    cfg = dataclasses.replace(C.C1_TINY, head_size=128, seq_len=12)
    sd = synthetic.state_dict(cfg, seed=1)
    prompt = synthetic.prompt_ids(5, cfg.vocab_size, seed=1)
    m = oracle.OracleQwen3(cfg, sd)
    f1, l1 = m.generate(prompt, 4)
    m.reset()
    f2, l2 = m.generate(prompt, 4)
    np.testing.assert_array_equal(f1, f2)
    np.testing.assert_array_equal(l1, l2)
    rf, rl = _numpy_qwen3_reference_graph(cfg, sd, prompt, 4)
    np.testing.assert_array_equal(f1, rf)
    np.testing.assert_allclose(l1, rl, rtol=0, atol=1e-11 * np.abs(rl).max())


def test_fp32_oracle_tracks_fp64():
    cfg = C.C1_TINY
    sd = synthetic.state_dict(cfg, seed=0)
    prompt = synthetic.prompt_ids(C.C1_PROMPT, cfg.vocab_size, seed=0)
    f64, l64 = oracle.OracleQwen3(cfg, sd, "fp64").generate(prompt, 8)
    f32, l32 = oracle.OracleQwen3(cfg, sd, "fp32").generate(prompt, 8)
    np.testing.assert_array_equal(f64, f32)
    assert np.abs(l64 - l32).max() / np.abs(l64).max() < 1e-5


def test_oracle_rejects_bad_weights_and_positions():
    cfg = C.C1_TINY
    m = oracle.OracleQwen3(cfg, {})
    with pytest.raises(KeyError):
        oracle.OracleQwen3(cfg, {"model.layers.0.mlp.up_proj.weight": np.zeros(3, np.float32)})
    with pytest.raises(RuntimeError):
        m.step(0)  # no embedding loaded


# ---- batched prompt pass ---------------------------------------------------------------------------
PREFILL_CASES = {
    # C1 (G = 2, hd 64), tied embeddings
    "c1": dataclasses.replace(C.C1_TINY),
    # GQA 4 with q_dim != dim, per-head QK-norm, q/k/v biases, untied head, a ragged dense width
    "gqa4": C.Qwen3Config(dim=200, hidden_dim=328, layer_count=3, head_count=8, kv_head_count=2, vocab_size=301,
                          seq_len=40, head_size=64, qk_norm_mode=C.QK_NORM_PER_HEAD, qkv_bias=True,
                          shared_weights=False),
    # G = 8 heads per KV head (all vector lanes), hd 128
    "gqa8": C.Qwen3Config(dim=256, hidden_dim=512, layer_count=2, head_count=8, kv_head_count=1, vocab_size=97,
                          seq_len=24, head_size=128),
}


@pytest.mark.parametrize("name", sorted(PREFILL_CASES))
@pytest.mark.parametrize("prec", ["fp64", "fp32"])
@pytest.mark.parametrize("full_seq", [False, True])
def test_prefill_equals_stepping_bit_for_bit(name, prec, full_seq):
    """oracle_model_prefill lays the prompt's work out over all rows (packed weight panels, heads in
    vector lanes, the last layer only for the last row) but must compute exactly what one step per
    token computes: tokens, last-row logits and hidden state equal bit for bit, then the decode steps
    after it too.  Prompts of 1, 5 (ragged blocks of 4) and 13 rows; a prefill that starts after 3
    stepped tokens; the full-sequence -10000 mask form."""
    cfg = PREFILL_CASES[name]
    sd = synthetic.state_dict(cfg, seed=5)
    prompt = synthetic.prompt_ids(16, cfg.vocab_size, seed=5)
    for n in (1, 5, 13):
        a = oracle.OracleQwen3(cfg, sd, precision=prec, full_seq_mask=full_seq)
        b = oracle.OracleQwen3(cfg, sd, precision=prec, full_seq_mask=full_seq)
        fed, logits = a.generate(prompt[:n], 4)
        nxt, lg = b.prefill(prompt[:n])
        assert nxt == fed[n] and np.array_equal(lg, logits[n - 1])
        assert np.array_equal(b.hidden(), a_hidden_after(cfg, sd, prec, full_seq, prompt[:n]))
        fed_b, logits_b = [], []
        for _ in range(4):
            fed_b.append(nxt)
            nxt, lgb = b.step(nxt)
            logits_b.append(lgb)
        assert fed_b == list(fed[n:]) and np.array_equal(np.stack(logits_b), logits[n:])
        a.close(); b.close()
    # starting mid-sequence: 3 stepped tokens, then the rest as one prefill
    a = oracle.OracleQwen3(cfg, sd, precision=prec, full_seq_mask=full_seq)
    b = oracle.OracleQwen3(cfg, sd, precision=prec, full_seq_mask=full_seq)
    fed, logits = a.generate(prompt[:11], 0)
    for t in prompt[:3]:
        b.step(int(t))
    nxt, lg = b.prefill(prompt[3:11])
    assert np.array_equal(lg, logits[10])
    assert np.array_equal(b.hidden(), a.hidden())


def a_hidden_after(cfg, sd, prec, full_seq, prompt):
    o = oracle.OracleQwen3(cfg, sd, precision=prec, full_seq_mask=full_seq)
    for t in prompt:
        o.step(int(t), want_logits=False)
    h = o.hidden()
    o.close()
    return h


def test_prefill_rejects_what_stepping_rejects():
    cfg = PREFILL_CASES["c1"]
    sd = synthetic.state_dict(cfg, seed=1)
    o = oracle.OracleQwen3(cfg, sd)
    with pytest.raises(RuntimeError):
        o.prefill(np.arange(cfg.seq_len + 1) % cfg.vocab_size)   # past the cache
    with pytest.raises(RuntimeError):
        o.prefill([0, cfg.vocab_size])                            # token outside the vocabulary
    assert o.prefill([1, 2, 3])[0] >= 0                           # nothing was consumed by the failures
