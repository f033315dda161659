"""GPU parity of the MFMA prefill path, through the C-ABI.

GEMM: against float64 products of the same bf16-rounded operands (fp32 accumulation, 1e-5
relative; the SwiGLU epilogue rounds its output to bf16, 8e-3).  Prefill: a batched prompt must
leave the model where sequential next() calls would (north-star bf16 tolerance 2e-2 on logits,
since prefill feeds bf16 activations to the MFMA units), checked against the GPU decode path and
against the FP64 oracle on the same bf16-rounded weights.  The bf16 prefill tests run on both
product backends (ar_hip_qwen3_prefill_gemm): rocBLAS gemm_ex (the default) and the library's own
fused MFMA kernels.
"""
import dataclasses

import numpy as np
import pytest

import oracle
from common_amd import config as C
from common_amd import hardware as hw
from common_amd import synthetic
from common_amd import qwen3 as q
from common_amd.qwen3 import Qwen3
from conftest import rel_err

pytestmark = pytest.mark.gpu
BF16_TOL = 2e-2
BACKENDS = [pytest.param(q.PREFILL_GEMM_ROCBLAS, id="rocblas"), pytest.param(q.PREFILL_GEMM_OWN, id="own")]


def bf16(a):
    return synthetic.bf16_round(np.asarray(a, np.float32))


def bits(a):
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("M,N,K", [(1, 128, 64), (300, 512, 256), (129, 768, 1024), (2048, 4096, 2048)])
def test_gemm_store_bias(ctx, M, N, K):
    r = np.random.default_rng(M + N + K)
    A = bf16(r.standard_normal((M, K)))
    W = bf16(r.standard_normal((N, K)) * 0.05)
    b = r.standard_normal(N).astype(np.float32)
    Cd = ctx.allocate(M * N * 4)
    ctx.gemm_bf16(ctx.to_device(bits(A)), ctx.to_device(bits(W)), M, N, K, hw.GEMM_STORE, bias=ctx.to_device(b), C=Cd)
    ctx.synchronize()
    got = Cd.download(np.float32, M * N).reshape(M, N)
    ref = A.astype(np.float64) @ W.astype(np.float64).T + b
    assert rel_err(got, ref) <= 1e-5


def test_gemm_residual_and_swiglu(ctx):
    M, N, K = 200, 384, 512
    r = np.random.default_rng(9)
    A = bf16(r.standard_normal((M, K)))
    W = bf16(r.standard_normal((N, K)) * 0.05)
    W2 = bf16(r.standard_normal((N, K)) * 0.05)
    C0 = r.standard_normal((M, N)).astype(np.float32)
    Cd = ctx.to_device(C0)
    Ad, Wd, W2d = ctx.to_device(bits(A)), ctx.to_device(bits(W)), ctx.to_device(bits(W2))
    ctx.gemm_bf16(Ad, Wd, M, N, K, hw.GEMM_RESIDUAL, C=Cd)
    Od = ctx.allocate(M * N * 2)
    ctx.gemm_bf16(Ad, Wd, M, N, K, hw.GEMM_SWIGLU, W2=W2d, O=Od)
    ctx.synchronize()
    g = A.astype(np.float64) @ W.astype(np.float64).T
    u = A.astype(np.float64) @ W2.astype(np.float64).T
    assert rel_err(Cd.download(np.float32, M * N).reshape(M, N), C0 + g) <= 1e-5
    o = (Od.download(np.uint16, M * N).astype(np.uint32) << 16).view(np.float32).reshape(M, N)
    assert rel_err(o, u * (g / (1 + np.exp(-g)))) <= 8e-3


@pytest.mark.parametrize("K", [64, 192, 320])
def test_gemm_large_tile_path(ctx, K):
    """Products with >= 1024 256x256 tiles take the direct-to-LDS kernel: ragged M (8200 rows),
    1, 3 and 5 k-tiles (fewer k-tiles than stages included), all three epilogues."""
    M, N = 8200, 8192
    r = np.random.default_rng(K)
    A = bf16(r.standard_normal((M, K)))
    W = bf16(r.standard_normal((N, K)) * 0.05)
    W2 = bf16(r.standard_normal((N // 2, K)) * 0.05)
    b = r.standard_normal(N).astype(np.float32)
    C0 = r.standard_normal((M, N)).astype(np.float32)
    rows = np.concatenate([np.arange(64), r.choice(M, 64, replace=False), np.arange(M - 40, M)])
    Ad, Wd, W2d = ctx.to_device(bits(A)), ctx.to_device(bits(W)), ctx.to_device(bits(W2))
    Cd = ctx.allocate(M * N * 4)
    ctx.gemm_bf16(Ad, Wd, M, N, K, hw.GEMM_STORE, bias=ctx.to_device(b), C=Cd)
    ctx.synchronize()
    got = Cd.download(np.float32, M * N).reshape(M, N)[rows]
    ref = A[rows].astype(np.float64) @ W.astype(np.float64).T + b
    assert rel_err(got, ref) <= 1e-5
    Cd.upload(C0)
    ctx.gemm_bf16(Ad, Wd, M, N, K, hw.GEMM_RESIDUAL, C=Cd)
    ctx.synchronize()
    got = Cd.download(np.float32, M * N).reshape(M, N)[rows]
    assert rel_err(got, C0[rows] + A[rows].astype(np.float64) @ W.astype(np.float64).T) <= 1e-5
    Nh = N // 2
    Od = ctx.allocate(M * Nh * 2)
    ctx.gemm_bf16(Ad, Wd, M, Nh, K, hw.GEMM_SWIGLU, W2=W2d, O=Od)
    ctx.synchronize()
    g = A[rows].astype(np.float64) @ W[:Nh].astype(np.float64).T
    u = A[rows].astype(np.float64) @ W2.astype(np.float64).T
    o = (Od.download(np.uint16, M * Nh).astype(np.uint32) << 16).view(np.float32).reshape(M, Nh)[rows]
    assert rel_err(o, u * (g / (1 + np.exp(-g)))) <= 8e-3


@pytest.mark.parametrize("M,N,K,epi", [(2048, 6144, 2048, "swiglu"), (1100, 16384, 128, "store"),
                                       (1100, 16384, 128, "residual")])
def test_gemm_tile_rounds_with_half_height_remainder(ctx, M, N, K, epi):
    """Tile counts past whole rounds of the CUs: the columns of the last partial round go to
    128-row tiles (C4 gate/up: 384 tiles of 256 x 256 on 256 CUs; 1100 ragged rows: 320 tiles)."""
    r = np.random.default_rng(M + N + K)
    A = bf16(r.standard_normal((M, K)))
    W = bf16(r.standard_normal((N, K)) * 0.05)
    Ad, Wd = ctx.to_device(bits(A)), ctx.to_device(bits(W))
    rows = np.concatenate([np.arange(40), r.choice(M, 40, replace=False), np.arange(M - 40, M)])
    g = A[rows].astype(np.float64) @ W.astype(np.float64).T
    if epi == "swiglu":
        W2 = bf16(r.standard_normal((N, K)) * 0.05)
        Od = ctx.allocate(M * N * 2)
        ctx.gemm_bf16(Ad, Wd, M, N, K, hw.GEMM_SWIGLU, W2=ctx.to_device(bits(W2)), O=Od)
        ctx.synchronize()
        u = A[rows].astype(np.float64) @ W2.astype(np.float64).T
        o = (Od.download(np.uint16, M * N).astype(np.uint32) << 16).view(np.float32).reshape(M, N)[rows]
        assert rel_err(o, u * (g / (1 + np.exp(-g)))) <= 8e-3
        return
    C0 = r.standard_normal((M, N)).astype(np.float32) if epi == "residual" else np.zeros((M, N), np.float32)
    Cd = ctx.to_device(C0)
    ctx.gemm_bf16(Ad, Wd, M, N, K, hw.GEMM_RESIDUAL if epi == "residual" else hw.GEMM_STORE, C=Cd)
    ctx.synchronize()
    got = Cd.download(np.float32, M * N).reshape(M, N)[rows]
    assert rel_err(got, C0[rows] + g) <= 1e-5


def test_gemm_rejects_bad_shapes(ctx):
    z = ctx.allocate(1 << 16)
    with pytest.raises(hw.HardwareException):
        ctx.gemm_bf16(z, z, 4, 100, 64, hw.GEMM_STORE, C=z)   # N not a multiple of 128
    with pytest.raises(hw.HardwareException):
        ctx.gemm_bf16(z, z, 4, 128, 40, hw.GEMM_STORE, C=z)   # K not a multiple of 64


def _bf16_cfg(base, **kw):
    return dataclasses.replace(base, weight_dtype=C.DTYPE_BF16, **kw)


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("per_head,batch", [(False, 1), (True, 2)])
def test_prefill_matches_sequential_decode_and_oracle(ctx, per_head, batch, backend):
    cfg = _bf16_cfg(C.C1_TINY, seq_len=200, max_batch=batch,
                    qk_norm_mode=C.QK_NORM_PER_HEAD if per_head else C.QK_NORM_WHOLE)
    sd = synthetic.state_dict(cfg, seed=5)
    T = 150  # several 128-row query tiles, ragged
    prompts = [synthetic.prompt_ids(T, cfg.vocab_size, seed=20 + b) for b in range(batch)]
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        am.prefill_gemm = backend
        assert am.prefill_gemm == backend
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        lp = am.prefill(return_logits=True)
        assert am.get_current_step() == T
        after_prefill = am.run(6)
        # the same prompt fed one token per step through the decode plan
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        am.run(T - 1)
        _, ls = am.next(return_logits=True)
        after_seq = am.run(6)
    assert rel_err(lp, ls) <= BF16_TOL
    for b, p in enumerate(prompts):
        ref = oracle.OracleQwen3(cfg, sd, precision="fp64")
        rf, rl = ref.generate(p, 6)
        assert rel_err(lp[b], rl[T - 1]) <= BF16_TOL
        # greedy continuations agree unless the oracle's top-2 margin is within the bf16 tolerance
        for s in range(6):
            top = np.sort(rl[T - 1 + s])[-2:]
            if (top[1] - top[0]) / abs(top[1]) < BF16_TOL:
                break
            assert after_prefill[b, s] == rf[T + s] == after_seq[b, s]


@pytest.mark.parametrize("M,N,K", [(1, 64, 32), (16, 512, 256), (33, 64, 96), (40, 128, 768), (100, 768, 1024),
                                   (128, 4096, 1024), (600, 1024, 3072), (520, 128, 160)])
def test_gemm_f32_vs_float64(ctx, M, N, K):
    """fp32 MFMA projection (ar_hip_gemm_f32): 32- and 64-row tiles, ragged M, 1 / 2 / 4 k-groups per
    block with odd and even iteration counts, all three epilogues, against float64 products of the
    same fp32 operands (1e-5 relative)."""
    r = np.random.default_rng(M + N + K)
    A = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.05).astype(np.float32)
    W2 = (r.standard_normal((N, K)) * 0.05).astype(np.float32)
    b = r.standard_normal(N).astype(np.float32)
    C0 = r.standard_normal((M, N)).astype(np.float32)
    Ad, Wd, W2d = ctx.to_device(A), ctx.to_device(W), ctx.to_device(W2)
    g = A.astype(np.float64) @ W.astype(np.float64).T
    u = A.astype(np.float64) @ W2.astype(np.float64).T
    Cd = ctx.allocate(M * N * 4)
    ctx.gemm_f32(Ad, Wd, M, N, K, hw.GEMM_STORE, bias=ctx.to_device(b), C=Cd)
    ctx.synchronize()
    assert rel_err(Cd.download(np.float32, M * N).reshape(M, N), g + b) <= 1e-5
    Rd = ctx.to_device(C0)
    ctx.gemm_f32(Ad, Wd, M, N, K, hw.GEMM_RESIDUAL, C=Rd)
    ctx.gemm_f32(Ad, Wd, M, N, K, hw.GEMM_SWIGLU, W2=W2d, C=Cd)
    ctx.synchronize()
    assert rel_err(Rd.download(np.float32, M * N).reshape(M, N), C0 + g) <= 1e-5
    assert rel_err(Cd.download(np.float32, M * N).reshape(M, N), u * (g / (1 + np.exp(-g)))) <= 1e-5


def test_prefill_fp32_weights_vs_oracle(ctx):
    """fp32 weights: the prompt runs as fp32 MFMA GEMMs + fp32 causal attention (no decode steps);
    logits within the fp32 bar of the FP64 oracle, greedy continuation equal."""
    cfg = dataclasses.replace(C.C1_TINY, max_batch=2)
    sd = synthetic.state_dict(cfg, seed=0)
    prompts = [synthetic.prompt_ids(C.C1_PROMPT, cfg.vocab_size, seed=b) for b in range(2)]
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        lp = am.prefill(return_logits=True)
        toks = am.run(6)
        assert am.prefill_by_steps() == 0
    T = C.C1_PROMPT
    for b, p in enumerate(prompts):
        rf, rl = oracle.OracleQwen3(cfg, sd, precision="fp64").generate(p, 6)
        assert rel_err(lp[b], rl[T - 1]) <= 1e-4, rel_err(lp[b], rl[T - 1])
        np.testing.assert_array_equal(toks[b], rf[T:])


def test_prefill_fp32_c3_prompt_vs_oracle(ctx):
    """BASELINE config 3 (Qwen3-0.6B shape, fp32, q_dim 2048 != dim): the 128-token prompt through
    the fp32 batched prefill, then 8 greedy steps, against the FP32 oracle's batched prompt pass
    (bit-equal to stepping it) -- logits 1e-4, tokens equal except at a genuine near-tie."""
    cfg = C.C3_0_6B
    T, steps = C.C3_PROMPT, 8
    prompt = synthetic.prompt_ids(T, cfg.vocab_size, seed=0)
    sd = synthetic.state_dict(cfg, seed=0)
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        am.reset()
        am.set_prompt(prompt)
        lp = am.prefill(return_logits=True)
        fed, lgs = [], []
        for _ in range(steps):
            t, lg = am.next(return_logits=True)
            fed.append(int(t[0]))
            lgs.append(lg[0])
        assert am.prefill_by_steps() == 0
    ref = oracle.OracleQwen3(cfg, sd, precision="fp32")
    del sd
    rfed, rl = ref.generate_prefilled(prompt, steps)
    ref.close()
    assert rel_err(lp[0], rl[0]) <= 1e-4, rel_err(lp[0], rl[0])
    for s in range(steps):
        if fed[s] != rfed[s]:
            top = np.sort(rl[s])[-2:]
            assert (top[1] - top[0]) / abs(top[1]) < 1e-5, (s, fed[s], rfed[s])
            break
        assert rel_err(lgs[s], rl[s + 1]) <= 1e-4, (s, rel_err(lgs[s], rl[s + 1]))


@pytest.mark.parametrize("backend", BACKENDS)
def test_prefill_c4_shape_matches_sequential_decode(ctx, backend):
    """Qwen3-1.7B shape, bf16 weights, prefill 2048 tokens vs the decode step."""
    cfg = dataclasses.replace(C.C4_1_7B, seq_len=C.C4_PROMPT + 8)
    T = C.C4_PROMPT
    prompt = synthetic.prompt_ids(T, cfg.vocab_size, seed=4)
    with Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=4), ctx) as m:
        am = m.model
        am.prefill_gemm = backend
        am.reset()
        am.set_prompt(prompt)
        lp = am.prefill(return_logits=True)
        after_prefill = am.run(4)
        am.reset()
        am.set_prompt(prompt)
        am.run(T - 1)
        _, ls = am.next(return_logits=True)
        after_seq = am.run(4)
    assert rel_err(lp, ls) <= BF16_TOL
    top = np.sort(ls[0])[-2:]
    if (top[1] - top[0]) / abs(top[1]) > BF16_TOL:
        assert after_prefill[0, 0] == after_seq[0, 0]


def test_prefill_gqa4_batch8_matches_oracle(ctx):
    """The C5 structure at small size: 4 query heads per KV head, q_dim != dim, batch 8, ragged prompt."""
    cfg = _bf16_cfg(C.C1_TINY, head_count=8, kv_head_count=2, head_size=64, seq_len=140, max_batch=8)
    assert cfg.q_dim != cfg.dim
    sd = synthetic.state_dict(cfg, seed=7)
    T, steps = 100, 4
    prompts = [synthetic.prompt_ids(T, cfg.vocab_size, seed=40 + b) for b in range(8)]
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        lp = am.prefill(return_logits=True)
        after_prefill = am.run(steps)
    for b, p in enumerate(prompts):
        rf, rl = oracle.OracleQwen3(cfg, sd, precision="fp64").generate(p, steps)
        assert rel_err(lp[b], rl[T - 1]) <= BF16_TOL, b
        for s in range(steps):
            top = np.sort(rl[T - 1 + s])[-2:]
            if (top[1] - top[0]) / abs(top[1]) < BF16_TOL:
                break
            assert after_prefill[b, s] == rf[T + s], (b, s)


@pytest.mark.parametrize("backend", BACKENDS)
def test_prefill_c5_shape_batch8_matches_sequential_decode(ctx, backend):
    """Qwen3-4B layer shape (d2560, 32Q/8KV, hd128, F9728), batch 8, two layers
    and a 512-token context: batched prefill vs the decode step fed one token at a time."""
    T = 512
    cfg = dataclasses.replace(C.C5_4B, layer_count=2, seq_len=T + 8, max_batch=8)
    prompts = [synthetic.prompt_ids(T, cfg.vocab_size, seed=50 + b) for b in range(8)]
    with Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=5), ctx) as m:
        am = m.model
        am.prefill_gemm = backend
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        lp = am.prefill(return_logits=True)
        after_prefill = am.run(2)
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        am.run(T - 1)
        _, ls = am.next(return_logits=True)
        after_seq = am.run(2)
    for b in range(8):
        assert rel_err(lp[b], ls[b]) <= BF16_TOL, b
        top = np.sort(ls[b])[-2:]
        if (top[1] - top[0]) / abs(top[1]) > BF16_TOL:
            assert after_prefill[b, 0] == after_seq[b, 0], b


@pytest.mark.parametrize("prefill", [True, False])
def test_fp16_kv_cache_matches_oracle(ctx, prefill):
    """kv_dtype = fp16 (half the cache bytes): prompt by prefill or token by token, then greedy decode;
    logits within the bf16 north-star tolerance of the FP64 oracle, continuations checked until
    the oracle's top-2 margin falls inside the tolerance."""
    cfg = _bf16_cfg(C.C1_TINY, head_count=8, kv_head_count=2, head_size=64, seq_len=120, max_batch=2,
                    kv_dtype=C.DTYPE_F16)
    sd = synthetic.state_dict(cfg, seed=9)
    T, steps = 70, 6
    prompts = [synthetic.prompt_ids(T, cfg.vocab_size, seed=60 + b) for b in range(2)]
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        if prefill:
            lp = am.prefill(return_logits=True)
        else:
            am.run(T - 1)
            _, lp = am.next(return_logits=True)
        toks = am.run(steps)
    for b, p in enumerate(prompts):
        rf, rl = oracle.OracleQwen3(cfg, sd, precision="fp64").generate(p, steps)
        assert rel_err(lp[b], rl[T - 1]) <= BF16_TOL, b
        for s in range(steps):
            top = np.sort(rl[T - 1 + s])[-2:]
            if (top[1] - top[0]) / abs(top[1]) < BF16_TOL:
                break
            assert toks[b, s] == rf[T + s], (b, s)


def test_fp16_kv_cache_c5_layer_shape_close_to_fp32_cache(ctx):
    """C5 layer shape (32 Q / 8 KV heads, hd 128), batch 8 decode after a 512-token prefill: the fp16
    cache gives logits within the bf16 tolerance of the fp32 cache."""
    T = 512
    base = dataclasses.replace(C.C5_4B, layer_count=2, seq_len=T + 8, max_batch=8)
    prompts = [synthetic.prompt_ids(T, base.vocab_size, seed=70 + b) for b in range(8)]
    out = {}
    for kv in (C.DTYPE_F32, C.DTYPE_F16):
        cfg = dataclasses.replace(base, kv_dtype=kv)
        with Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=6), ctx) as m:
            am = m.model
            am.reset()
            for b, p in enumerate(prompts):
                am.set_prompt(p, seq=b)
            am.prefill()
            am.run(3)
            _, out[kv] = am.next(return_logits=True)
    for b in range(8):
        assert rel_err(out[C.DTYPE_F16][b], out[C.DTYPE_F32][b]) <= BF16_TOL, b


def _prefill_vs_oracle(ctx, cfg, sd, prompts, steps, backend=q.PREFILL_GEMM_ROCBLAS):
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        am.prefill_gemm = backend
        am.reset()
        for b, p in enumerate(prompts):
            am.set_prompt(p, seq=b)
        lp = am.prefill(return_logits=True)
        toks = am.run(steps)
        by_steps = am.prefill_by_steps()
    T = len(prompts[0])
    for b, p in enumerate(prompts):
        rf, rl = oracle.OracleQwen3(cfg, sd, precision="fp64").generate(p, steps)
        assert rel_err(lp[b], rl[T - 1]) <= BF16_TOL, (b, rel_err(lp[b], rl[T - 1]))
        for s in range(steps):
            top = np.sort(rl[T - 1 + s])[-2:]
            if (top[1] - top[0]) / abs(top[1]) < BF16_TOL:
                break
            assert toks[b, s] == rf[T + s], (b, s)
    return by_steps


@pytest.mark.parametrize("backend", BACKENDS)
@pytest.mark.parametrize("where", ["ffn_norm_gain", "swiglu_output", "gate_value"])
def test_prefill_fp16_overflow_takes_the_decode_step(ctx, where, backend):
    """Activations past the fp16 range (a real checkpoint's outliers): a post-attention RMSNorm gain
    of 2^17 (normalised rows ~1e5) or gate/up weights scaled by 2^11 (SwiGLU outputs ~1e6).  The
    batched pass sees the overflow and the prompt goes through the decode step: logits and tokens
    still match the FP64 oracle."""
    cfg = _bf16_cfg(C.C1_TINY, seq_len=96, max_batch=2)
    sd = synthetic.state_dict(cfg, seed=31)
    if where == "ffn_norm_gain":
        sd["model.layers.0.post_attention_layernorm.weight"] = sd["model.layers.0.post_attention_layernorm.weight"] * 2.0 ** 17
    elif where == "swiglu_output":
        for k in ("mlp.gate_proj.weight", "mlp.up_proj.weight"):
            sd["model.layers.1." + k] = sd["model.layers.1." + k] * 2.0 ** 11
    else:  # gate pre-activations past the fp16 range with small up values: the rocBLAS path's fp16
        # gate/up rows overflow although the SwiGLU outputs would fit
        # (gate rows ~4e4 rms, up rows ~2e-2: outputs up to ~1e4)
        sd["model.layers.1.mlp.gate_proj.weight"] = sd["model.layers.1.mlp.gate_proj.weight"] * 2.0 ** 17
        sd["model.layers.1.mlp.up_proj.weight"] = sd["model.layers.1.mlp.up_proj.weight"] * 2.0 ** -4
    prompts = [synthetic.prompt_ids(40, cfg.vocab_size, seed=32 + b) for b in range(2)]
    by_steps = _prefill_vs_oracle(ctx, cfg, sd, prompts, 4, backend)
    # (the own kernels' fused epilogue keeps gate and up in fp32: only the SwiGLU output is checked)
    assert by_steps == (0 if where == "gate_value" and backend == q.PREFILL_GEMM_OWN else 1)


def test_prefill_tiny_weights_stay_on_the_batched_path(ctx):
    """Weights below 2^-17 lose bits in their fp16 copies (the fp16 grid there is 2^-24, an absolute
    error of at most 2^-25 per weight): a down projection scaled by 2^-12 (|w| ~ 5e-6) stays on the
    batched path and still matches the FP64 oracle within the bf16 tolerance."""
    cfg = _bf16_cfg(C.C1_TINY, seq_len=96, max_batch=1)
    sd = synthetic.state_dict(cfg, seed=33)
    sd["model.layers.1.mlp.down_proj.weight"] = sd["model.layers.1.mlp.down_proj.weight"] * 2.0 ** -12
    w = sd["model.layers.1.mlp.down_proj.weight"]
    assert np.mean(np.abs(w) < 2.0 ** -17) > 0.5
    prompts = [synthetic.prompt_ids(40, cfg.vocab_size, seed=34)]
    assert _prefill_vs_oracle(ctx, cfg, sd, prompts, 4) == 0


def test_prefill_backends_agree_and_reject_unknown(ctx):
    """The two product backends on one prompt (C1 shape, bf16, batch 2): logits within float
    rounding of each other (same fp16 operands, fp32 accumulation in both; the rocBLAS path rounds
    gate and up to fp16 before the SwiGLU), and an unknown backend is refused."""
    cfg = _bf16_cfg(C.C1_TINY, seq_len=160, max_batch=2)
    sd = synthetic.state_dict(cfg, seed=41)
    prompts = [synthetic.prompt_ids(130, cfg.vocab_size, seed=42 + b) for b in range(2)]
    out = {}
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        with pytest.raises(hw.HardwareException) as e:
            am.prefill_gemm = 7
        assert e.value.code == hw.AR_HIP_ERR_INVALID
        assert am.prefill_gemm == q.PREFILL_GEMM_ROCBLAS  # the default, unchanged by the refused call
        for backend in (q.PREFILL_GEMM_OWN, q.PREFILL_GEMM_ROCBLAS):
            am.prefill_gemm = backend
            am.reset()
            for b, p in enumerate(prompts):
                am.set_prompt(p, seq=b)
            out[backend] = am.prefill(return_logits=True)
            assert am.prefill_by_steps() == 0
    assert rel_err(out[q.PREFILL_GEMM_ROCBLAS], out[q.PREFILL_GEMM_OWN]) <= 5e-3
