"""GPU parity of the stand-alone operators against the CPU oracle, through the C-ABI.

Tolerances (fp32 arithmetic on the GPU, oracle in fp64 with sequential sums):
  GEMV / SwiGLU / RMSNorm / attention: max|gpu-ref| / max|ref| <= 1e-5
  RoPE: <= 1e-6 (angles in double on both sides)
  indexOfMax: exact (first maximum wins)
"""
import numpy as np
import pytest

import oracle
from common_amd import hardware as hw
from common_amd.synthetic import bf16_round
from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("rows,cols,batch,norm,bias,bf16", [
    (64, 256, 1, False, False, False),
    (1000, 1024, 1, True, False, False),
    (4096, 1024, 1, True, True, False),
    (1024, 2048, 1, False, False, False),
    (1024, 3072, 1, False, False, True),
    (300, 2048, 3, True, False, False),
    (1001, 1024, 5, True, True, False),
    (2560, 9728, 8, False, False, True),
    (17, 9728, 8, False, True, True),
    (8200, 2560, 8, True, False, True),
    (20000, 1024, 1, True, False, False),
    (20000, 1024, 6, True, False, True),
])
def test_dense(ctx, rows, cols, batch, norm, bias, bf16):
    r = _rng(rows * 7 + cols)
    W = (r.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if bf16:
        W = bf16_round(W)
    x = r.standard_normal((batch, cols)).astype(np.float32)
    g = (1 + 0.02 * r.standard_normal(cols)).astype(np.float32)
    b = r.standard_normal(rows).astype(np.float32) if bias else None
    if bf16:
        Wd = ctx.to_device((W.view(np.uint32) >> 16).astype(np.uint16))
    else:
        Wd = ctx.to_device(W)
    xd, yd = ctx.to_device(x), ctx.allocate(batch * rows * 4)
    gd = ctx.to_device(g) if norm else None
    bd = ctx.to_device(b) if bias else None
    ctx.dense(Wd, hw.DTYPE_BF16 if bf16 else hw.DTYPE_F32, xd, yd, rows, cols, batch, bias=bd, norm_w=gd, eps=1e-6)
    ctx.synchronize()
    y = yd.download(np.float32, batch * rows).reshape(batch, rows)
    for i in range(batch):
        h = oracle.rmsnorm(x[i], g, 1e-6) if norm else x[i]
        ref = oracle.dense(W, h, bias=b)
        assert rel_err(y[i], ref) <= TOL, (i, rel_err(y[i], ref))


@pytest.mark.parametrize("rows,cols,batch,bf16", [(768, 256, 1, False), (3072, 1024, 1, False),
                                                  (6144, 2048, 2, True), (9728, 2560, 8, True),
                                                  (3000, 1024, 4, False)])
def test_swiglu(ctx, rows, cols, batch, bf16):
    r = _rng(rows + cols)
    Wg = (r.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    Wu = (r.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if bf16:
        Wg, Wu = bf16_round(Wg), bf16_round(Wu)
    x = r.standard_normal((batch, cols)).astype(np.float32)
    g = (1 + 0.02 * r.standard_normal(cols)).astype(np.float32)
    enc = (lambda a: (a.view(np.uint32) >> 16).astype(np.uint16)) if bf16 else (lambda a: a)
    yd = ctx.allocate(batch * rows * 4)
    ctx.swiglu(ctx.to_device(enc(Wg)), ctx.to_device(enc(Wu)), hw.DTYPE_BF16 if bf16 else hw.DTYPE_F32,
               ctx.to_device(x), yd, rows, cols, batch, norm_w=ctx.to_device(g))
    ctx.synchronize()
    y = yd.download(np.float32, batch * rows).reshape(batch, rows)
    for i in range(batch):
        h = oracle.rmsnorm(x[i], g, 1e-6)
        gate, up = oracle.dense(Wg, h), oracle.dense(Wu, h)
        ref = up * (gate * (1.0 / (np.exp(-gate) + 1.0)))
        assert rel_err(y[i], ref) <= TOL


@pytest.mark.parametrize("rows,n", [(1, 256), (3, 1024), (2, 2560), (1, 4096)])
def test_rmsnorm(ctx, rows, n):
    r = _rng(n)
    x = r.standard_normal((rows, n)).astype(np.float32)
    w = (1 + 0.02 * r.standard_normal(n)).astype(np.float32)
    yd = ctx.allocate(rows * n * 4)
    ctx.rmsnorm(ctx.to_device(x), ctx.to_device(w), yd, rows, n, 1e-6)
    ctx.synchronize()
    y = yd.download(np.float32, rows * n).reshape(rows, n)
    assert rel_err(y, oracle.rmsnorm(x, w, 1e-6)) <= TOL


@pytest.mark.parametrize("heads,hd,pos", [(4, 64, 0), (16, 128, 3), (8, 128, 4096), (32, 128, 8255), (3, 4, 7)])
def test_rope(ctx, heads, hd, pos):
    r = _rng(heads * hd + pos)
    x = r.standard_normal((2, heads * hd)).astype(np.float32)
    xd = ctx.to_device(x)
    ctx.rope(xd, heads, hd, pos, 1e6, rows=2)
    ctx.synchronize()
    y = xd.download(np.float32, x.size).reshape(x.shape)
    ref = oracle.rope_flat(x, heads, hd, pos, 1e6)
    assert rel_err(y, ref) <= 1e-6
    if pos == 0:
        np.testing.assert_array_equal(y, x)


def test_index_of_max(ctx):
    r = _rng(5)
    x = r.standard_normal((4, 151936)).astype(np.float32)
    x[1, 77] = x[1, 900] = 50.0          # tie: the first index wins
    x[2, :] = 1.0                       # all equal: index 0
    x[3, -1] = 99.0                     # last element
    od = ctx.allocate(16)
    ctx.index_of_max(ctx.to_device(x), 4, x.shape[1], od)
    ctx.synchronize()
    got = od.download(np.int32, 4)
    np.testing.assert_array_equal(got, oracle.index_of_max(x))
    np.testing.assert_array_equal(got[1:], [77, 0, 151935])
    # the reference's own known answer: [[5,3],[7,10]] -> [0, 1] (CollectionComputationTests.indexOfMax2d)
    kd = ctx.to_device(np.array([[5, 3], [7, 10]], np.float32))
    ctx.index_of_max(kd, 2, 2, od)
    ctx.synchronize()
    np.testing.assert_array_equal(od.download(np.int32, 2), [0, 1])


def _attention_case(ctx, heads, kv_heads, hd, max_seq, pos, per_head, seed, filled=None):
    r = _rng(seed)
    qd, kd = heads * hd, kv_heads * hd
    q = r.standard_normal(qd).astype(np.float32)
    k = r.standard_normal(kd).astype(np.float32)
    v = r.standard_normal(kd).astype(np.float32)
    qn = (1 + 0.02 * r.standard_normal(qd)).astype(np.float32)
    kn = (1 + 0.02 * r.standard_normal(kd)).astype(np.float32)
    filled = pos if filled is None else filled
    # reference-layout caches (seq, kv_heads, hd); device layout (kv_heads, seq, hd)
    kc = np.zeros((max_seq, kv_heads, hd), np.float32)
    vc = np.zeros((max_seq, kv_heads, hd), np.float32)
    kc[:filled] = r.standard_normal((filled, kv_heads, hd))
    vc[:filled] = r.standard_normal((filled, kv_heads, hd))
    kcd = ctx.to_device(np.ascontiguousarray(kc.transpose(1, 0, 2)))
    vcd = ctx.to_device(np.ascontiguousarray(vc.transpose(1, 0, 2)))
    od = ctx.allocate(qd * 4)
    ctx.attention_decode(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), ctx.to_device(qn), ctx.to_device(kn),
                         1e-6, 1 if per_head else 0, kcd, vcd, max_seq, pos, heads, kv_heads, hd, 1e6, od)
    ctx.synchronize()
    out = od.download(np.float32, qd)
    kc64, vc64 = kc.astype(np.float64), vc.astype(np.float64)
    ref = oracle.attention_block(q, k, v, qn, kn, kc64, vc64, heads, kv_heads, hd, pos, 1e6, 1e-6,
                                 per_head_norm=per_head)
    kgot = kcd.download(np.float32, kv_heads * max_seq * hd).reshape(kv_heads, max_seq, hd)
    vgot = vcd.download(np.float32, kv_heads * max_seq * hd).reshape(kv_heads, max_seq, hd)
    return out, ref, kgot[:, pos], kc64[pos], vgot[:, pos], vc64[pos]


@pytest.mark.parametrize("per_head", [False, True])
def test_attention_c2(ctx, per_head):
    """16 Q / 8 KV heads, hd 128, cache filled 0..4095, decode at position 4096."""
    out, ref, kg, kr, vg, vr = _attention_case(ctx, 16, 8, 128, 4097, 4096, per_head, seed=2)
    assert rel_err(out, ref) <= TOL
    assert rel_err(kg, kr) <= 1e-6
    np.testing.assert_array_equal(vg, vr.astype(np.float32))


@pytest.mark.parametrize("heads,kv,hd,max_seq,pos", [
    (4, 2, 64, 48, 0), (4, 2, 64, 48, 1), (4, 2, 64, 48, 47), (16, 8, 128, 384, 200), (32, 8, 128, 8256, 8192),
    (8, 8, 128, 100, 63), (16, 2, 128, 700, 699), (8, 8, 128, 1000, 999), (4, 2, 64, 600, 599),
    (8, 1, 128, 4096, 4000)])
def test_attention_edges(ctx, heads, kv, hd, max_seq, pos):
    """One-block form (caches <= 256 rows) and split form with G = 1, 2, 4, 8 query heads per KV
    head, head_dim 64 and 128, up to 256 splits."""
    out, ref, kg, kr, vg, vr = _attention_case(ctx, heads, kv, hd, max_seq, pos, False, seed=pos + heads)
    assert rel_err(out, ref) <= TOL
    assert rel_err(kg, kr) <= 1e-6


def test_attention_consecutive_calls(ctx):
    """Consecutive calls with different split counts (positions 300, 3000, 17, 3000) reuse the op's
    split buffers and all match the oracle."""
    for i, pos in enumerate([300, 3000, 17, 3000]):
        out, ref, *_ = _attention_case(ctx, 16, 8, 128, 4097, pos, False, seed=40 + i)
        assert rel_err(out, ref) <= TOL, pos


def test_attention_rejects_out_of_range_position(ctx):
    z = ctx.allocate(4096)
    with pytest.raises(hw.HardwareException) as e:
        ctx.attention_decode(z, z, z, None, None, 1e-6, 0, z, z, 4, 4, 1, 1, 64, 1e6, z)
    assert e.value.code == hw.AR_HIP_ERR_INVALID


@pytest.mark.parametrize("heads,kv,hd,max_seq,pos", [(4, 2, 64, 48, 20), (16, 8, 128, 384, 200), (16, 8, 128, 4097, 3000)])
def test_attention_ignores_stale_nan_rows(ctx, heads, kv, hd, max_seq, pos):
    """Rows at and past the position hold NaN (a previous sequence that overflowed): row pos is
    overwritten by this step and the rest are masked, so the output is finite and matches the oracle
    (one-block form and split form)."""
    r = _rng(pos)
    qd, kd = heads * hd, kv * hd
    q, k, v = (r.standard_normal(n).astype(np.float32) for n in (qd, kd, kd))
    kc = np.full((max_seq, kv, hd), np.nan, np.float32)
    vc = np.full((max_seq, kv, hd), np.nan, np.float32)
    kc[:pos] = r.standard_normal((pos, kv, hd))
    vc[:pos] = r.standard_normal((pos, kv, hd))
    kcd = ctx.to_device(np.ascontiguousarray(kc.transpose(1, 0, 2)))
    vcd = ctx.to_device(np.ascontiguousarray(vc.transpose(1, 0, 2)))
    od = ctx.allocate(qd * 4)
    ctx.attention_decode(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), None, None, 1e-6, 0, kcd, vcd, max_seq,
                         pos, heads, kv, hd, 1e6, od)
    ctx.synchronize()
    out = od.download(np.float32, qd)
    kc64, vc64 = kc.astype(np.float64), vc.astype(np.float64)
    ref = oracle.attention_block(q, k, v, None, None, kc64, vc64, heads, kv, hd, pos, 1e6, 1e-6)
    assert np.isfinite(out).all()
    assert rel_err(out, ref) <= TOL


def test_device_selected_by_environment(monkeypatch):
    """ar_hip_init(-1): the device AR_HIP_DEVICE names (default 0); a device that does not exist is
    an argument error."""
    monkeypatch.setenv("AR_HIP_DEVICE", "0")
    with hw.HipContext() as c:
        assert c.info()["num_cus"] > 0
    monkeypatch.setenv("AR_HIP_DEVICE", "99")
    with pytest.raises(hw.HardwareException) as e:
        hw.HipContext()
    assert e.value.code == hw.AR_HIP_ERR_INVALID
