"""GPU check of the allocation-free attention entry point (ar_hip_attention_decode_noalloc),
through the C-ABI: on the same inputs it must give exactly what ar_hip_attention_decode gives
(same kernels, partials in the library's fixed per-device scratch array instead of allocated
memory), on two calls in a row whose second is smaller, and match the oracle to the attention
tolerance.  Shapes whose partials exceed the scratch array are rejected."""
import numpy as np
import pytest

import oracle
from common_amd import hardware as hw
from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _inputs(heads, kv_heads, hd, max_seq, pos, seed):
    r = np.random.default_rng(seed)
    qd, kd = heads * hd, kv_heads * hd
    q, k, v = (r.standard_normal(n).astype(np.float32) for n in (qd, kd, kd))
    qn = (1 + 0.02 * r.standard_normal(qd)).astype(np.float32)
    kn = (1 + 0.02 * r.standard_normal(kd)).astype(np.float32)
    kc = np.zeros((max_seq, kv_heads, hd), np.float32)
    vc = np.zeros((max_seq, kv_heads, hd), np.float32)
    kc[:pos] = r.standard_normal((pos, kv_heads, hd))
    vc[:pos] = r.standard_normal((pos, kv_heads, hd))
    return q, k, v, qn, kn, kc, vc


def _run(ctx, noalloc, heads, kv_heads, hd, max_seq, pos, inputs):
    q, k, v, qn, kn, kc, vc = inputs
    kcd = ctx.to_device(np.ascontiguousarray(kc.transpose(1, 0, 2)))
    vcd = ctx.to_device(np.ascontiguousarray(vc.transpose(1, 0, 2)))
    od = ctx.allocate(heads * hd * 4)
    ctx.attention_decode(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), ctx.to_device(qn), ctx.to_device(kn),
                         1e-6, 0, kcd, vcd, max_seq, pos, heads, kv_heads, hd, 1e6, od, noalloc=noalloc)
    ctx.synchronize()
    out = od.download(np.float32, heads * hd)
    krow = kcd.download(np.float32, kv_heads * max_seq * hd).reshape(kv_heads, max_seq, hd)[:, pos]
    return out, krow


def test_noalloc_attention_equals_allocating_entry_point(ctx):
    # C2 (16 Q / 8 KV heads, hd 128, 4097-row cache: 32 splits), then a smaller call (8 / 2 heads,
    # 600 rows) that uses fewer scratch slots, then the C2 call again
    for i, (heads, kv, hd, max_seq, pos) in enumerate([(16, 8, 128, 4097, 4096), (8, 2, 128, 600, 599),
                                                        (16, 8, 128, 4097, 4096)]):
        print(f"no-alloc attention call {i}: heads {heads}/{kv} hd {hd} cache {max_seq} pos {pos}", flush=True)
        inputs = _inputs(heads, kv, hd, max_seq, pos, seed=70 + i)
        got, krow = _run(ctx, True, heads, kv, hd, max_seq, pos, inputs)
        want, krow_want = _run(ctx, False, heads, kv, hd, max_seq, pos, inputs)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(krow, krow_want)
        q, k, v, qn, kn, kc, vc = inputs
        ref = oracle.attention_block(q, k, v, qn, kn, kc.astype(np.float64), vc.astype(np.float64), heads, kv, hd,
                                     pos, 1e6, 1e-6, per_head_norm=False)
        assert rel_err(got, ref) <= TOL


def test_noalloc_attention_rejects_partials_beyond_the_scratch(ctx):
    # 64 heads / 64 KV heads x hd 128 over 65,536 rows: 256 splits x 64 heads x 130 floats > 2^18
    # (rejected before any launch: no buffer is touched)
    z = ctx.allocate(1 << 16)
    with pytest.raises(hw.HardwareException, match="scratch") as e:
        ctx.attention_decode(z, z, z, None, None, 1e-6, 0, z, z, 65536, 10, 64, 64, 128, 1e6, z, noalloc=True)
    assert e.value.code == hw.AR_HIP_ERR_INVALID
