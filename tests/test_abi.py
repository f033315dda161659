"""CPU checks of the C-ABI library: it loads, exports every symbol include/ar_hip.h declares,
and reports errors through the documented channel.  No compute call needs a GPU here."""
import ctypes
import os
import subprocess

import pytest

from common_amd import _native
from common_amd import hardware as hw
from common_amd import synthetic


def test_library_exports_every_declared_symbol():
    names = hw.declared_symbols()
    assert len(names) >= 30
    L = hw.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", _native.HIP_LIB], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(names) <= exported


def test_library_is_gfx950_only(tmp_path):
    fb = tmp_path / "fatbin.bin"
    ex = subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", _native.HIP_LIB, str(fb)],
                        capture_output=True, text=True)
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o", f"--input={fb}"],
                         capture_output=True, text=True)
    if ex.returncode != 0 or out.returncode != 0:
        pytest.skip("offload bundle listing unavailable")
    targets = [t for t in out.stdout.split() if "amdgcn" in t]
    assert targets and all("gfx950" in t for t in targets), targets


def test_version_and_empty_error():
    assert b"gfx950" in hw.lib().ar_hip_version()
    assert isinstance(hw.lib().ar_hip_last_error(), bytes)


def test_init_without_gpu_reports_no_device():
    if hw.device_count() > 0:
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    rc = hw.lib().ar_hip_init(0, ctypes.byref(h))
    assert rc == hw.AR_HIP_ERR_NO_DEVICE
    assert h.value is None
    assert b"device" in hw.lib().ar_hip_last_error()
    with pytest.raises(hw.HardwareException) as e:
        hw.HipContext(0)
    assert e.value.code == hw.AR_HIP_ERR_NO_DEVICE


def test_null_arguments_are_rejected_without_a_device():
    L = hw.lib()
    assert L.ar_hip_device_count(None) == hw.AR_HIP_ERR_INVALID
    assert L.ar_hip_synchronize(None) == hw.AR_HIP_ERR_INVALID
    assert L.ar_hip_alloc(None, 16, None) == hw.AR_HIP_ERR_INVALID
    assert L.ar_hip_qwen3_create(None, None, None) == hw.AR_HIP_ERR_INVALID
    assert L.ar_hip_qwen3_next(None, None, None) == hw.AR_HIP_ERR_INVALID
    assert b"null" in L.ar_hip_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_cache", {})
    with pytest.raises(_native.NativeLibraryMissing):
        _native._load(str(tmp_path / "libar_hip.so"), "HIP backend library")


def test_synthetic_inputs_are_deterministic_and_shaped():
    a = synthetic.normal_tensor("model.layers.0.mlp.up_proj.weight", (64, 32), seed=7)
    b = synthetic.normal_tensor("model.layers.0.mlp.up_proj.weight", (64, 32), seed=7)
    c = synthetic.normal_tensor("model.layers.0.mlp.up_proj.weight", (64, 32), seed=8)
    assert (a == b).all() and not (a == c).all()
    big = synthetic.normal_tensor("x", (1 << 20,), seed=0)
    assert abs(big.std() - 0.02) < 2e-4 and abs(big.mean()) < 1e-4
    g = synthetic.normal_tensor("g", (1 << 16,), seed=0, mean=1.0)
    assert abs(g.mean() - 1.0) < 1e-3
    bf = synthetic.normal_tensor("x", (1000,), seed=0, bf16=True)
    assert ((bf.view("uint32") & 0xFFFF) == 0).all()
    ids = synthetic.prompt_ids(4096, 151936, seed=0)
    assert ids.min() >= 0 and ids.max() < 151936 and len(set(ids.tolist())) > 4000
    assert (synthetic.prompt_ids(16, 1024, seed=0, batch=2)[0] == synthetic.prompt_ids(16, 1024, seed=0)).all()


def test_bf16_rounding_is_nearest_even():
    import numpy as np
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5e-3], np.float32)
    r = synthetic.bf16_round(x)
    assert r[0] == 1.0
    assert r[1] == 1.0                      # tie -> even (mantissa 0)
    assert r[2] == 1.0 + 4 * 2 ** -8        # tie -> even (rounds up)
    assert r[3] == 1.0
    assert abs(r[4] + 2.5e-3) < 2e-5


def test_log_flag_writes_errors_to_stderr():
    """AR_HIP_LOG=1: every error message the library sets is also written to stderr."""
    import sys
    code = ("import ctypes; from common_amd import hardware as hw; "
            "assert hw.lib().ar_hip_device_count(None) == hw.AR_HIP_ERR_INVALID")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for flag, expect in (("1", True), ("0", False)):
        env = dict(os.environ, AR_HIP_LOG=flag, PYTHONPATH=root)
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, cwd=root)
        assert r.returncode == 0, r.stderr
        assert ("[ar_hip] count is null" in r.stderr) == expect, r.stderr


def test_kv_dtype_default_from_environment(monkeypatch):
    from common_amd import config as C
    monkeypatch.delenv("AR_HIP_KV_DTYPE", raising=False)
    assert C.Qwen3Config(dim=64, hidden_dim=64, layer_count=1, head_count=1, kv_head_count=1, vocab_size=8,
                         seq_len=4).kv_dtype == C.DTYPE_F32
    monkeypatch.setenv("AR_HIP_KV_DTYPE", "fp16")
    assert C.Qwen3Config(dim=64, hidden_dim=64, layer_count=1, head_count=1, kv_head_count=1, vocab_size=8,
                         seq_len=4).kv_dtype == C.DTYPE_F16
    monkeypatch.setenv("AR_HIP_KV_DTYPE", "int4")
    with pytest.raises(ValueError):
        C.Qwen3Config(dim=64, hidden_dim=64, layer_count=1, head_count=1, kv_head_count=1, vocab_size=8, seq_len=4)
