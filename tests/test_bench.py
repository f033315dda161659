"""bench.py is the driver's entry point: its helpers must all exist and its static inputs parse
(no GPU needed)."""
import ast
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_every_called_module_function_exists():
    tree = ast.parse(open(os.path.join(ROOT, "bench.py")).read())
    defined = {n.name for n in tree.body if isinstance(n, ast.FunctionDef)}
    called = {n.func.id for n in ast.walk(tree) if isinstance(n, ast.Call) and isinstance(n.func, ast.Name)}
    local_names = {n.id for n in ast.walk(tree) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Store)}
    local_names |= {a.arg for n in ast.walk(tree) if isinstance(n, (ast.FunctionDef, ast.Lambda))
                    for a in n.args.args}
    local_names |= {n.name for n in ast.walk(tree) if isinstance(n, ast.FunctionDef)}
    local_names |= {(a.asname or a.name).split(".")[0] for n in ast.walk(tree)
                    if isinstance(n, (ast.Import, ast.ImportFrom)) for a in n.names}
    import builtins as _b
    builtins = set(dir(_b))
    missing = sorted(c for c in called if c not in defined and c not in local_names and c not in builtins)
    assert not missing, missing


def test_sections_and_traffic_file():
    b = _load_bench()
    for name in ("c2_section", "c4_section", "c5_section", "traffic_probe", "load_traffic", "traffic_summary",
                 "c3_class_bytes", "step_bytes_batch", "prefill_flops", "kernel_bytes", "algorithmic_bytes_per_token"):
        assert callable(getattr(b, name)), name
    tr = b.load_traffic()
    assert isinstance(tr, dict)
    for name, e in tr.items():  # the committed counter summary: every weight byte read at least once
        if name.endswith("_gemv_swiglu") or name.endswith("_gemv_residual") or name.endswith("_gemv_rmsnorm"):
            assert e["hbm_bytes_per_launch"] > 0.99 * e["algorithmic_bytes_per_launch"], name


def test_traffic_summary_scales_counters_by_the_copy(tmp_path, capsys):
    """The counter passes' CSVs -> per-class bytes: each counter is scaled so that the probe's plain
    256 MiB copy reads (FETCH) / writes (WRITE) exactly its size."""
    import json
    b = _load_bench()
    hdr = "Kernel_Name,Counter_Name,Counter_Value\n"
    gu = b.C3_CLASS_KERNELS["gate_up_gemv_swiglu"]
    for d, counter, copy_kib, gu_kib in (("f", "FETCH_SIZE", 131072.0, 12300.0), ("w", "WRITE_SIZE", 262144.0, 12.0)):
        (tmp_path / d).mkdir()
        rows = [f"__amd_rocclr_copyBuffer,{counter},{copy_kib}", f'"{gu}(gemv::Params, int)",{counter},{gu_kib}',
                f'"{gu}(gemv::Params, int)",{counter},{gu_kib + 2}']
        (tmp_path / d / "run_counter_collection.csv").write_text(hdr + "\n".join(rows) + "\n")
    b.traffic_summary(str(tmp_path / "f"), str(tmp_path / "w"))
    out = json.loads(capsys.readouterr().out)
    assert abs(out["fetch_scale"] - 2.0) < 1e-9 and abs(out["write_scale"] - 1.0) < 1e-9
    e = out["classes"]["gate_up_gemv_swiglu"]
    assert e["launches"] == 2
    assert e["fetch_bytes_per_launch"] == round(12301.0 * 1024 * 2.0)
    assert e["write_bytes_per_launch"] == round(13.0 * 1024)
    assert e["algorithmic_bytes_per_launch"] == b.kernel_bytes(b_cfg(), 2)


def b_cfg():
    from common_amd import config as C
    return C.C3_0_6B


def test_step_bytes_consistent():
    b = _load_bench()
    from common_amd import config as C
    cfg = C.C5_4B
    one = b.step_bytes_batch(cfg, 100, 1)
    assert abs(one - b.algorithmic_bytes_per_token(cfg, 100)) < 1
    # halving the cache element halves only the KV part
    kv32 = b.step_bytes_batch(cfg, 100, 8) - b.step_bytes_batch(cfg, 0, 8)
    kv16 = b.step_bytes_batch(cfg, 100, 8, 2) - b.step_bytes_batch(cfg, 0, 8, 2)
    assert abs(kv32 - 2 * kv16) < 1
