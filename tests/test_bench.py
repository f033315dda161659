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
    for name in ("c2_section", "c4_section", "c5_section", "traffic_probe", "load_traffic", "step_bytes_batch",
                 "prefill_flops", "kernel_bytes", "algorithmic_bytes_per_token"):
        assert callable(getattr(b, name)), name
    tr = b.load_traffic()
    assert tr is not None and tr["hbm_bytes_per_launch"] > tr["algorithmic_bytes_per_launch"] * 0.99


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
