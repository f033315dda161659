"""The debug pointer check (AR_HIP_CHECK_PTRS=1) over the decode path, in a child process (the flag is
read once per process): every launch of the step begin, GEMV, attention + split combine and persistent
kernels first checks each device pointer argument's extent against the HIP allocation that holds it.
The workloads: the C4 layer shape (bf16, 2 layers) with a 2048-token prompt, eager steps on the
persistent kernel and then as separate launches (attention + combine over 2K-row splits); the C5 layer
shape at batch 8 (MFMA GEMVs with operand planes and the k-split workspace); the C3 layer shape
(fp32).  Every launch must pass, and the checks must have run."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r'''
import ctypes, dataclasses, json, sys
sys.path.insert(0, ROOT)
import numpy as np
from common_amd import config as C, hardware as hw, synthetic
from common_amd.qwen3 import Qwen3
out = {}
def run(label, cfg, T, steps, batch=1, both=True):
    sd = synthetic.state_dict(cfg, seed=5)
    prompts = synthetic.prompt_ids(T, cfg.vocab_size, seed=6, batch=batch)
    prompts = prompts if batch > 1 else [prompts]
    with Qwen3(cfg, sd) as m:
        am = m.model
        am.use_graph(False)
        for persistent in ((True, False) if both else (am.persistent,)):
            am.use_persistent(persistent)
            am.reset()
            for b in range(batch):
                am.set_prompt(prompts[b], seq=b)
            am.prefill()
            toks = [am.next(return_logits=True)[0] for _ in range(steps)]
            out[f"{label}/{'persistent' if am.persistent else 'separate'}"] = np.stack(toks, axis=1).tolist()
run("c4", dataclasses.replace(C.C4_1_7B, layer_count=2, vocab_size=4096, shared_weights=False, seq_len=2048 + 16), 2048, 8)
run("c5", dataclasses.replace(C.C5_4B, layer_count=2, vocab_size=4096, shared_weights=False, seq_len=256, max_batch=8), 192, 4, batch=8, both=False)
run("c3", dataclasses.replace(C.C3_0_6B, layer_count=2, vocab_size=4096, shared_weights=False, seq_len=160), 128, 8)
n = ctypes.c_ulonglong()
hw.check(hw.lib().ar_hip_pointer_checks(ctypes.byref(n)))
out["checks"] = n.value
print(json.dumps(out))
'''.replace("ROOT", repr(ROOT))


def test_decode_path_pointer_ranges_inside_their_allocations():
    env = dict(os.environ, AR_HIP_CHECK_PTRS="1")
    p = subprocess.run([sys.executable, "-c", CHILD], env=env, capture_output=True, text=True, timeout=240)
    assert p.returncode == 0, p.stderr[-3000:]
    res = json.loads(p.stdout.strip().splitlines()[-1])
    print(f"pointer ranges checked: {res['checks']}", flush=True)
    assert res["checks"] > 1000, res["checks"]
    for k in ("c4/persistent", "c4/separate", "c5/separate", "c3/persistent", "c3/separate"):
        assert k in res, sorted(res)
    # the check changes nothing the kernels compute: the two forms agree token for token
    assert res["c4/persistent"] == res["c4/separate"] and res["c3/persistent"] == res["c3/separate"]
