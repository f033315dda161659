"""Qwen3 decode benchmark on one MI355X (BASELINE metric: decode tok/s + % HBM roofline,
Qwen3-0.6B shape, batch 1; prefill tok/s).

Workload: Qwen3-0.6B shape, fp32 weights, random init N(0, 0.02) from a
seed (synthetic; no checkpoint), prompt of 128 uniform random token ids, greedy decode.  A
"step" is one decode token.  The prompt (positions 0..127) and `--warmup` tokens run untimed;
then exactly `--steps` tokens are timed with the tokens kept on the device (no host round
trip inside the timed region).  Default: warmup 5 + 251 timed = the config's 256 decode tokens.

Extra fields on the JSON line:
  roofline      dominant kernel's achieved HBM GB/s: the persistent decode kernel (every layer, the
                final norm, the logits and the greedy keys of a step in one launch), its average
                launch timed by HIP events on the model's stream over --probe-steps eager steps,
                against the step's algorithmic bytes
  multi_launch  the same decode as separate launches per layer (tok/s over MULTI_STEPS steps), each
                kernel class timed by HIP events carried in its dispatches and by a graph-replayed
                loop of its launches over the layers (roofline of its dominant class and of its
                logits GEMV)
  cpu_baseline  the CPU oracle (reference semantics, fp32) on this host, over a bounded sample
  c4            BASELINE config 4 (Qwen3-1.7B shape, bf16 weights): a 2048-token prompt through the
                MFMA prefill path (tok/s and fraction of the 2.5 PFLOP/s dense bf16/fp16 MFMA peak),
                then greedy decode tok/s and HBM fraction on the same model
  c5            BASELINE config 5 (Qwen3-4B shape, bf16 weights): 8 sequences x 8192-token prompts
                prefilled together, then 64 greedy steps of all 8 (aggregate tok/s, HBM fraction)
  c2            BASELINE config 2: the decode-step attention op at a 4096-row cache (us per call)
  llama2        the Llama2 family: a stories110M-shaped llama2.c checkpoint (synthetic weights)
                loaded through the checkpoint path, greedy decode tok/s and HBM fraction
  sampled_c3    the C3 decode with on-device sampling instead of greedy selection: sampleToken
                at temperature 0.8 / top-p 0.9, and the sample function of AutoregressiveModel.of
                at temperature 0.7 (tok/s)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def algorithmic_bytes_per_token(cfg, pos):
    """Bytes one decode step must move at position `pos` (weights once + KV read/write)."""
    wb = 4 if cfg.weight_dtype == 0 else 2
    layer_w = cfg.layer_weight_params() * wb
    norms = (2 * cfg.dim + cfg.q_dim + cfg.kv_dim) * 4
    head = cfg.vocab_size * cfg.dim * wb
    kv = cfg.layer_count * 2 * cfg.kv_dim * 4 * (pos + 1)
    return cfg.layer_count * (layer_w + norms) + head + cfg.dim * 4 + kv


def kernel_bytes(cfg, which, batch=1):
    from common_amd import qwen3 as q
    wb = 4 if cfg.weight_dtype == 0 else 2
    d, F, V = cfg.dim, cfg.hidden_dim, cfg.vocab_size
    act = 4 * batch
    if which == q.KT_LOGITS:
        return V * d * wb + d * 4 + d * act
    if which == q.KT_GATE_UP:
        return 2 * F * d * wb + d * 4 + d * act + F * act
    if which == q.KT_QKV:
        n = cfg.q_dim + 2 * cfg.kv_dim
        return n * d * wb + d * 4 + d * act + n * act
    if which == q.KT_DOWN:
        return d * F * wb + F * act + 2 * d * act
    if which == q.KT_O:
        return d * cfg.q_dim * wb + cfg.q_dim * act + 2 * d * act
    return None


MFMA_PEAK_TFLOPS = 2500.0      # dense bf16 / fp16
MFMA_F32_PEAK_TFLOPS = 157.3   # dense fp32


def prefill_flops(cfg, T):
    """Useful FLOPs of a T-token prefill: linear layers, causal attention, last-row logits."""
    linear = 2.0 * T * cfg.layer_count * cfg.layer_weight_params()
    attn = cfg.layer_count * 2 * 2 * cfg.head_count * cfg.head_size * T * (T + 1) / 2
    return linear + attn + 2.0 * cfg.vocab_size * cfg.dim


def c4_section(args):
    """prefill 2048 tokens on the MFMA path, then greedy decode."""
    import dataclasses

    import numpy as np

    from common_amd import config as C
    from common_amd import synthetic
    from common_amd.qwen3 import Qwen3

    T, n_dec = C.C4_PROMPT, C.C4_DECODE
    cfg = dataclasses.replace(C.C4_1_7B, seq_len=T + n_dec + 8)
    prompt = synthetic.prompt_ids(T, cfg.vocab_size, seed=args.seed + 4)
    t0 = time.time()
    model = Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=args.seed + 4))
    log(f"[bench] C4 weights generated + uploaded in {time.time() - t0:.1f}s")
    am = model.model
    am.use_graph(not args.no_graph)
    am.reset()
    am.set_prompt(prompt)
    am.prefill()  # first call makes the fp16 weight copies and the prefill buffers

    def timed_prefills():
        ts = []
        for _ in range(3):
            am.reset()
            am.set_prompt(prompt)
            model.ctx.synchronize()
            tp = time.perf_counter()
            am.prefill()
            ts.append(time.perf_counter() - tp)
        return min(ts)

    from common_amd import qwen3 as q
    t_pre = timed_prefills()
    # the same prefill with the products on the library's own fused MFMA kernels (one warm call)
    am.prefill_gemm = q.PREFILL_GEMM_OWN
    am.reset()
    am.set_prompt(prompt)
    am.prefill()
    t_pre_own = timed_prefills()
    am.prefill_gemm = q.PREFILL_GEMM_ROCBLAS
    flops = prefill_flops(cfg, T)
    warm = 5
    am.run(warm)
    model.ctx.synchronize()
    td = time.perf_counter()
    am.run(n_dec - warm)
    t_dec = time.perf_counter() - td
    model.close()
    dec_tok_s = (n_dec - warm) / t_dec
    bytes_tok = float(np.mean([algorithmic_bytes_per_token(cfg, p) for p in range(T + warm, T + n_dec)]))
    out = {
        "workload": "C4: Qwen3-1.7B shape bf16 weights (d2048, 28L, 16Q/8KV, hd128, F6144, V151936), batch 1",
        "prefill": {"tokens": T, "ms": round(1000 * t_pre, 3), "tok_s": round(T / t_pre, 1),
                    "tflop": round(flops / 1e12, 3), "achieved_tflops": round(flops / t_pre / 1e12, 1),
                    "mfma_frac": round(flops / t_pre / 1e12 / MFMA_PEAK_TFLOPS, 4),
                    "path": "fp16 products on exact fp16 copies of the bf16 weights (rocBLAS gemm_ex, the default "
                            "ar_hip_qwen3_prefill_gemm backend) + causal flash attention",
                    "own_kernels": {"ms": round(1000 * t_pre_own, 3),
                                    "achieved_tflops": round(flops / t_pre_own / 1e12, 1),
                                    "path": "the library's fused MFMA GEMMs (AR_PREFILL_GEMM_OWN) + causal flash attention"}},
        "decode": {"tokens": n_dec - warm, "tok_s": round(dec_tok_s, 2), "ms_per_token": round(1000 * t_dec / (n_dec - warm), 4),
                   "algorithmic_bytes_per_token": round(bytes_tok),
                   "hbm_frac": round(bytes_tok * dec_tok_s / 1e9 / HBM_PEAK_GBS, 4)},
    }
    log(f"[bench] C4 prefill {T} tokens: {1000 * t_pre:.2f} ms = {T / t_pre:.0f} tok/s, "
        f"{flops / t_pre / 1e12:.0f} TFLOP/s ({100 * flops / t_pre / 1e12 / MFMA_PEAK_TFLOPS:.1f}% of MFMA peak); "
        f"decode {dec_tok_s:.1f} tok/s ({100 * out['decode']['hbm_frac']:.1f}% of HBM)")
    return out


def c5_section(args):
    """8 independent sequences, each an 8192-token prompt through the MFMA
    prefill path, then greedy decode of all 8 together (long-context GQA decode)."""
    import dataclasses

    import numpy as np

    from common_amd import config as C
    from common_amd import synthetic
    from common_amd.qwen3 import Qwen3

    B, T, n_dec = C.C5_BATCH, C.C5_PROMPT, C.C5_DECODE
    base = dataclasses.replace(C.C5_4B, seq_len=T + n_dec + 8, max_batch=B)
    prompts = [synthetic.prompt_ids(T, base.vocab_size, seed=args.seed + 500 + b) for b in range(B)]
    warm = 4
    steps = n_dec - warm

    def run(kv_dtype):
        cfg = dataclasses.replace(base, kv_dtype=kv_dtype)
        t0 = time.time()
        model = Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=args.seed + 5))
        log(f"[bench] C5 weights generated + uploaded in {time.time() - t0:.1f}s")
        am = model.model
        am.use_graph(not args.no_graph)

        def start():
            am.reset()
            for b, p in enumerate(prompts):
                am.set_prompt(p, seq=b)
            model.ctx.synchronize()

        start()
        am.prefill()  # first call makes the fp16 weight copies and the prefill buffers
        start()
        tp = time.perf_counter()
        am.prefill()
        t_pre = time.perf_counter() - tp
        am.run(warm)
        model.ctx.synchronize()
        td = time.perf_counter()
        toks = am.run(steps)
        t_dec = time.perf_counter() - td
        model.close()
        kv_b = 2 if kv_dtype == C.DTYPE_F16 else 4
        step_bytes = float(np.mean([step_bytes_batch(cfg, p, B, kv_b) for p in range(T + warm, T + n_dec)]))
        dec = {"steps": steps, "tok_s": round(B * steps / t_dec, 1), "ms_per_step": round(1000 * t_dec / steps, 3),
               "algorithmic_bytes_per_step": round(step_bytes),
               "hbm_frac": round(step_bytes * steps / t_dec / 1e9 / HBM_PEAK_GBS, 4),
               "kv_cache": "fp16" if kv_dtype == C.DTYPE_F16 else "fp32"}
        return t_pre, dec, toks

    t_pre, dec, toks = run(C.DTYPE_F32)
    flops = B * prefill_flops(base, T)
    out = {
        "workload": "C5: Qwen3-4B shape bf16 weights (d2560, 36L, 32Q/8KV, hd128, F9728, V151936), "
                    f"batch {B} x {T}-token prompts, greedy decode {n_dec}",
        "prefill": {"tokens": B * T, "ms": round(1000 * t_pre, 2), "tok_s": round(B * T / t_pre, 1),
                    "tflop": round(flops / 1e12, 2), "achieved_tflops": round(flops / t_pre / 1e12, 1),
                    "mfma_frac": round(flops / t_pre / 1e12 / MFMA_PEAK_TFLOPS, 4)},
        "decode": dec,
        "distinct_sequences": int(len({tuple(t) for t in toks})),
    }
    log(f"[bench] C5 prefill {B}x{T} tokens: {1000 * t_pre:.1f} ms = {B * T / t_pre:.0f} tok/s, "
        f"{flops / t_pre / 1e12:.0f} TFLOP/s; decode {dec['tok_s']} tok/s aggregate, "
        f"{dec['ms_per_step']} ms/step ({100 * dec['hbm_frac']:.1f}% of HBM)")
    if not args.no_fp16_kv:
        _, dec16, toks16 = run(C.DTYPE_F16)
        dec16["tokens_equal_fp32_cache"] = int(np.sum(toks16 == toks))
        dec16["tokens_compared"] = int(toks.size)
        out["decode_fp16_kv"] = dec16
        log(f"[bench] C5 decode with an fp16 KV cache: {dec16['tok_s']} tok/s aggregate, {dec16['ms_per_step']} "
            f"ms/step ({100 * dec16['hbm_frac']:.1f}% of HBM); {dec16['tokens_equal_fp32_cache']}/{toks.size} "
            f"greedy tokens equal to the fp32-cache run")
    return out


def c2_section(args):
    """the decode-step GQA attention op (16 Q / 8 KV heads, hd 128, cache filled
    to 4096 rows, query at position 4096) through ar_hip_attention_decode.  Eight caches are used in
    turn (8 x 33.6 MB > the 256 MB Infinity Cache) so every call streams its cache from HBM."""
    import numpy as np

    from common_amd import hardware as hw

    H, KV, HD, pos = 16, 8, 128, 4096
    S = pos + 1
    ncache, calls = 8, 200
    r = np.random.default_rng(args.seed + 2)
    with hw.HipContext() as ctx:
        caches = []
        for i in range(ncache):
            kc = r.standard_normal(KV * S * HD, dtype=np.float32)
            vc = r.standard_normal(KV * S * HD, dtype=np.float32)
            caches.append((ctx.to_device(kc), ctx.to_device(vc)))
        q = ctx.to_device(r.standard_normal(H * HD, dtype=np.float32))
        k = ctx.to_device(r.standard_normal(KV * HD, dtype=np.float32))
        v = ctx.to_device(r.standard_normal(KV * HD, dtype=np.float32))
        qn = ctx.to_device((1 + 0.02 * r.standard_normal(H * HD)).astype(np.float32))
        kn = ctx.to_device((1 + 0.02 * r.standard_normal(KV * HD)).astype(np.float32))
        out = ctx.allocate(H * HD * 4)

        def call(i):
            kc, vc = caches[i % ncache]
            ctx.attention_decode(q, k, v, qn, kn, 1e-6, 0, kc, vc, S, pos, H, KV, HD, 1e6, out)

        for i in range(2 * ncache):
            call(i)
        ctx.synchronize()
        t = time.perf_counter()
        for i in range(calls):
            call(i)
        ctx.synchronize()
        us = 1e6 * (time.perf_counter() - t) / calls
    kv_bytes = 2 * KV * S * HD * 4
    gbs = kv_bytes / us / 1e3
    log(f"[bench] C2 attention op: {us:.2f} us/call, {gbs:.0f} GB/s of K/V ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM)")
    return {"workload": "C2: decode-step GQA attention op, 16Q/8KV heads, hd 128, cache 0..4095 + new row at 4096, fp32",
            "us_per_call": round(us, 2), "kv_bytes": kv_bytes, "GBs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "note": "wall time per C-ABI call (host-side argument checks, one attention launch and its split "
                    "combine launch, no copies)"}


TRAFFIC_STEPS = 8


def traffic_probe(args):
    """Workload for the rocprofv3 FETCH_SIZE / WRITE_SIZE passes behind roofline.traffic: one plain
    256 MiB device copy (the counter scale: known bytes), the C3 prompt (128 tokens) through the
    prefill, then TRAFFIC_STEPS eager C3 decode steps at positions 128.. with the persistent kernel
    (when the model runs it) and TRAFFIC_STEPS more as separate launches, so every launch of every
    decode kernel is its own dispatch."""
    from common_amd import config as C
    from common_amd import hardware as hw
    from common_amd import synthetic
    from common_amd.qwen3 import Qwen3

    nbytes = 256 << 20
    cfg = C.C3_0_6B
    prompt = synthetic.prompt_ids(C.C3_PROMPT, cfg.vocab_size, seed=args.seed)
    with hw.HipContext() as ctx:
        a, b = ctx.allocate(nbytes), ctx.allocate(nbytes)
        ctx.copy(b, a, nbytes)
        ctx.synchronize()
        with Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=args.seed), ctx) as model:
            am = model.model
            am.use_graph(False)
            am.reset()
            am.set_prompt(prompt)
            am.prefill()
            am.run(TRAFFIC_STEPS)
            am.use_persistent(False)
            am.run(TRAFFIC_STEPS)
            am.use_persistent(True)
            ctx.synchronize()
    print(json.dumps({"traffic_probe": {"copy_bytes": nbytes, "prompt": C.C3_PROMPT, "decode_steps": TRAFFIC_STEPS}}),
          flush=True)


PREFILL_PROBE_RUNS = 2
MULTI_STEPS = 64  # timed steps of the multi-launch comparison run
LOOP_ROUNDS = 8  # loop probe: launches per layer (x layers) for each weight-streaming decode class


def prefill_probe(args):
    """Workload for the rocprofv3 counter passes over the prefill kernels (MFMA busy, VALU busy, LDS
    bank conflicts): the C3 prompt (128 tokens, fp32 weights, fp32 MFMA path) or the C4 prompt
    (2048 tokens, bf16 weights, fp16 MFMA path) through the batched prefill, a warm call and
    PREFILL_PROBE_RUNS more.  No decode step is launched."""
    import dataclasses

    from common_amd import config as C
    from common_amd import synthetic
    from common_amd.qwen3 import Qwen3

    if args.prefill_probe == "c3":
        cfg, T, seed = C.C3_0_6B, C.C3_PROMPT, args.seed
    else:
        cfg, T, seed = C.C4_1_7B, C.C4_PROMPT, args.seed + 4
        cfg = dataclasses.replace(cfg, seq_len=T + 8)
    prompt = synthetic.prompt_ids(T, cfg.vocab_size, seed=seed)
    with Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=seed)) as model:
        am = model.model
        am.use_graph(False)
        for _ in range(1 + PREFILL_PROBE_RUNS):
            am.reset()
            am.set_prompt(prompt)
            am.prefill()
        model.ctx.synchronize()
        by_steps = am.prefill_by_steps()
    print(json.dumps({"prefill_probe": {"workload": args.prefill_probe, "prompt": T, "runs": 1 + PREFILL_PROBE_RUNS,
                                        "by_steps": by_steps}}), flush=True)


TRACE_MARKS = ["layer start", "QKV input (thread 0)", "QKV stored", "attention input (thread 0)", "attention stored",
               "merge input (thread 0)", "merge stored", "O input (thread 0)", "O stored", "gate/up input (thread 0)",
               "gate/up stored", "down input (thread 0)", "down stored", "final input", "logits end",
               "QKV all inputs", "attention all inputs", "attention q/k normalised", "attention rows scored (wave 0)",
               "attention waves merged", "merge all inputs", "O all inputs", "gate/up all inputs", "down all inputs"]
TRACE_STEPS = 24


def profile_tree(args):
    """The C3 model's decode step as a profile tree (common_amd.profile): the prompt through the batched
    prefill, 5 warm-up steps, then PROFILE_STEPS steps per kernel class (the persistent launch, then
    each class of the step as separate launches), written as the XML document the reference's
    OperationProfileNode.load reads and printed as an indented summary and one JSON line."""
    from common_amd import config as C
    from common_amd import profile as prof
    from common_amd import synthetic
    from common_amd.qwen3 import Qwen3

    cfg = C.C3_0_6B
    prompt = synthetic.prompt_ids(C.C3_PROMPT, cfg.vocab_size, seed=args.seed)
    model = Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=args.seed))
    am = model.model
    am.reset()
    am.set_prompt(prompt)
    am.prefill()
    am.run(5)
    tree = prof.decode_profile(am, PROFILE_STEPS, name="C3 decode")
    prof.save(tree, args.profile_tree)
    log(prof.summary(tree))
    print(json.dumps({"profile_tree": {"xml": args.profile_tree, "tree": tree}}), flush=True)


PROFILE_STEPS = 16


def stage_trace(args):
    """Per-stage timeline of the persistent decode kernel at C3 (or C4 with --stage-trace c4): needs the
    diagnostic build (python -m common_amd.build --trace, loaded with AR_HIP_LIB=common_amd/lib/trace/
    libar_hip.so), whose kernel records the wall clock (10 ns ticks, common to all CUs) at every stage
    boundary of every layer in thread 0 of every block.  The prompt is prefilled, TRACE_STEPS decode
    steps are traced one by one; per layer (layers 1..L-2), times are taken from the median block's
    layer start: the median over the blocks that run a stage of its input / stored marks, the slowest
    producer's store, and the exchange latency = consumers' median input - slowest producer's store.
    Printed as one JSON line; medians over layers and steps."""
    import ctypes
    import dataclasses

    import numpy as np

    from common_amd import config as C
    from common_amd import hardware as hw
    from common_amd import synthetic
    from common_amd.qwen3 import Qwen3

    L_lib = hw.lib()
    if not hasattr(L_lib, "ar_hip_pk_trace_read"):
        raise SystemExit("stage trace: load the trace build (AR_HIP_LIB=common_amd/lib/trace/libar_hip.so)")
    if args.stage_trace == "c4":
        cfg, T = C.C4_1_7B, C.C4_PROMPT
    else:
        cfg, T = C.C3_0_6B, C.C3_PROMPT
    cfg = dataclasses.replace(cfg, seq_len=max(cfg.seq_len, T + 8 + TRACE_STEPS))
    prompt = synthetic.prompt_ids(T, cfg.vocab_size, seed=args.seed)
    buf = np.zeros((64, 256, 24), np.uint64)
    L_lib.ar_hip_pk_trace_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    G = cfg.head_count // cfg.kv_head_count
    rows = {k: [] for k in ("input", "stored", "slowest_store", "exchange", "att", "mrg", "free")}
    per_layer_us = []
    with Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=args.seed)) as model:
        am = model.model
        assert am.persistent, "the stage trace needs the persistent decode kernel"
        am.reset()
        am.set_prompt(prompt)
        am.prefill()
        am.run(5)
        smax = 8 if cfg.dim == 1024 else 28
        for step in range(TRACE_STEPS):
            pos = T + 5 + step
            am.run(1)
            hw.check(L_lib.ar_hip_pk_trace_read(buf.ctypes.data, buf.nbytes))
            nsplit = min(max(-(-(pos + 1) // 32), 1), smax)
            att = np.arange(cfg.kv_head_count * nsplit)
            mrg = np.arange(256 - cfg.head_count, 256)
            if nsplit > 1:  # the split merge may run in dedicated blocks or in the attention blocks
                lt = buf[2].astype(np.int64)
                t_ref = np.median(lt[:, 0])
                alt = np.arange(min(cfg.head_count, cfg.kv_head_count * nsplit))
                if np.median(np.abs(lt[alt, 5] - t_ref)) < np.median(np.abs(lt[mrg, 5] - t_ref)):
                    mrg = alt
            allb = np.arange(256)
            who = {1: allb, 2: allb, 3: att, 4: att, 5: mrg, 6: mrg, 7: allb, 8: allb, 9: allb, 10: allb, 11: allb,
                   12: allb, 15: allb, 16: att, 17: att, 18: att, 19: att, 20: mrg, 21: allb, 22: allb, 23: allb}
            # each stage's input: (consumer all-inputs mark, producer stored mark, producer blocks, layer offset)
            feeds = {"QKV": (15, 12, allb, -1), "attention": (16, 2, allb, 0), "merge": (20, 4, att, 0),
                     "O": (21, 6, mrg, 0), "gate/up": (22, 8, allb, 0), "down": (23, 10, allb, 0)}
            for l in range(1, cfg.layer_count - 1):
                t = buf[l].astype(np.int64)
                t0 = np.median(t[:, 0])
                per_layer_us.append((np.median(buf[l + 1][:, 0].astype(np.int64)) - t0) * 0.01)
                inp = {k: (np.median(t[who[k], k]) - t0) * 0.01 for k in who}
                rows["input"].append([inp.get(k, np.nan) for k in range(24)])
                ex = []
                for name, (ci, ps, pb, dl) in feeds.items():
                    prod = buf[l + dl].astype(np.int64)[pb, ps]
                    cons = t[who[ci], ci]
                    ex.append((np.median(cons) - prod.max()) * 0.01)
                rows["exchange"].append(ex)
                rows["slowest_store"].append([(t[who[k], k].max() - t0) * 0.01 if k in who else np.nan
                                              for k in range(24)])
                free = np.setdiff1d(allb, np.concatenate([att, mrg]))
                for g, bl in (("att", att), ("mrg", mrg), ("free", free)):
                    rows[g].append([(np.median(t[bl, k]) - t0) * 0.01 if who.get(k) is allb else np.nan
                                    for k in range(24)])
    med = lambda a: [round(float(v), 2) for v in np.nanmedian(np.array(a, np.float64), axis=0)]
    out = {"stage_trace": {"workload": args.stage_trace, "steps": TRACE_STEPS, "positions": f"{T + 5}..{T + 4 + TRACE_STEPS}",
                           "layer_us_median": round(float(np.median(per_layer_us)), 2),
                           "median_block_us": dict(zip(TRACE_MARKS, med(rows["input"]))),
                           "slowest_block_us": dict(zip(TRACE_MARKS, med(rows["slowest_store"]))),
                           "by_role_median_us": {g: dict(zip(TRACE_MARKS, med(rows[g])))
                                                 for g in ("att", "mrg", "free")},
                           "exchange_us": dict(zip(["QKV", "attention", "merge", "O", "gate/up", "down"],
                                                   med(rows["exchange"])))}}
    print(json.dumps(out), flush=True)


# kernel-name prefixes of the C3 decode classes in a rocprofv3 trace (batch 1, fp32 weights)
C3_CLASS_KERNELS = {
    "decode_persistent": "decode_persistent_kernel",
    "qkv_gemv_rmsnorm": "gemv_rx_kernel<float, 2, 4, 0>",
    "o_gemv_residual": "gemv_rx_kernel<float, 1, 8, 1>",
    "gate_up_gemv_swiglu": "gemv_rx_kernel<float, 2, 4, 2>",
    "down_gemv_residual": "gemv_rx_kernel<float, 1, 12, 1>",
    "attention_decode": "attn_decode_kernel",
    "attention_combine": "attn_combine_kernel",
    "logits_gemv_argmax": "gemv_argmax_kernel",
    "step_begin": "step_begin_kernel",
}


def c3_class_bytes(cfg, name, pos):
    """Algorithmic bytes of one launch of a C3 decode class at position `pos`."""
    from common_amd import qwen3 as q
    kt = {"qkv_gemv_rmsnorm": q.KT_QKV, "o_gemv_residual": q.KT_O, "gate_up_gemv_swiglu": q.KT_GATE_UP,
          "down_gemv_residual": q.KT_DOWN, "logits_gemv_argmax": q.KT_LOGITS}
    if name in kt:
        return kernel_bytes(cfg, kt[name])
    if name == "decode_persistent":  # the whole step but the step-begin kernel (which reads the embedding row)
        return algorithmic_bytes_per_token(cfg, pos)
    if name == "attention_decode":  # K and V rows 0..pos read, row pos written, q/k/v and gains in, out
        return 2 * (pos + 1) * cfg.kv_dim * 4 + 2 * cfg.kv_dim * 4 + (cfg.q_dim + 2 * cfg.kv_dim) * 4 * 2 + cfg.q_dim * 4
    return None


def traffic_summary(fetch_dir, write_dir):
    """Per-class HBM traffic from the two counter passes' CSVs (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    of `bench.py --traffic-probe`), each counter scaled by what it reads for the probe's plain copy of
    known size; prints the JSON that profiles/c3_decode_traffic.json holds."""
    import csv
    import glob

    from common_amd import config as C

    def read(d, counter):
        rows = []
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                rows += [r for r in csv.DictReader(f) if r.get("Counter_Name") == counter]
        return rows

    out = {"classes": {}}
    cfg = C.C3_0_6B
    pos_mean = C.C3_PROMPT + (TRAFFIC_STEPS - 1) / 2  # the persistent steps come first
    pos_mean_multi = pos_mean + TRAFFIC_STEPS
    for counter, d, key in (("FETCH_SIZE", fetch_dir, "fetch"), ("WRITE_SIZE", write_dir, "write")):
        rows = read(d, counter)
        copy = [float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]]
        if not copy:
            raise SystemExit(f"no copy dispatch in {d}")
        scale = (256 << 20) / (max(copy) * 1024.0)  # counter KiB -> bytes, calibrated on the copy
        out[f"{key}_scale"] = round(scale, 4)
        for name, prefix in C3_CLASS_KERNELS.items():
            vals = [float(r["Counter_Value"]) * 1024.0 * scale for r in rows if prefix in r["Kernel_Name"]]
            if vals:
                e = out["classes"].setdefault(name, {"kernel": prefix})
                e[f"{key}_bytes_per_launch"] = round(sum(vals) / len(vals))
                e["launches"] = len(vals)
    for name, e in out["classes"].items():
        alg = c3_class_bytes(cfg, name, pos_mean if name == "decode_persistent" else pos_mean_multi)
        e["hbm_bytes_per_launch"] = e.get("fetch_bytes_per_launch", 0) + e.get("write_bytes_per_launch", 0)
        e["algorithmic_bytes_per_launch"] = round(alg) if alg else None
        e["traffic_over_algorithmic"] = round(e["hbm_bytes_per_launch"] / alg, 4) if alg else None
    print(json.dumps(out, indent=1), flush=True)


def load_traffic():
    """Per-class HBM traffic from the committed rocprofv3 counter summary, when present."""
    path = os.path.join(ROOT, "profiles", "c3_decode_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("classes", {})
    except (OSError, ValueError):
        return {}


def llama2_section(args):
    """The Llama2 family (Llama2.java): a stories110M-shaped llama2.c checkpoint (d768, 12 layers,
    12 heads, F2048, V32000, seq 1024, tied classifier) with synthetic weights, written to a
    temporary file and loaded through the checkpoint path; BOS then greedy decode, timed over
    the decode steps as Llama2.main reports tokens per second (Llama2.java:80-96)."""
    import shutil
    import tempfile

    import numpy as np

    from common_amd.llama2 import BOS, Llama2, Llama2Config, write_checkpoint

    cfg = Llama2Config(768, 2048, 12, 12, 12, 32000, 1024, True, 64)
    d, F, L, V, S, hd = cfg.dim, cfg.hidden_dim, cfg.layer_count, cfg.vocab_size, cfg.seq_len, cfg.head_size
    rng = np.random.default_rng(args.seed + 7)

    def normal(shape, mean=0.0):
        return (mean + 0.02 * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)

    invf = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    ang = np.outer(np.arange(S), invf)
    w = {"tokenEmbeddings": normal((V, d)), "rmsAttWeights": normal((L, d), 1.0), "wq": normal((L, d, d)),
         "wk": normal((L, d, d)), "wv": normal((L, d, d)), "wo": normal((L, d, d)),
         "rmsFfn": normal((L, d), 1.0), "w1": normal((L, F, d)), "w2": normal((L, d, F)), "w3": normal((L, F, d)),
         "rmsFinalWeight": normal(d, 1.0), "freqCisReal": np.cos(ang), "freqCisImag": np.sin(ang)}
    tmp = tempfile.mkdtemp(prefix="llama2_bench_")
    try:
        path = os.path.join(tmp, "stories110M_synthetic.bin")
        write_checkpoint(path, cfg, w)
        del w
        t0 = time.time()
        with Llama2(path, None) as m:
            load_s = time.time() - t0
            am = m.model
            am.use_graph(not args.no_graph)
            am.reset()
            am.set_prompt([BOS])
            warm = 8
            am.run(1 + warm)
            steps = S - 1 - warm - 1
            m.ctx.synchronize()
            t1 = time.perf_counter()
            am.run(steps)
            el = time.perf_counter() - t1
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    weights = (V * d + L * (4 * d * d + 3 * d * F + 2 * d) + d) * 4
    pos0 = 1 + warm
    kv = float(np.mean([2 * (p + 1) * d * 4 * L for p in range(pos0, pos0 + steps)]))
    per_tok = weights + kv
    tok_s = steps / el
    log(f"[bench] Llama2 (stories110M shape, fp32): {1000 * el / steps:.3f} ms/token, {tok_s:.0f} tok/s; "
        f"checkpoint load {load_s:.2f} s")
    return {"workload": "Llama2: stories110M shape fp32 (d768, 12L, 12 heads, hd64, F2048, V32000, tied), "
                        "llama2.c checkpoint with synthetic N(0,0.02) weights, BOS + greedy decode",
            "steps": steps, "decode_positions": f"{pos0}..{pos0 + steps - 1}", "tok_s": round(tok_s, 1),
            "ms_per_token": round(1000 * el / steps, 4), "algorithmic_bytes_per_token": round(per_tok),
            "hbm_frac": round(per_tok * tok_s / 1e9 / HBM_PEAK_GBS, 4), "checkpoint_load_s": round(load_s, 2)}


CPU_RUNS, CPU_WARMUP, CPU_TOKENS = 3, 5, 20  # Qwen3BenchmarkTest.java:54-60 (runs, warm-up, timed tokens)


def cpu_model_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(cfg, prompt, seed, gpu_generated):
    """The reference-semantics CPU oracle timed on this host the way Qwen3BenchmarkTest times the
    reference (engine/ml/src/test/java/org/almostrealism/ml/qwen3/Qwen3BenchmarkTest.java:54-183):
    per precision, the C3 prompt is taken in by the oracle's batched prompt pass (untimed), then
    CPU_RUNS runs of CPU_WARMUP untimed and CPU_TOKENS timed greedy decode steps, each on
    max(2, nproc / 2) threads (the reference's JNI pool, KernelPreferences.java:68-71) and on all
    nproc threads.  FP64 is the reference's default precision (Hardware.java:684); FP32 is its
    AR_HARDWARE_PRECISION=FP32 mode and the GPU's arithmetic.  The greedy tokens of both are compared
    with the GPU's generated tokens over the positions both produced."""
    import numpy as np

    import oracle
    from common_amd import synthetic
    nproc = os.cpu_count() or 1
    half = max(2, nproc // 2)
    runs, parity = {}, {}
    for precision in ("fp64", "fp32"):
        t0 = time.perf_counter()
        ref = oracle.OracleQwen3(cfg, synthetic.iter_state_dict(cfg, seed=seed), precision=precision)
        oracle.set_threads(nproc)
        nxt, _ = ref.prefill(prompt, want_logits=False)
        setup_s = time.perf_counter() - t0
        generated = []
        for threads in (half, nproc):
            used = oracle.set_threads(threads)
            if threads == half:
                half_used = used
            per_run = []
            for _ in range(CPU_RUNS):
                for _ in range(CPU_WARMUP):
                    generated.append(nxt)
                    nxt, _ = ref.step(nxt, want_logits=False)
                tc = time.perf_counter()
                for _ in range(CPU_TOKENS):
                    generated.append(nxt)
                    nxt, _ = ref.step(nxt, want_logits=False)
                per_run.append(CPU_TOKENS / (time.perf_counter() - tc))
            runs[f"{precision}_{used}t"] = {"precision": precision, "threads": used,
                                            "tok_s_runs": [round(v, 3) for v in per_run],
                                            "tok_s_mean": round(float(np.mean(per_run)), 3)}
            log(f"[bench] cpu oracle {precision} on {used} threads: {runs[f'{precision}_{used}t']['tok_s_mean']} "
                f"tok/s (runs {runs[f'{precision}_{used}t']['tok_s_runs']})")
        ref.close()
        k = min(len(generated), len(gpu_generated))
        eq = int(np.sum(np.asarray(generated[:k]) == np.asarray(gpu_generated[:k])))
        parity[precision] = {"generated_tokens_compared": k, "equal": eq, "all_equal": bool(eq == k),
                             "setup_s": round(setup_s, 1)}
    primary = runs[f"fp64_{half_used}t"]
    return {"value": primary["tok_s_mean"], "unit": "tok/s", "cores": primary["threads"], "kind": "port",
            "precision": "fp64", "cpu_model": cpu_model_name(), "nproc": nproc, "runs": runs,
            "sample": f"C3 decode: prompt of {len(prompt)} tokens through the oracle's batched prompt pass (untimed), "
                      f"then per precision and thread count {CPU_RUNS} runs x ({CPU_WARMUP} warm-up + {CPU_TOKENS} "
                      f"timed greedy tokens), positions {len(prompt)}..{len(prompt) + 2 * CPU_RUNS * (CPU_WARMUP + CPU_TOKENS) - 1}; "
                      f"value = FP64 (reference default) on max(2, nproc/2) = {primary['threads']} threads"}, parity


def step_bytes_batch(cfg, pos, batch, kv_bytes=4):
    """Bytes one batched decode step must move at position `pos`: weights once, KV per sequence."""
    kv = cfg.layer_count * 2 * cfg.kv_dim * kv_bytes * (pos + 1)
    one = algorithmic_bytes_per_token(cfg, pos) - cfg.layer_count * 2 * cfg.kv_dim * 4 * (pos + 1) + kv
    return one + (batch - 1) * (kv + cfg.dim * 4)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=251)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--probe-steps", type=int, default=16)
    ap.add_argument("--cpu-steps", type=int, default=1, help="time the CPU oracle baseline (0: skip)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-c4", action="store_true", help="skip the config-4 prefill/decode section")
    ap.add_argument("--no-c5", action="store_true", help="skip the config-5 batch-8 long-context section")
    ap.add_argument("--no-c2", action="store_true", help="skip the config-2 attention-op section")
    ap.add_argument("--no-fp16-kv", action="store_true", help="skip the config-5 decode run with an fp16 KV cache")
    ap.add_argument("--no-llama2", action="store_true", help="skip the Llama2 (stories110M shape) section")
    ap.add_argument("--sections", default="c3,c4,c5,c2,llama2",
                    help="comma list of workloads to run (c3 is the headline; the others are extra fields)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only run the workload of the rocprofv3 FETCH_SIZE / WRITE_SIZE passes and exit")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise the two counter passes' CSV output directories per decode class and exit")
    ap.add_argument("--stage-trace", choices=("c3", "c4"),
                    help="per-stage timeline of the persistent decode kernel (needs the trace build) and exit")
    ap.add_argument("--profile-tree", metavar="XML",
                    help="time 16 C3 decode steps per kernel class, print the profile tree and write it to XML in "
                         "the reference's OperationProfileNode format, and exit")
    ap.add_argument("--prefill-probe", choices=("c3", "c4"),
                    help="only run that workload's prompt through the batched prefill (a warm call and "
                         "PREFILL_PROBE_RUNS more, no decode step) for rocprofv3 counter passes, and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the path has no "
              f"collectives. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.traffic_probe:
        traffic_probe(args)
        return
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary)
        return
    if args.prefill_probe:
        prefill_probe(args)
        return
    if args.stage_trace:
        stage_trace(args)
        return
    if args.profile_tree:
        profile_tree(args)
        return
    sections = {x.strip() for x in args.sections.split(",") if x.strip()}
    if "c3" not in sections:  # profiling aid: only the named extra sections, one JSON line of them
        out = {"c4": c4_section(args) if "c4" in sections and not args.no_c4 else None,
               "c5": c5_section(args) if "c5" in sections and not args.no_c5 else None,
               "c2": c2_section(args) if "c2" in sections and not args.no_c2 else None,
               "llama2": llama2_section(args) if "llama2" in sections and not args.no_llama2 else None}
        print(json.dumps(out), flush=True)
        return

    import numpy as np

    from common_amd import config as C
    from common_amd import qwen3 as q
    from common_amd import synthetic
    from common_amd.qwen3 import Qwen3

    cfg = C.C3_0_6B
    n_prompt = C.C3_PROMPT
    n_classes = 6  # kernel classes of the multi-launch step timed by the probe pass below
    total = n_prompt + args.warmup + args.steps + args.probe_steps * (n_classes + 1) + MULTI_STEPS + 2
    if total > cfg.seq_len:
        import dataclasses
        cfg = dataclasses.replace(cfg, seq_len=total)
    prompt = synthetic.prompt_ids(n_prompt, cfg.vocab_size, seed=args.seed)

    t0 = time.time()
    model = Qwen3(cfg, synthetic.iter_state_dict(cfg, seed=args.seed))
    info = model.ctx.info()
    log(f"[bench] weights generated + uploaded in {time.time() - t0:.1f}s on {info}")
    am = model.model
    am.use_graph(not args.no_graph)
    am.reset()
    am.set_prompt(prompt)

    # prompt token by token through the decode step (as AutoregressiveModel feeds it), timed once
    model.ctx.synchronize()
    tp = time.perf_counter()
    am.run(n_prompt)
    by_steps_s = time.perf_counter() - tp
    # the same prompt as one batched prefill (fp32 MFMA GEMMs + fp32 causal attention), best of 3;
    # the last one leaves the model at position n_prompt for the timed decode
    pre_times = []
    for _ in range(3):
        am.reset()
        am.set_prompt(prompt)
        model.ctx.synchronize()
        tp = time.perf_counter()
        am.prefill()
        pre_times.append(time.perf_counter() - tp)
    assert am.prefill_by_steps() == 0, "the C3 prompt must take the batched fp32 path"
    prefill_s = min(pre_times)
    pre_flops = prefill_flops(cfg, n_prompt)
    log(f"[bench] C3 prompt {n_prompt} tokens: batched fp32 prefill {1000 * prefill_s:.2f} ms = "
        f"{n_prompt / prefill_s:.0f} tok/s ({pre_flops / prefill_s / 1e12:.1f} TFLOP/s, "
        f"{100 * pre_flops / prefill_s / 1e12 / MFMA_F32_PEAK_TFLOPS:.1f}% of the fp32 MFMA peak); "
        f"token by token {n_prompt / by_steps_s:.0f} tok/s")
    fed_prompt = np.asarray(prompt, np.int32)[None, :]
    warm = am.run(args.warmup) if args.warmup else np.zeros((1, 0), np.int32)

    # ---- timed region ----------------------------------------------------------------
    # The persistent kernel is timed over these same steps: each launch's dispatch records a start /
    # stop event pair (hipExtLaunchKernel), which adds no packet or wait to the stream.
    if am.persistent:
        am.kernel_timing(q.KT_LAYERS)
    model.ctx.synchronize()
    t1 = time.perf_counter()
    toks = am.run(args.steps)  # enqueues K steps, synchronises once at the end
    t2 = time.perf_counter()
    if am.persistent:
        ms_k, n_k = am.kernel_time()
        am.kernel_timing(q.KT_NONE)
    elapsed = t2 - t1
    tok_s = args.steps / elapsed
    ms = 1000.0 * elapsed / args.steps
    pos0 = n_prompt + args.warmup
    mean_bytes = float(np.mean([algorithmic_bytes_per_token(cfg, p) for p in range(pos0, pos0 + args.steps)]))
    e2e_gbs = mean_bytes * tok_s / 1e9
    log(f"[bench] decode {args.steps} tokens: {ms:.3f} ms/token, {tok_s:.1f} tok/s, "
        f"{e2e_gbs:.0f} GB/s algorithmic ({100 * e2e_gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")

    traffic = load_traffic()
    persistent = am.persistent
    kernels = {}
    roofline = None
    # ---- the persistent kernel over the timed steps (events recorded by each launch's dispatch) ----
    # (one launch per step covers the 28 layers, the final norm, the logits and the greedy keys, so
    # its algorithmic bytes are the step's)
    probe_pos0 = pos0 + args.steps
    if persistent:
        avg_us = 1000.0 * ms_k / max(n_k, 1)
        b = float(np.mean([c3_class_bytes(cfg, "decode_persistent", p) for p in range(pos0, pos0 + n_k)]))
        gbs = b / avg_us / 1e3
        tr = traffic.get("decode_persistent", {})
        kernels["decode_persistent"] = {"avg_us": round(avg_us, 3), "launches": n_k, "bytes_per_launch": round(b),
                                        "GBs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                                        "share_of_step": round(avg_us / (1000.0 * ms), 4)}
        roofline = {"bound": "hbm", "kernel": "decode_persistent_kernel (28 layers + final RMSNorm + logits + "
                    "greedy keys, one launch per step)", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": tr.get("hbm_bytes_per_launch"),
                    "traffic_source": "profiles/c3_decode_traffic.md" if tr else None, "bytes_per_launch": round(b),
                    "avg_launch_us": round(avg_us, 3), "launches_timed": n_k,
                    "timing": "HIP events recorded by each launch's own dispatch (hipExtLaunchKernel) over the timed steps",
                    "share_of_step": round(avg_us / (1000.0 * ms), 4)}
        log(f"[bench] persistent decode kernel: {avg_us:.1f} us/launch = {gbs:.0f} GB/s "
            f"({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak), {100 * avg_us / (1000.0 * ms):.1f}% of the step")
        am.use_persistent(False)  # the comparison below runs the step as separate launches

    # ---- the step as separate launches: its tok/s, and each kernel class timed ---------------
    # (per class: a start / stop HIP event pair carried inside the class's own dispatches
    # (hipExtLaunchKernel), so each interval is kernel execution as rocprofv3's trace measures it)
    multi = None
    n_multi = min(MULTI_STEPS, cfg.seq_len - probe_pos0 - args.probe_steps * n_classes)
    if n_multi > 0:
        am.run(2)  # (captures the multi-launch step graph)
        model.ctx.synchronize()
        tm = time.perf_counter()
        am.run(n_multi)
        el = time.perf_counter() - tm
        multi = {"tok_s": round(n_multi / el, 1), "ms_per_step": round(1000.0 * el / n_multi, 4), "steps": n_multi,
                 "positions": f"{probe_pos0 + 2}..{probe_pos0 + 2 + n_multi - 1}"}
        probe_pos0 += 2 + n_multi
        log(f"[bench] the same decode as separate launches: {multi['ms_per_step']} ms/token, {multi['tok_s']} tok/s")
    names = {q.KT_LOGITS: "logits_gemv_argmax", q.KT_GATE_UP: "gate_up_gemv_swiglu", q.KT_QKV: "qkv_gemv_rmsnorm",
             q.KT_DOWN: "down_gemv_residual", q.KT_O: "o_gemv_residual", q.KT_ATTENTION: "attention_decode"}
    assert len(names) == n_classes
    per_class = min(args.probe_steps, (cfg.seq_len - probe_pos0) // n_classes)
    ms_multi = multi["ms_per_step"] if multi else ms
    for which, name in names.items():
        if per_class == 0:
            break
        am.kernel_timing(which)
        am.run(per_class)
        ms_k, n_k = am.kernel_time()
        am.kernel_timing(q.KT_NONE)
        avg_us = 1000.0 * ms_k / max(n_k, 1)
        per_tok_us = 1000.0 * ms_k / per_class
        probe_pos = probe_pos0 + (len(kernels) - int(persistent)) * per_class + (per_class - 1) / 2
        b = c3_class_bytes(cfg, name, probe_pos)
        kernels[name] = {"avg_us": round(avg_us, 3), "launches": n_k, "us_per_token": round(per_tok_us, 2),
                         "bytes_per_launch": round(b) if b else None, "GBs": round(b / avg_us / 1e3, 1) if b else None,
                         "hbm_frac": round(b / avg_us / 1e3 / HBM_PEAK_GBS, 4) if b else None,
                         "share_of_multi_launch_step": round(per_tok_us / (1000.0 * ms_multi), 4)}
        log(f"[bench] {name}: {avg_us:.2f} us/launch x {n_k // per_class}/token"
            + (f" = {b / avg_us / 1e3:.0f} GB/s" if b else ""))
    # ---- loop probe: each weight-streaming class alone, LOOP_ROUNDS launches per layer cycling
    # through the 28 layers' weights (so they stream from HBM as in the step), captured into one HIP
    # graph and timed by two events around its replay: the average launch duration with no event
    # inside any dispatch (the probe above carries ~1.2 us per dispatch for its events).  It
    # overwrites the step's activations; the sampling runs below reset the model first.
    loop_ids = {"qkv_gemv_rmsnorm": q.KT_QKV, "o_gemv_residual": q.KT_O, "gate_up_gemv_swiglu": q.KT_GATE_UP,
                "down_gemv_residual": q.KT_DOWN, "logits_gemv_argmax": q.KT_LOGITS}
    for name, which in loop_ids.items():
        if name not in kernels:
            continue
        per_tok = kernels[name]["launches"] // max(per_class, 1)
        reps = LOOP_ROUNDS * (per_tok if per_tok > 1 else 1)
        lus = am.kernel_loop(which, reps)
        b = kernels[name]["bytes_per_launch"]
        kernels[name].update({"loop_avg_us": round(lus, 3), "loop_launches": reps,
                              "loop_GBs": round(b / lus / 1e3, 1), "loop_hbm_frac": round(b / lus / 1e3 / HBM_PEAK_GBS, 4),
                              "loop_share_of_multi_launch_step": round(lus * per_tok / (1000.0 * ms_multi), 4)})
        log(f"[bench] {name} loop: {lus:.2f} us/launch over {reps} launches = {b / lus / 1e3:.0f} GB/s")
    am.use_persistent(True)

    def roof(name):  # a kernel of the multi-launch step (its loop-probe duration where there is one)
        kd = kernels[name]
        tr = traffic.get(name, {})
        looped = "loop_avg_us" in kd
        us = kd["loop_avg_us"] if looped else kd["avg_us"]
        gbs = kd["bytes_per_launch"] / us / 1e3
        return {"bound": "hbm", "kernel": name, "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": tr.get("hbm_bytes_per_launch"),
                "traffic_source": "profiles/c3_decode_traffic.md" if tr else None,
                "bytes_per_launch": kd["bytes_per_launch"], "avg_launch_us": round(us, 3),
                "timing": ("graph-replayed loop of the class's launches over the layers, two HIP events around it"
                           if looped else "HIP events inside the class's dispatches"),
                "probe_avg_launch_us": kd["avg_us"]}

    gemv_classes = [k for k in names.values() if k in kernels and k != "attention_decode" and kernels[k]["GBs"]]
    # the multi-launch step's dominant weight-streaming class (gate/up + SwiGLU at C3) and its logits GEMV
    roofline_multi = roof(max(gemv_classes, key=lambda k: kernels[k]["us_per_token"])) if gemv_classes else None
    roofline_logits = roof("logits_gemv_argmax") if "logits_gemv_argmax" in kernels else None
    if roofline is None:
        roofline = roofline_multi

    # ---- the same decode with on-device sampling instead of greedy selection ----------------
    sampled = {}
    for name, mode, temp, top_p in (("top_p", q.hw.SAMPLE_TOKEN, 0.8, 0.9), ("model_of", q.hw.SAMPLE_MODEL, 0.7, 1.0)):
        am.set_temperature(0.0)
        am.reset()
        am.set_prompt(prompt)
        am.run(n_prompt + args.warmup)
        am.set_sampling(mode, temp, top_p, seeds=[args.seed])
        n_s = min(args.steps, cfg.seq_len - (n_prompt + args.warmup))
        model.ctx.synchronize()
        ts = time.perf_counter()
        am.run(n_s)
        el = time.perf_counter() - ts
        sampled[name] = {"tok_s": round(n_s / el, 1), "ms_per_step": round(1000.0 * el / n_s, 4), "steps": n_s,
                         "temperature": temp, "top_p": top_p,
                         "fn": "AutoregressiveModel.sampleToken" if mode == q.hw.SAMPLE_TOKEN
                         else "AutoregressiveModel.of sample function"}
        log(f"[bench] decode with sampling ({name}, T={temp}, top_p={top_p}): {sampled[name]['ms_per_step']} ms/token, "
            f"{sampled[name]['tok_s']} tok/s")
    am.set_temperature(0.0)
    model.close()

    # ---- CPU baseline: the oracle (reference semantics) on this host, FP64 and FP32 ----------
    cpu = None
    parity = None
    if args.cpu_steps > 0:
        gpu_generated = np.concatenate([warm[0], toks[0]]).tolist()
        cpu, parity = cpu_baseline(cfg, prompt, args.seed, gpu_generated)
    out = {
        "metric": "decode tok/s (Qwen3-0.6B shape, b=1)",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        "config": {"workload": "C3: Qwen3-0.6B shape fp32 (d1024, 28L, 16Q/8KV, hd128, F3072, V151936), "
                               "batch 1, prompt 128, greedy decode",
                   "decode_positions": f"{pos0}..{pos0 + args.steps - 1}", "graph": not args.no_graph,
                   "persistent_kernel": persistent},
        "hbm": {"algorithmic_bytes_per_token": round(mean_bytes), "achieved_GBs": round(e2e_gbs, 1),
                "frac_of_peak": round(e2e_gbs / HBM_PEAK_GBS, 4)},
        "sampled_c3": sampled,
        "prompt_c3": {"tokens": n_prompt, "tok_s": round(n_prompt / prefill_s, 1), "ms": round(1000 * prefill_s, 3),
                      "tflop": round(pre_flops / 1e12, 4),
                      "achieved_tflops": round(pre_flops / prefill_s / 1e12, 2),
                      "mfma_f32_frac": round(pre_flops / prefill_s / 1e12 / MFMA_F32_PEAK_TFLOPS, 4),
                      "path": "batched prefill: fp32 MFMA GEMMs (v_mfma_f32_32x32x2_f32) + fp32 causal attention",
                      "by_steps_tok_s": round(n_prompt / by_steps_s, 1)},
        "c4": c4_section(args) if "c4" in sections and not args.no_c4 else None,
        "c5": c5_section(args) if "c5" in sections and not args.no_c5 else None,
        "c2": c2_section(args) if "c2" in sections and not args.no_c2 else None,
        "llama2": llama2_section(args) if "llama2" in sections and not args.no_llama2 else None,
        "roofline": roofline,
        "multi_launch": dict(multi or {}, roofline=roofline_multi, roofline_logits=roofline_logits),
        "kernels": kernels,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
