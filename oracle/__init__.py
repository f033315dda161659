"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (oracle/qwen3_oracle_impl.h).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only as the checker or the CPU baseline; the product library never calls it.

``precision`` is "fp64" (the reference default, Hardware.java:684) or "fp32".
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle_qwen3.so")

_lib = None


class OracleCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn_dim", "vocab", "seq_len",
        "qk_norm_mode", "full_seq_mask", "tied", "reserved")] + [
        ("rope_theta", ctypes.c_double), ("eps", ctypes.c_double), ("qk_eps", ctypes.c_double)]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        assert _lib.oracle_cfg_size() == ctypes.sizeof(OracleCfg)
        for sfx in ("_f64", "_f32"):
            getattr(_lib, "oracle_model_create" + sfx).restype = ctypes.c_void_p
            getattr(_lib, "oracle_model_create" + sfx).argtypes = [ctypes.c_void_p]
            getattr(_lib, "oracle_model_destroy" + sfx).argtypes = [ctypes.c_void_p]
            getattr(_lib, "oracle_model_set_weight" + sfx).argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                                                      ctypes.c_void_p, ctypes.c_longlong]
            getattr(_lib, "oracle_model_step" + sfx).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
            getattr(_lib, "oracle_model_reset" + sfx).argtypes = [ctypes.c_void_p]
            getattr(_lib, "oracle_model_position" + sfx).argtypes = [ctypes.c_void_p]
            getattr(_lib, "oracle_model_hidden" + sfx).argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            for name in ("oracle_rope_flat", "oracle_attention", "oracle_attention_block"):
                fn = getattr(_lib, name + sfx)
                fn.restype = None
            getattr(_lib, "oracle_rope_flat" + sfx).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                               ctypes.c_int, ctypes.c_double]
            getattr(_lib, "oracle_rmsnorm" + sfx).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                             ctypes.c_int, ctypes.c_double]
            getattr(_lib, "oracle_rmsnorm_grouped" + sfx).argtypes = [
                ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_double]
            getattr(_lib, "oracle_rope_freqs" + sfx).argtypes = [ctypes.c_void_p, ctypes.c_double, ctypes.c_int,
                                                                ctypes.c_int]
    return _lib


def set_threads(n: int) -> int:
    lib().oracle_set_threads(int(n))
    return lib().oracle_get_threads()


def _dt(precision: str):
    if precision == "fp64":
        return np.float64, "_f64"
    if precision == "fp32":
        return np.float32, "_f32"
    raise ValueError(precision)


def _fn(name, precision):
    return getattr(lib(), name + _dt(precision)[1])


def _arr(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- operators ----------------------------------------------------------------------
def rmsnorm(x, w, eps=1e-6, precision="fp64", group=None):
    dt, _ = _dt(precision)
    x = _arr(x, dt)
    w = _arr(w, dt)
    out = np.empty_like(x)
    n = x.shape[-1]
    for r in range(x.size // n):
        xr, orow = x.reshape(-1, n)[r], out.reshape(-1, n)[r]
        if group:
            _fn("oracle_rmsnorm_grouped", precision)(orow.ctypes.data, xr.ctypes.data, w.ctypes.data, n, group, eps)
        else:
            _fn("oracle_rmsnorm", precision)(orow.ctypes.data, xr.ctypes.data, w.ctypes.data, n, ctypes.c_double(eps))
    return out


def dense(W, x, bias=None, precision="fp64"):
    dt, _ = _dt(precision)
    W = _arr(W, dt)
    x = _arr(x, dt)
    rows, cols = W.shape
    y = np.empty(rows, dtype=dt)
    b = _arr(bias, dt) if bias is not None else None
    _fn("oracle_dense", precision).argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_int]
    _fn("oracle_dense", precision)(y.ctypes.data, W.ctypes.data, x.ctypes.data, b.ctypes.data if b is not None else None,
                                   rows, cols)
    return y


def rope_freqs(theta, head_dim, seq_len, precision="fp64"):
    dt, _ = _dt(precision)
    out = np.empty((seq_len, head_dim // 2, 2), dtype=dt)
    _fn("oracle_rope_freqs", precision)(out.ctypes.data, ctypes.c_double(theta), head_dim, seq_len)
    return out


def split_half(x, heads, hd, precision="fp64"):
    dt, _ = _dt(precision)
    x = _arr(x, dt)
    out = np.empty(heads * hd, dtype=dt)
    _fn("oracle_split_half", precision).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    _fn("oracle_split_half", precision)(out.ctypes.data, x.ctypes.data, heads, hd)
    return out


def unsplit_half(x, heads, hd, precision="fp64"):
    dt, _ = _dt(precision)
    x = _arr(x, dt)
    out = np.empty(heads * hd, dtype=dt)
    _fn("oracle_unsplit_half", precision).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    _fn("oracle_unsplit_half", precision)(out.ctypes.data, x.ctypes.data, heads, hd)
    return out


def rope_rotate_split(x_split, heads, hd, freqs_at_pos, precision="fp64"):
    dt, _ = _dt(precision)
    x = _arr(x_split, dt).copy()
    f = _arr(freqs_at_pos, dt)
    _fn("oracle_rope_rotate_split", precision).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                            ctypes.c_void_p]
    _fn("oracle_rope_rotate_split", precision)(x.ctypes.data, heads, hd, f.ctypes.data)
    return x


def rope_flat(x, heads, hd, pos, theta, precision="fp64"):
    dt, _ = _dt(precision)
    x = _arr(x, dt).copy()
    rows = x.size // (heads * hd)
    for r in range(rows):
        xr = x.reshape(rows, -1)[r]
        _fn("oracle_rope_flat", precision)(xr.ctypes.data, heads, hd, pos, ctypes.c_double(theta))
    return x


def gqa_expand(x, kv_heads, heads, hd, precision="fp64"):
    dt, _ = _dt(precision)
    x = _arr(x, dt)
    out = np.empty(heads * hd, dtype=dt)
    _fn("oracle_gqa_expand", precision).argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 3
    _fn("oracle_gqa_expand", precision)(out.ctypes.data, x.ctypes.data, kv_heads, heads, hd)
    return out


def causal_mask(seq_len, pos, precision="fp64"):
    dt, _ = _dt(precision)
    out = np.empty(seq_len, dtype=dt)
    _fn("oracle_causal_mask", precision).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    _fn("oracle_causal_mask", precision)(out.ctypes.data, seq_len, pos)
    return out


def softmax(x, precision="fp64"):
    dt, _ = _dt(precision)
    x = _arr(x, dt).copy()
    n = x.shape[-1]
    _fn("oracle_softmax", precision).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    _fn("oracle_softmax", precision)(x.ctypes.data, x.size // n, n)
    return x


def attention(q, kc, vc, heads, kv_heads, hd, pos, seq_len, full_seq=False, precision="fp64"):
    """q (heads*hd) already normalised and rotated; caches (seq_len, kv_heads, hd)."""
    dt, _ = _dt(precision)
    q, kc, vc = _arr(q, dt), _arr(kc, dt), _arr(vc, dt)
    out = np.empty(heads * hd, dtype=dt)
    _fn("oracle_attention", precision).argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 6
    _fn("oracle_attention", precision)(out.ctypes.data, q.ctypes.data, kc.ctypes.data, vc.ctypes.data, heads,
                                       kv_heads, hd, pos, seq_len, int(full_seq))
    return out


def attention_block(q_raw, k_raw, v_raw, q_norm, k_norm, kc, vc, heads, kv_heads, hd, pos, theta, qk_eps=1e-6,
                    per_head_norm=False, full_seq=False, precision="fp64"):
    """QK-norm + RoPE + cache write at pos + attention.  kc / vc (seq, kv_heads, hd) are
    modified in place (they must already have the oracle's dtype)."""
    dt, _ = _dt(precision)
    assert kc.dtype == dt and vc.dtype == dt and kc.flags.c_contiguous and vc.flags.c_contiguous
    q_raw, k_raw, v_raw = _arr(q_raw, dt), _arr(k_raw, dt), _arr(v_raw, dt)
    qn = _arr(q_norm, dt) if q_norm is not None else None
    kn = _arr(k_norm, dt) if k_norm is not None else None
    out = np.empty(heads * hd, dtype=dt)
    fn = _fn("oracle_attention_block", precision)
    fn.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_int] * 5 + [ctypes.c_double, ctypes.c_double, ctypes.c_int,
                                                                ctypes.c_int]
    fn(out.ctypes.data, q_raw.ctypes.data, k_raw.ctypes.data, v_raw.ctypes.data,
       qn.ctypes.data if qn is not None else None, kn.ctypes.data if kn is not None else None,
       kc.ctypes.data, vc.ctypes.data, heads, kv_heads, hd, pos, kc.shape[0], theta, qk_eps, int(per_head_norm),
       int(full_seq))
    return out


def index_of_max(x, precision="fp64"):
    dt, _ = _dt(precision)
    x = _arr(x, dt)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(rows, dtype=np.int32)
    _fn("oracle_index_of_max", precision).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    _fn("oracle_index_of_max", precision)(x.ctypes.data, rows, n, out.ctypes.data)
    return out


# ---- whole model ---------------------------------------------------------------------
class OracleQwen3:
    """Reference-semantics CPU Qwen3 (one sequence).  ``cfg`` is a common_amd Qwen3Config."""

    def __init__(self, cfg, state_dict, precision="fp64", full_seq_mask=False):
        self.cfg = cfg
        self.precision = precision
        self.dt, self.sfx = _dt(precision)
        c = OracleCfg(cfg.dim, cfg.layer_count, cfg.head_count, cfg.kv_head_count, cfg.head_size, cfg.hidden_dim,
                      cfg.vocab_size, cfg.seq_len, cfg.qk_norm_mode, int(full_seq_mask), int(cfg.shared_weights), 0,
                      cfg.rope_theta, cfg.epsilon, cfg.epsilon)
        self.h = _fn("oracle_model_create", precision)(ctypes.byref(c))
        items = state_dict.items() if isinstance(state_dict, dict) else state_dict
        for k, v in items:
            v = np.ascontiguousarray(v, dtype=np.float32)
            rc = _fn("oracle_model_set_weight", precision)(self.h, k.encode(), v.ctypes.data, v.size)
            if rc != 0:
                raise KeyError(f"oracle rejected weight {k} (rc={rc})")

    def close(self):
        if self.h:
            _fn("oracle_model_destroy", self.precision)(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        _fn("oracle_model_reset", self.precision)(self.h)

    def step(self, token: int, want_logits: bool = True):
        logits = np.empty(self.cfg.vocab_size, dtype=self.dt) if want_logits else None
        nxt = _fn("oracle_model_step", self.precision)(self.h, int(token),
                                                        logits.ctypes.data if want_logits else None)
        if nxt < 0:
            raise RuntimeError("oracle step failed (position past capacity or bad token)")
        return nxt, logits

    def hidden(self):
        out = np.empty(self.cfg.dim, dtype=self.dt)
        _fn("oracle_model_hidden", self.precision)(self.h, out.ctypes.data)
        return out

    def prefill(self, tokens, want_logits: bool = True):
        """The prompt rows at once from the current position (oracle/qwen3_oracle_prefill.h): the
        same values as one step() per token, computed over all rows together.  Returns (greedy
        token after the last row, that row's logits)."""
        ids = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.empty(self.cfg.vocab_size, dtype=self.dt) if want_logits else None
        fn = _fn("oracle_model_prefill", self.precision)
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        nxt = fn(self.h, ids.ctypes.data, ids.size, logits.ctypes.data if want_logits else None)
        if nxt < 0:
            raise RuntimeError("oracle prefill failed (position past capacity, bad token or unsupported shape)")
        return nxt, logits

    def generate_prefilled(self, prompt, n_decode):
        """generate() with the prompt through prefill(): returns (tokens fed at each step past the
        prompt's last row, logits of the last prompt row and of every decode step)."""
        nxt, lg = self.prefill(prompt)
        fed, logits = [], [lg]
        for _ in range(n_decode):
            fed.append(nxt)
            nxt, lg = self.step(nxt)
            logits.append(lg)
        return np.array(fed, dtype=np.int32), np.stack(logits)

    def generate(self, prompt, n_decode, want_logits=True, sampler=None):
        """AutoregressiveModel semantics: returns (tokens fed at each step, logits per step).
        ``sampler(logits) -> token`` replaces the greedy choice past the prompt (it is called only
        there, as AutoregressiveModel.next applies its sample function, :295-308)."""
        fed, all_logits = [], []
        prev_next, prev_logits = None, None
        for s in range(len(prompt) + n_decode):
            if s < len(prompt):
                tok = int(prompt[s])
            else:
                tok = int(sampler(prev_logits)) if sampler is not None else prev_next
            prev_next, lg = self.step(tok, want_logits or sampler is not None)
            prev_logits = lg
            fed.append(tok)
            if want_logits:
                all_logits.append(lg)
        return np.array(fed, dtype=np.int32), (np.stack(all_logits) if want_logits else None)


# ---- token sampling (oracle/sample_oracle.c) ----------------------------------------
class JavaRandom:
    """java.util.Random(seed) state; draws advance it exactly as the Java class does."""

    def __init__(self, seed: int):
        lib().oracle_jrandom_seed.restype = ctypes.c_uint64
        lib().oracle_jrandom_seed.argtypes = [ctypes.c_int64]
        self.state = ctypes.c_uint64(lib().oracle_jrandom_seed(int(seed)))

    def next_int(self) -> int:
        lib().oracle_jrandom_next_int.restype = ctypes.c_int32
        lib().oracle_jrandom_next_int.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        return lib().oracle_jrandom_next_int(ctypes.byref(self.state))

    def next_double(self) -> float:
        lib().oracle_jrandom_next_double.restype = ctypes.c_double
        lib().oracle_jrandom_next_double.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        return lib().oracle_jrandom_next_double(ctypes.byref(self.state))


def _sample_call(name, values, args, rng):
    v = np.ascontiguousarray(values, dtype=np.float64)
    r, margin = ctypes.c_double(-1.0), ctypes.c_double(np.inf)
    fn = getattr(lib(), name)
    fn.restype = ctypes.c_int
    fn.argtypes = ([ctypes.c_void_p, ctypes.c_int] + [ctypes.c_double] * len(args) +
                   [ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)])
    k = fn(v.ctypes.data, v.size, *args, ctypes.byref(rng.state) if rng is not None else None, ctypes.byref(r),
           ctypes.byref(margin))
    return k, r.value, margin.value


def sample_token(values, temperature, top_p, rng: JavaRandom | None):
    """AutoregressiveModel.sampleToken (AutoregressiveModel.java:323-386).  Returns (index, r,
    margin): r is the uniform draw (-1 when greedy), margin its distance to the nearest boundary
    of the chosen index's cumulative interval."""
    return _sample_call("oracle_sample_token", values, (temperature, top_p), rng)


def model_sample(logits, temperature, rng: JavaRandom):
    """The sample function of AutoregressiveModel.of (AutoregressiveModel.java:413-425)."""
    return _sample_call("oracle_model_sample", logits, (temperature,), rng)


def softmax_ignore_zero(x):
    """DistributionFeatures.softmax(x, true) in FP64 (DistributionFeatures.java:129-141)."""
    x = np.ascontiguousarray(x, dtype=np.float64).copy()
    lib().oracle_softmax_ignore_zero.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib().oracle_softmax_ignore_zero(x.ctypes.data, x.size)
    return x
