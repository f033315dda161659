"""ctypes binding of the HIP backend's context, memory provider and operators.

Python stand-ins for the reference's backend SPI objects
(base/code/src/main/java/io/almostrealism/code/DataContext.java:81-88,
ComputeContext.java:89,133, MemoryProvider.java:60-188), written as a JNI bridge would
bind the same C-ABI (include/ar_hip.h).  Every call goes to the native library: there
is no Python or CPU fallback, and a missing library raises ``NativeLibraryMissing``.
"""
from __future__ import annotations

import ctypes
import glob
import os
import re

import numpy as np

from . import _native

AR_HIP_OK = 0
AR_HIP_ERR_INVALID = 1
AR_HIP_ERR_HIP = 2
AR_HIP_ERR_NO_DEVICE = 3
AR_HIP_ERR_STATE = 4
AR_HIP_ERR_NOT_FOUND = 5

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_F64 = 3

GEMM_STORE, GEMM_RESIDUAL, GEMM_SWIGLU = 0, 1, 2
SAMPLE_MODEL, SAMPLE_TOKEN = 0, 1  # AutoregressiveModel.of's sample function / AutoregressiveModel.sampleToken

_c_void_pp = ctypes.POINTER(ctypes.c_void_p)
_c_int_p = ctypes.POINTER(ctypes.c_int)
_c_float_p = ctypes.c_void_p
_SIGS = {
    "ar_hip_last_error": (ctypes.c_char_p, []),
    "ar_hip_version": (ctypes.c_char_p, []),
    "ar_hip_device_count": (ctypes.c_int, [_c_int_p]),
    "ar_hip_init": (ctypes.c_int, [ctypes.c_int, _c_void_pp]),
    "ar_hip_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_device_info": (ctypes.c_int, [ctypes.c_void_p, _c_int_p, ctypes.POINTER(ctypes.c_size_t),
                                          ctypes.c_char_p, ctypes.c_int]),
    "ar_hip_alloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, _c_void_pp]),
    "ar_hip_free": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_host_alloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, _c_void_pp]),
    "ar_hip_host_free": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_memcpy_h2d": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "ar_hip_memcpy_d2h": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "ar_hip_memcpy_d2d": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "ar_hip_memset": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]),
    "ar_hip_allocated_bytes": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]),
    "ar_hip_rmsnorm": (ctypes.c_int, [ctypes.c_void_p, _c_float_p, _c_float_p, _c_float_p, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_float]),
    "ar_hip_dense": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, _c_float_p, _c_float_p,
                                    _c_float_p, ctypes.c_float, _c_float_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int]),
    "ar_hip_swiglu": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, _c_float_p,
                                     _c_float_p, ctypes.c_float, _c_float_p, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int]),
    "ar_hip_rope": (ctypes.c_int, [ctypes.c_void_p, _c_float_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_double, ctypes.c_int]),
    "ar_hip_index_of_max": (ctypes.c_int, [ctypes.c_void_p, _c_float_p, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_void_p]),
    "ar_hip_attention_decode": (ctypes.c_int, [ctypes.c_void_p, _c_float_p, _c_float_p, _c_float_p, _c_float_p,
                                               _c_float_p, ctypes.c_float, ctypes.c_int, _c_float_p, _c_float_p,
                                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_double, _c_float_p]),
    "ar_hip_attention_decode_noalloc": (ctypes.c_int, [ctypes.c_void_p, _c_float_p, _c_float_p, _c_float_p,
                                                       _c_float_p, _c_float_p, ctypes.c_float, ctypes.c_int,
                                                       _c_float_p, _c_float_p, ctypes.c_int, ctypes.c_int,
                                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                                       _c_float_p]),
    "ar_hip_qwen3_create": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _c_void_pp]),
    "ar_hip_qwen3_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_qwen3_set_weight": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int,
                                               ctypes.c_int64]),
    "ar_hip_qwen3_finalize": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_qwen3_reset": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_qwen3_set_prompt": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]),
    "ar_hip_qwen3_next": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_qwen3_run": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]),
    "ar_hip_qwen3_position": (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    "ar_hip_qwen3_hidden": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_qwen3_kernel_timing": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "ar_hip_qwen3_kernel_time": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_double), _c_int_p]),
    "ar_hip_qwen3_kernel_loop": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
    "ar_hip_qwen3_use_graph": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "ar_hip_qwen3_use_fragment_gemv": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "ar_hip_qwen3_fragment_gemv": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]),
    "ar_hip_qwen3_use_persistent": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "ar_hip_qwen3_prefill_gemm": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "ar_hip_qwen3_prefill_gemm_backend": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]),
    "ar_hip_qwen3_persistent": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]),
    "ar_hip_qwen3_persistent_recomputed": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]),
    "ar_hip_qwen3_persistent_wait_limit": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint]),
    "ar_hip_pointer_checks": (ctypes.c_int, [ctypes.POINTER(ctypes.c_ulonglong)]),
    "ar_hip_qwen3_prefill": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_qwen3_prefill_by_steps": (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    "ar_hip_gemm_bf16": (ctypes.c_int, [ctypes.c_void_p] + [ctypes.c_void_p] * 6 + [ctypes.c_int] * 4),
    "ar_hip_gemm_f32": (ctypes.c_int, [ctypes.c_void_p] + [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4),
    "ar_hip_sample": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_double, ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_qwen3_set_sampling": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_double, ctypes.c_double,
                                                 ctypes.c_void_p]),
    # include/ar_tokenizer.h
    "ar_hip_tokenizer_load": (ctypes.c_int, [ctypes.c_char_p, _c_void_pp]),
    "ar_hip_tokenizer_from_vocab": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                                   _c_void_pp]),
    "ar_hip_tokenizer_load_merges": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p]),
    "ar_hip_tokenizer_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_tokenizer_vocab_size": (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    "ar_hip_tokenizer_merge_count": (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    "ar_hip_tokenizer_token": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), _c_int_p,
                                              ctypes.POINTER(ctypes.c_float)]),
    "ar_hip_tokenizer_encode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_void_p, ctypes.c_int, _c_int_p]),
    "ar_hip_tokenizer_decode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                               ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    "ar_hip_tokenizer_pretokenize": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                                    _c_int_p]),
    # include/ar_state_dict.h
    "ar_hip_state_dict_open": (ctypes.c_int, [ctypes.c_char_p, _c_void_pp]),
    "ar_hip_state_dict_create": (ctypes.c_int, [_c_void_pp]),
    "ar_hip_state_dict_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_state_dict_size": (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    "ar_hip_state_dict_key": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]),
    "ar_hip_state_dict_contains": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, _c_int_p]),
    "ar_hip_state_dict_files": (ctypes.c_int, [ctypes.c_void_p, _c_int_p, _c_int_p]),
    "ar_hip_state_dict_info": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, _c_int_p,
                                              ctypes.POINTER(ctypes.c_int32), _c_int_p, _c_int_p,
                                              ctypes.POINTER(ctypes.c_int64)]),
    "ar_hip_state_dict_read": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p,
                                              ctypes.c_int64]),
    "ar_hip_state_dict_put": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32),
                                             ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                             ctypes.c_int64]),
    "ar_hip_state_dict_save": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int]),
    "ar_hip_qwen3_infer_config": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_qwen3_load_state_dict": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    # include/ar_llama2.h
    "ar_hip_llama2_parse_config": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_void_p]),
    "ar_hip_llama2_open": (ctypes.c_int, [ctypes.c_char_p, _c_void_pp]),
    "ar_hip_llama2_close": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_llama2_config": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "ar_hip_llama2_tensor": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                            ctypes.POINTER(ctypes.c_int64)]),
    "ar_hip_llama2_create_model": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                  ctypes.c_int, _c_void_pp]),
    "ar_hip_bpe_load": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, _c_void_pp]),
    "ar_hip_bpe_create": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, _c_void_pp]),
    "ar_hip_bpe_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "ar_hip_bpe_vocab_size": (ctypes.c_int, [ctypes.c_void_p, _c_int_p]),
    "ar_hip_bpe_token": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), _c_int_p,
                                        ctypes.POINTER(ctypes.c_float)]),
    "ar_hip_bpe_lookup": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int, _c_int_p]),
    "ar_hip_bpe_encode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_int, _c_int_p]),
}


class HardwareException(RuntimeError):
    """Raised for a non-zero C-ABI status (the reference's HardwareException)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[ar_hip error {code}] {message}")
        self.code = code


def lib():
    L = _native.load_hip()
    if not getattr(L, "_ar_typed", False):
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        L._ar_typed = True
    return L


def check(code: int):
    if code != AR_HIP_OK:
        raise HardwareException(code, lib().ar_hip_last_error().decode(errors="replace"))


def declared_symbols(header: str | None = None) -> list[str]:
    """Names of every function the C-ABI headers (include/*.h, or one given header) declare."""
    if header is None:
        inc = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
        headers = sorted(glob.glob(os.path.join(inc, "*.h")))
    else:
        headers = [header]
    names = set()
    for h in headers:
        text = open(h).read()
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ar_hip_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def device_count() -> int:
    n = ctypes.c_int(0)
    rc = lib().ar_hip_device_count(ctypes.byref(n))
    return n.value if rc == AR_HIP_OK else 0


class DeviceBuffer:
    """A device allocation owned by a HipMemoryProvider (HipMemory in the JNI mapping)."""

    def __init__(self, ctx: "HipContext", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().ar_hip_alloc(ctx.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, ctx: "HipContext", a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(ctx, max(a.nbytes, 16))
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        check(lib().ar_hip_memcpy_h2d(self.ctx.handle, self.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        check(lib().ar_hip_memcpy_d2h(self.ctx.handle, out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def zero(self):
        check(lib().ar_hip_memset(self.ctx.handle, self.ptr, 0, self.nbytes))

    def free(self):
        if self.ptr is not None:
            check(lib().ar_hip_free(self.ctx.handle, self.ptr))
            self.ptr = None


class HipContext:
    """One GPU: data context + compute context (one in-order stream) + memory provider."""

    def __init__(self, device: int | None = None):
        """device None: the device AR_HIP_DEVICE names (default 0)."""
        h = ctypes.c_void_p()
        check(lib().ar_hip_init(-1 if device is None else device, ctypes.byref(h)))
        self.handle = h.value
        self.device = device

    def close(self):
        if self.handle:
            check(lib().ar_hip_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def synchronize(self):
        check(lib().ar_hip_synchronize(self.handle))

    def info(self):
        cus = ctypes.c_int()
        hbm = ctypes.c_size_t()
        name = ctypes.create_string_buffer(64)
        check(lib().ar_hip_device_info(self.handle, ctypes.byref(cus), ctypes.byref(hbm), name, 64))
        return {"num_cus": cus.value, "hbm_bytes": hbm.value, "arch": name.value.decode()}

    def allocated_bytes(self) -> int:
        v = ctypes.c_size_t()
        check(lib().ar_hip_allocated_bytes(self.handle, ctypes.byref(v)))
        return v.value

    # memory provider --------------------------------------------------------------
    def allocate(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        return DeviceBuffer.from_array(self, a)

    def copy(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int):
        """Device-to-device copy on the context's stream."""
        check(lib().ar_hip_memcpy_d2d(self.handle, dst.ptr, src.ptr, nbytes))

    # operators (see include/ar_hip.h for the reference each mirrors) ----------------
    def rmsnorm(self, x: DeviceBuffer, w: DeviceBuffer, y: DeviceBuffer, rows: int, n: int, eps: float):
        check(lib().ar_hip_rmsnorm(self.handle, x.ptr, w.ptr, y.ptr, rows, n, eps))

    def dense(self, W: DeviceBuffer, w_dtype: int, x: DeviceBuffer, y: DeviceBuffer, rows: int, cols: int,
              batch: int = 1, bias: DeviceBuffer | None = None, norm_w: DeviceBuffer | None = None,
              eps: float = 1e-6):
        check(lib().ar_hip_dense(self.handle, W.ptr, w_dtype, bias.ptr if bias else None, x.ptr,
                                 norm_w.ptr if norm_w else None, eps, y.ptr, rows, cols, batch))

    def swiglu(self, Wg: DeviceBuffer, Wu: DeviceBuffer, w_dtype: int, x: DeviceBuffer, y: DeviceBuffer,
               rows: int, cols: int, batch: int = 1, norm_w: DeviceBuffer | None = None, eps: float = 1e-6):
        check(lib().ar_hip_swiglu(self.handle, Wg.ptr, Wu.ptr, w_dtype, x.ptr, norm_w.ptr if norm_w else None,
                                  eps, y.ptr, rows, cols, batch))

    def rope(self, x: DeviceBuffer, heads: int, head_dim: int, pos: int, theta: float, rows: int = 1):
        check(lib().ar_hip_rope(self.handle, x.ptr, heads, head_dim, pos, theta, rows))

    def index_of_max(self, x: DeviceBuffer, rows: int, n: int, out: DeviceBuffer):
        check(lib().ar_hip_index_of_max(self.handle, x.ptr, rows, n, out.ptr))

    def sample(self, logits: DeviceBuffer, rows: int, n: int, mode: int, temperature: float, top_p: float,
               rng_state: DeviceBuffer | None, out: DeviceBuffer):
        """One draw per row (ar_hip_sample): rng_state holds rows java.util.Random states (u64)."""
        check(lib().ar_hip_sample(self.handle, logits.ptr, rows, n, mode, temperature, top_p,
                                  rng_state.ptr if rng_state else None, out.ptr))

    def gemm_bf16(self, A: DeviceBuffer, W: DeviceBuffer, M: int, N: int, K: int, epilogue: int = GEMM_STORE,
                  W2: DeviceBuffer | None = None, bias: DeviceBuffer | None = None, C: DeviceBuffer | None = None,
                  O: DeviceBuffer | None = None):
        check(lib().ar_hip_gemm_bf16(self.handle, A.ptr, W.ptr, W2.ptr if W2 else None, bias.ptr if bias else None,
                                     C.ptr if C else None, O.ptr if O else None, M, N, K, epilogue))

    def gemm_f32(self, A: DeviceBuffer, W: DeviceBuffer, M: int, N: int, K: int, epilogue: int = GEMM_STORE,
                 W2: DeviceBuffer | None = None, bias: DeviceBuffer | None = None, C: DeviceBuffer | None = None):
        check(lib().ar_hip_gemm_f32(self.handle, A.ptr, W.ptr, W2.ptr if W2 else None, bias.ptr if bias else None,
                                    C.ptr if C else None, M, N, K, epilogue))

    def attention_decode(self, q, k, v, q_norm, k_norm, qk_eps, qk_norm_mode, k_cache, v_cache, max_seq, pos,
                         heads, kv_heads, head_dim, theta, out, noalloc: bool = False):
        """ar_hip_attention_decode, or with ``noalloc`` ar_hip_attention_decode_noalloc (partials in the
        library's fixed per-device scratch array instead of memory it allocates)."""
        fn = lib().ar_hip_attention_decode_noalloc if noalloc else lib().ar_hip_attention_decode
        check(fn(self.handle, q.ptr, k.ptr, v.ptr, q_norm.ptr if q_norm else None, k_norm.ptr if k_norm else None,
                 qk_eps, qk_norm_mode, k_cache.ptr, v_cache.ptr, max_seq, pos, heads, kv_heads, head_dim, theta,
                 out.ptr))


def java_random_state(seed: int) -> int:
    """The 48-bit state of java.util.Random(seed): (seed ^ 0x5DEECE66D) mod 2^48."""
    return (int(seed) ^ 0x5DEECE66D) & ((1 << 48) - 1)
