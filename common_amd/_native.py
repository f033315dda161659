"""Locates and loads the native libraries built in-tree by ``common_amd.build``.

The HIP backend library is required: there is no CPU fallback for the product path, so a
missing library raises instead of silently degrading.
"""
from __future__ import annotations

import ctypes
import os

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
# AR_HIP_LIB names another build of the backend library (the stage-trace build, lib/trace/libar_hip.so)
HIP_LIB = os.environ.get("AR_HIP_LIB") or os.path.join(LIB_DIR, "libar_hip.so")
SYNTH_LIB = os.path.join(LIB_DIR, "libar_synth.so")

_cache = {}


class NativeLibraryMissing(RuntimeError):
    pass


def _load(path: str, what: str):
    if path in _cache:
        return _cache[path]
    if not os.path.exists(path):
        raise NativeLibraryMissing(
            f"{what} not built: {path} is missing. Run `python -c 'import __graft_entry__ as g; g.build()'` "
            f"or `python -m common_amd.build` first.")
    lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    _cache[path] = lib
    return lib


def load_synth():
    return _load(SYNTH_LIB, "synthetic-input library")


def load_hip():
    return _load(HIP_LIB, "HIP backend library")
