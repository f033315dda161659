"""Builds the native libraries in-tree (common_amd/lib/), for gfx950 only.

  libar_hip.so    HIP kernels + C-ABI (hipcc, --offload-arch=gfx950) + host-only C++ (g++)
  libar_synth.so  seeded synthetic-input generator (gcc, host only)

Every HIP translation unit is compiled with packed-FP32 instructions disabled.
Run: python -m common_amd.build
"""
from __future__ import annotations

import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "lib", "obj")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n  " + " ".join(cmd) + "\n" + r.stdout)
    return r.stdout


def build_synth():
    src = os.path.join(CSRC, "synth", "ar_synth.c")
    out = os.path.join(LIB, "libar_synth.so")
    _run(["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-std=c11", "-o", out + ".tmp", src, "-lm"])
    os.replace(out + ".tmp", out)
    return out


def build_hip(jobs: int = 8, trace: bool = False):
    """libar_hip.so; trace=True builds the diagnostic variant with the persistent decode kernel's stage
    timeline (-DAR_PK_TRACE) into lib/trace/ (load it with AR_HIP_LIB=<that path>)."""
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    obj_dir = os.path.join(OBJ, "trace") if trace else OBJ
    lib_dir = os.path.join(LIB, "trace") if trace else LIB
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(lib_dir, exist_ok=True)
    extra = ["-DAR_PK_TRACE"] if trace else []

    def compile_one(src):
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        _run([HIPCC, *HIP_FLAGS, *extra, "-I", os.path.join(HERE, "..", "include"), "-c", src, "-o", obj])
        return obj

    def compile_host(src):
        # host-only C++ (no device code): the host compiler, as its own objects in the library
        obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
        _run(["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-I", os.path.join(HERE, "..", "include"), "-c", src,
              "-o", obj])
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
        objs += list(ex.map(compile_host, sorted(glob.glob(os.path.join(CSRC, "*.cpp")))))
    out = os.path.join(lib_dir, "libar_hip.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out + ".tmp", *objs, "-L/opt/rocm/lib",
          "-lrocblas"])
    os.replace(out + ".tmp", out)
    return out


def build(jobs: int = 8):
    os.makedirs(LIB, exist_ok=True)
    if shutil.which("gcc") is None:
        raise RuntimeError("gcc not found")
    paths = [build_synth(), build_hip(jobs)]
    return paths


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if a != "--trace"]
    jobs = int(args[0]) if args else 8
    if "--trace" in sys.argv[1:]:
        print("built", build_hip(jobs, trace=True))
    else:
        for p in build(jobs):
            print("built", p)
