"""The Java binding sources (common_amd/jni/: the HIP natives class, the SPI classes and the JNI
shim) are not compiled here (no JDK in the image).  These CPU checks keep them consistent with each
other and with the library: every Java native has exactly one JNIEXPORT function of the mangled
name and the matching arity, and every C-ABI function the shim calls is declared in include/*.h and
exported by libar_hip.so."""
import os
import re
import subprocess

from common_amd import _native
from common_amd import hardware as hw

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JNI = os.path.join(ROOT, "common_amd", "jni")
JAVA = os.path.join(JNI, "java", "org", "almostrealism", "hardware", "hip")
SHIM = os.path.join(JNI, "ar_hip_jni.c")


def _java_natives():
    text = open(os.path.join(JAVA, "HIP.java")).read()
    out = {}
    for m in re.finditer(r"static\s+native\s+[\w\[\]]+\s+(\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip()]
        assert m.group(1) not in out, f"overloaded native {m.group(1)} (JNI short names would clash)"
        out[m.group(1)] = len(params)
    return out


def _shim_functions():
    text = open(SHIM).read()
    out = {}
    for m in re.finditer(r"JNIEXPORT\s+\w+\s+JNICALL\s+HIP_CLASS\((\w+)\)\s*\(([^)]*)\)", text):
        params = [p for p in m.group(2).split(",") if p.strip()]
        assert m.group(1) not in out, f"two definitions of {m.group(1)}"
        out[m.group(1)] = len(params)
    return out


def test_every_native_has_one_jniexport_of_matching_arity():
    natives, shim = _java_natives(), _shim_functions()
    assert len(natives) >= 40
    assert sorted(natives) == sorted(shim)
    for name, n in natives.items():
        assert shim[name] == n + 2, (name, n, shim[name])  # JNIEnv *, jclass + the Java parameters


def test_shim_mangles_to_the_java_package():
    text = open(SHIM).read()
    assert "#define HIP_CLASS(name) Java_org_almostrealism_hardware_hip_HIP_##name" in text
    assert "package org.almostrealism.hardware.hip;" in open(os.path.join(JAVA, "HIP.java")).read()


def test_shim_calls_only_declared_and_exported_symbols():
    called = set(re.findall(r"\b(ar_hip_\w+)\s*\(", open(SHIM).read()))
    declared = set(hw.declared_symbols())
    assert called and called <= declared, sorted(called - declared)
    out = subprocess.run(["nm", "-D", "--defined-only", _native.HIP_LIB], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert called <= exported, sorted(called - exported)


def test_spi_classes_present_and_use_the_natives():
    for cls in ("HipDataContext", "HipComputeContext", "HipMemoryProvider", "HipMemory", "HipQwen3"):
        text = open(os.path.join(JAVA, cls + ".java")).read()
        assert f"class {cls}" in text, cls
        assert "Not compiled in this repository" in text, cls
    used = set()
    for f in os.listdir(JAVA):
        if f != "HIP.java":
            used |= set(re.findall(r"\bHIP\.(\w+)\s*\(", open(os.path.join(JAVA, f)).read()))
    natives = _java_natives()
    assert used <= set(natives), sorted(used - set(natives))


def test_memory_provider_maps_elements_to_fp32_bytes():
    """MemoryProvider sizes and offsets are elements; the provider multiplies by its number size (4)."""
    text = open(os.path.join(JAVA, "HipMemoryProvider.java")).read()
    assert "private long bytes(long elements) { return elements * numberSize; }" in text
    assert "HIP.alloc(ctx(), b)" in text and "long b = bytes(size);" in text
    assert "HIP.setMem(ctx(), mem.getContentPointer(), bytes(offset), source, srcOffset, length)" in text
    assert "if (numberSize != 4)" in text


def test_next_returns_one_token_per_sequence():
    text = open(SHIM).read()
    body = text[text.index("HIP_CLASS(qwen3Next)"):]
    body = body[:body.index("\n}\n")]
    assert "NewIntArray(env, h->max_batch)" in body
    assert "SetIntArrayRegion(env, out, 0, h->max_batch" in body
