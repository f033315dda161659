"""Protobuf weight I/O (include/ar_state_dict.h) against the protobuf runtime.

The checker is Google's protobuf library (the ``protobuf`` Python package), given the
reference's schema (engine/ml/src/main/proto/collections.proto:1-27) as a descriptor built
here: files it serializes must read back exactly, files the native writer produces must parse
with it and equal its own serialization of the same message byte for byte.  The loading rules
follow StateDictionary.loadWeights (engine/ml/.../ml/StateDictionary.java:119-150) and
CollectionEncoder / CollectionDataMemory (engine/ml/.../persist/assets/); the value pattern
of test_reference_collection_round_trip is CollectionDataMemoryProviderTest's (1 + 0.25 i,
96 values; FP64 exact, FP32 within 1e-6).  No GPU is used.
"""
import dataclasses
import os

import numpy as np
import pytest

from common_amd import hardware as hw
from common_amd import synthetic
from common_amd.config import C1_TINY
from common_amd.state_dict import DTYPE_F64, StateDictionary, save_split

pb = pytest.importorskip("google.protobuf")
from google.protobuf import descriptor_pb2, descriptor_pool, message_factory  # noqa: E402

F32 = hw.DTYPE_F32


def _schema(packed: bool = True, extra_fields: bool = False):
    """Message classes for collections.proto (proto3).  packed=False gives the one-key-per-value
    encoding of repeated scalars; extra_fields adds fields the reference schema does not have."""
    FD = descriptor_pb2.FieldDescriptorProto
    pkg = f"almostrealism_t{int(packed)}{int(extra_fields)}"
    fdp = descriptor_pb2.FileDescriptorProto(name=pkg + ".proto", package=pkg, syntax="proto3")

    def field(msg, name, number, ftype, label=FD.LABEL_OPTIONAL, type_name=None):
        f = msg.field.add(name=name, number=number, type=ftype, label=label)
        if type_name:
            f.type_name = f".{pkg}.{type_name}"
        if label == FD.LABEL_REPEATED and ftype in (FD.TYPE_INT32, FD.TYPE_DOUBLE, FD.TYPE_FLOAT) and not packed:
            f.options.packed = False
        return f

    tp = fdp.message_type.add(name="TraversalPolicyData")
    field(tp, "dims", 1, FD.TYPE_INT32, FD.LABEL_REPEATED)
    field(tp, "traversal_axis", 2, FD.TYPE_INT32)
    cd = fdp.message_type.add(name="CollectionData")
    field(cd, "traversal_policy", 1, FD.TYPE_MESSAGE, type_name="TraversalPolicyData")
    field(cd, "data", 2, FD.TYPE_DOUBLE, FD.LABEL_REPEATED)
    field(cd, "data_32", 3, FD.TYPE_FLOAT, FD.LABEL_REPEATED)
    if extra_fields:
        field(cd, "note", 7, FD.TYPE_STRING)
        field(cd, "scale", 8, FD.TYPE_FIXED64)
        field(tp, "stride", 5, FD.TYPE_INT64, FD.LABEL_REPEATED)
    en = fdp.message_type.add(name="CollectionLibraryEntry")
    field(en, "key", 1, FD.TYPE_STRING)
    field(en, "collection", 2, FD.TYPE_MESSAGE, type_name="CollectionData")
    if extra_fields:
        field(en, "version", 9, FD.TYPE_FIXED32)
    lib = fdp.message_type.add(name="CollectionLibraryData")
    field(lib, "collections", 1, FD.TYPE_MESSAGE, FD.LABEL_REPEATED, type_name="CollectionLibraryEntry")
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fdp)
    return {m: message_factory.GetMessageClass(pool.FindMessageTypeByName(f"{pkg}.{m}"))
            for m in ("TraversalPolicyData", "CollectionData", "CollectionLibraryEntry", "CollectionLibraryData")}


def _library(S, tensors, precision=F32, axes=None):
    lib = S["CollectionLibraryData"]()
    for key, arr in tensors.items():
        e = lib.collections.add()
        e.key = key
        e.collection.traversal_policy.dims.extend(int(d) for d in arr.shape)
        e.collection.traversal_policy.traversal_axis = (axes or {}).get(key, 0)
        if precision == DTYPE_F64:
            e.collection.data.extend(np.asarray(arr, np.float64).ravel().tolist())
        else:
            e.collection.data_32.extend(np.asarray(arr, np.float32).ravel().tolist())
    return lib


def _tensors(seed=0):
    rng = np.random.default_rng(seed)
    return {
        "model.embed_tokens.weight": rng.standard_normal((37, 16)).astype(np.float32),
        "model.layers.0.self_attn.q_norm.weight": (1 + 0.02 * rng.standard_normal((4, 8))).astype(np.float32),
        "scalarish": np.array([3.5], np.float32),
        "three.d": rng.standard_normal((2, 3, 5)).astype(np.float32),
        "big": rng.standard_normal(70_000).astype(np.float32),  # a multi-byte length prefix
    }


@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("precision", [F32, DTYPE_F64])
def test_reads_what_the_protobuf_runtime_writes(tmp_path, packed, precision):
    S = _schema(packed)
    t = _tensors()
    axes = {"three.d": 2, "scalarish": 0}
    p = tmp_path / "weights"
    p.write_bytes(_library(S, t, precision, axes).SerializeToString())
    with StateDictionary(p) as sd:
        assert sorted(sd.keySet()) == sorted(t)
        assert sd.size() == len(t) and sd.files() == (1, 0)
        for k, v in t.items():
            shape, ax, stored, n = sd.info(k)
            assert shape == v.shape and n == v.size and ax == axes.get(k, 0)
            assert stored == precision
            np.testing.assert_array_equal(sd.get(k), v)
            np.testing.assert_array_equal(sd.get(k, np.float64), v.astype(np.float64))


def test_unknown_fields_are_skipped(tmp_path):
    S = _schema(extra_fields=True)
    lib = _library(S, _tensors())
    for e in lib.collections:
        e.version = 7
        e.collection.note = "from a newer writer"
        e.collection.scale = 123456789
        e.collection.traversal_policy.stride.extend([1, -5, 1 << 40])
    p = tmp_path / "w"
    p.write_bytes(lib.SerializeToString())
    with StateDictionary(p) as sd:
        for k, v in _tensors().items():
            np.testing.assert_array_equal(sd.get(k), v)


@pytest.mark.parametrize("precision", [F32, DTYPE_F64])
def test_writer_output_is_the_runtime_serialization(tmp_path, precision):
    S = _schema()
    t = _tensors(1)
    axes = {"three.d": 1}
    with StateDictionary() as sd:
        for k, v in t.items():
            sd.put(k, v, traversal_axis=axes.get(k, 0))
        sd.save(tmp_path / "out", precision)
    raw = (tmp_path / "out").read_bytes()
    lib = S["CollectionLibraryData"]()
    lib.ParseFromString(raw)
    got = {e.key: e for e in lib.collections}
    assert sorted(got) == sorted(t)
    for k, v in t.items():
        c = got[k].collection
        assert list(c.traversal_policy.dims) == list(v.shape)
        assert c.traversal_policy.traversal_axis == axes.get(k, 0)
        vals = np.array(c.data if precision == DTYPE_F64 else c.data_32)
        assert (len(c.data), len(c.data_32)) == ((v.size, 0) if precision == DTYPE_F64 else (0, v.size))
        np.testing.assert_array_equal(vals, v.ravel())
    # entries are written in key order: the runtime's own encoding of the same message is identical
    ordered = {k: t[k] for k in sorted(t)}
    assert raw == _library(S, ordered, precision, axes).SerializeToString()


@pytest.mark.parametrize("precision", [DTYPE_F64, F32])
def test_reference_collection_round_trip(tmp_path, precision):
    # CollectionDataMemoryProviderTest.deferredHostReadsMatchSource: 1 + 0.25 i, i < 96
    src = 1.0 + 0.25 * np.arange(96, dtype=np.float64)
    with StateDictionary({"c": src}) as sd:
        sd.save(tmp_path / "c", precision)
    with StateDictionary(tmp_path / "c") as sd:
        got = sd.get("c", np.float64)
        assert sd.info("c")[2] == precision
    tol = 0.0 if precision == DTYPE_F64 else 1e-6
    assert np.abs(got - src).max() <= tol


def test_data_takes_precedence_over_data_32(tmp_path):
    # CollectionDataMemory.java:51,73: the double list wins when it is non-empty
    S = _schema()
    lib = S["CollectionLibraryData"]()
    e = lib.collections.add()
    e.key = "both"
    e.collection.traversal_policy.dims.extend([3])
    e.collection.data.extend([1.0, 2.0, 3.0])
    e.collection.data_32.extend([9.0, 9.0, 9.0])
    (tmp_path / "f").write_bytes(lib.SerializeToString())
    with StateDictionary(tmp_path / "f") as sd:
        assert sd.info("both")[2] == DTYPE_F64
        np.testing.assert_array_equal(sd.get("both"), [1.0, 2.0, 3.0])


def test_directory_rules(tmp_path, capfd):
    S = _schema()

    def write(name, tensors):
        (tmp_path / name).write_bytes(_library(S, tensors).SerializeToString())

    one = np.ones((2, 2), np.float32)
    write("embeddings", {"model.embed_tokens.weight": one, "dup": one})
    write("layer_00", {"model.layers.0.x": 2 * one, "dup": 3 * one})       # later name replaces "dup"
    write(".hidden", {"secret": one})                                      # names starting with '.' are skipped
    (tmp_path / "tokenizer.bin").write_bytes(b"\x0a\xff\xff\xff\x0f\x00")  # not a message: skipped whole
    lib = _library(S, {"good": one, "bad": one, "after": one})
    bad = lib.collections[1].collection
    bad.traversal_policy.dims[:] = [3, 2]                                  # 4 values for a shape of 6
    empty = lib.collections.add()
    empty.key = "no_dims"
    (tmp_path / "layer_01").write_bytes(lib.SerializeToString())
    (tmp_path / "subdir").mkdir()
    with StateDictionary(tmp_path) as sd:
        keys = set(sd.keySet())
        assert keys == {"model.embed_tokens.weight", "dup", "model.layers.0.x", "good"}
        np.testing.assert_array_equal(sd.get("dup"), 3 * one)
        assert sd.get("secret") is None and not sd.containsKey("after")
        assert sd.files() == (2, 2)
    err = capfd.readouterr().err
    assert "tokenizer.bin" in err and "layer_01" in err


def test_entry_without_dimensions_is_dropped(tmp_path):
    S = _schema()
    lib = _library(S, {"a": np.ones(3, np.float32)})
    e = lib.collections.add()
    e.key = "shapeless"
    e.collection.data_32.extend([])
    (tmp_path / "f").write_bytes(lib.SerializeToString())
    with StateDictionary(tmp_path / "f") as sd:
        assert sd.keySet() == ["a"] and sd.files() == (1, 0)


def test_errors():
    with pytest.raises(hw.HardwareException) as e:
        StateDictionary("/nonexistent/weights")
    assert e.value.code == hw.AR_HIP_ERR_NOT_FOUND
    with StateDictionary() as sd:
        with pytest.raises(hw.HardwareException) as e:
            sd.info("missing")
        assert e.value.code == hw.AR_HIP_ERR_NOT_FOUND
        assert sd.get("missing") is None
        L = hw.lib()
        import ctypes
        dims = (ctypes.c_int32 * 2)(2, 3)
        buf = np.zeros(5, np.float32)
        assert L.ar_hip_state_dict_put(sd.handle, b"k", dims, 2, 0, buf.ctypes.data, F32, 5) == hw.AR_HIP_ERR_INVALID
        assert b"shape" in L.ar_hip_last_error()
        assert L.ar_hip_state_dict_save(sd.handle, b"/tmp/x", 7) == hw.AR_HIP_ERR_INVALID
        # a shape whose element count overflows 64 bits matches no value count
        big = (ctypes.c_int32 * 3)(2 ** 31 - 1, 2 ** 31 - 1, 2 ** 31 - 1)
        assert L.ar_hip_state_dict_put(sd.handle, b"k", big, 3, 0, buf.ctypes.data, F32, 5) == hw.AR_HIP_ERR_INVALID


def test_overflowing_shape_in_a_file_is_a_parse_error(tmp_path, capfd):
    """An entry whose dims multiply past 64 bits is a parse error (the file's later entries are
    skipped with a warning, as for any undecodable entry), not a wrapped size that matches."""
    S = _schema()
    lib = _library(S, {"ok": np.ones(2, np.float32)})
    e = lib.collections.add()
    e.key = "huge"
    e.collection.traversal_policy.dims.extend([2 ** 31 - 1] * 3)
    e.collection.data_32.extend([1.0] * 5)
    (tmp_path / "f").write_bytes(lib.SerializeToString())
    with StateDictionary(tmp_path / "f") as sd:
        assert sd.keySet() == ["ok"]


def test_qwen3_layout_round_trip_and_config_inference(tmp_path):
    cfg = C1_TINY
    weights = synthetic.state_dict(cfg, seed=3)
    paths = save_split(weights, tmp_path)
    names = sorted(os.path.basename(p) for p in paths)
    assert names == ["embeddings"] + [f"layer_{i:02d}" for i in range(cfg.layer_count)]
    with StateDictionary(tmp_path) as sd:
        assert sorted(sd.keySet()) == sorted(weights)
        for k, v in weights.items():
            np.testing.assert_array_equal(sd.get(k), v)
        inferred = sd.infer_config()
    # Qwen3.inferConfigFromWeights: seqLen 131072, theta 1e6, shared weights without lm_head
    assert inferred == dataclasses.replace(cfg, seq_len=131072)


def test_config_inference_errors_follow_the_reference():
    with StateDictionary({"x": np.ones(2, np.float32)}) as sd:
        with pytest.raises(hw.HardwareException, match="embed_tokens"):
            sd.infer_config()
    with StateDictionary({"model.embed_tokens.weight": np.ones((8, 4), np.float32)}) as sd:
        with pytest.raises(hw.HardwareException, match="QK-Norm"):
            sd.infer_config()
