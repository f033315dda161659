"""Decode-step profile tree in the reference's OperationProfileNode format (common_amd.profile).

CPU: the XML document has the shape java.beans.XMLDecoder reads for OperationProfileNode.load
(base/code/src/main/java/io/almostrealism/profile/OperationProfileNode.java:824-838): a java root
naming XMLDecoder, one OperationProfileNode object per node, its key / name set as string properties,
metricEntries (seconds, double) and metricCounts (int) as HashMaps, children as an ArrayList, nested
in the tree's order; totals add a node's own entries to its children's (:397-420).  No JDK is in the
image, so the document is checked against that structure, not loaded by XMLDecoder.
GPU: the tree of a small model has one node for the persistent launch (one launch per step) and
one per separate-launch class (one launch per layer per step), every timing positive, and the model
keeps its persistent setting."""
import dataclasses
import xml.etree.ElementTree as ET

import pytest

from common_amd import config as C
from common_amd import profile as prof
from common_amd import synthetic
from common_amd.qwen3 import Qwen3

NODE = "io.almostrealism.profile.OperationProfileNode"


def _props(obj):
    return {v.get("property"): v for v in obj.findall("void") if v.get("property")}


def _parse_node(obj):
    assert obj.tag == "object" and obj.get("class") == NODE
    p = _props(obj)
    out = {"key": p["key"].find("string").text, "name": p["name"].find("string").text, "children": []}
    for prop, tag, conv in (("metricEntries", "double", float), ("metricCounts", "int", int)):
        if prop in p:
            m = p[prop].find("object")
            assert m.get("class") == "java.util.HashMap"
            entries = {}
            for put in m.findall("void"):
                assert put.get("method") == "put"
                k, v = list(put)
                assert k.tag == "string" and v.tag == tag
                entries[k.text] = conv(v.text)
            out[prop] = entries
    if "children" in p:
        lst = p["children"].find("object")
        assert lst.get("class") == "java.util.ArrayList"
        for add in lst.findall("void"):
            assert add.get("method") == "add"
            (child,) = list(add)
            out["children"].append(_parse_node(child))
    return out


def test_xml_is_the_xmldecoder_form_of_the_tree():
    leaf1 = prof.node("dense o + residual", key="step.6", seconds=1.25e-4, count=28)
    leaf2 = prof.node("a <name> & more", key="k2", seconds=2.5e-5, count=3)
    mid = prof.node("separate launches per stage", key="separate_launches", children=[leaf1, leaf2])
    root = prof.node("decode: 1 steps per class", key="decode",
                     children=[prof.node("decode_persistent", seconds=5.5e-4, count=1), mid])
    doc = prof.to_xml(root)
    assert doc.startswith('<?xml version="1.0" encoding="UTF-8"?>')
    java = ET.fromstring(doc)
    assert java.tag == "java" and java.get("class") == "java.beans.XMLDecoder"
    (obj,) = list(java)
    back = _parse_node(obj)
    assert back == root  # every key, name, entry, count and child survives, in order
    assert back["children"][1]["children"][1]["name"] == "a <name> & more"
    assert prof.total_seconds(root) == pytest.approx(5.5e-4 + 1.25e-4 + 2.5e-5)
    assert prof.total_seconds(mid) == pytest.approx(1.5e-4)
    assert "metricEntries" not in back and "metricEntries" not in back["children"][1]
    lines = prof.summary(root).splitlines()
    assert len(lines) == 5 and lines[3].startswith("    dense o + residual: 0.125 ms (28 launches)")


@pytest.mark.gpu
def test_decode_profile_tree_of_a_small_model(ctx, tmp_path):
    cfg = dataclasses.replace(C.C1_TINY, seq_len=160)
    sd = synthetic.state_dict(cfg, seed=5)
    prompt = synthetic.prompt_ids(8, cfg.vocab_size, seed=6)
    steps = 4
    with Qwen3(cfg, sd, ctx) as m:
        am = m.model
        am.reset()
        am.set_prompt(prompt)
        am.prefill()
        was = am.persistent
        tree = prof.decode_profile(am, steps, name="C1 decode")
        assert am.persistent == was
        tokens = am.run(2)  # the model still steps after the probes
        assert tokens.shape == (1, 2)
    kids = tree["children"]
    if was:
        per = kids[0]
        assert per["key"] == "decode_persistent" and sum(per["metricCounts"].values()) == steps
        assert sum(per["metricEntries"].values()) > 0
        kids = kids[1:]
    (sep,) = kids
    assert [c["name"] for c in sep["children"]] == [label for _, label, _ in prof.STEP_CLASSES]
    for c in sep["children"]:
        n = sum(c["metricCounts"].values())
        expect = steps if c["key"] == f"step.{prof.STEP_CLASSES[-1][0]}" else steps * cfg.layer_count
        assert n == expect, (c["name"], n)
        assert sum(c["metricEntries"].values()) > 0
    path = tmp_path / "profile.xml"
    prof.save(tree, str(path))
    assert _parse_node(list(ET.parse(path).getroot())[0]) == tree
