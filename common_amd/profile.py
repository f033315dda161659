"""Decode-step profile tree in the reference's profile format.

The reference records per-operation timings in a tree of OperationProfileNode objects
(base/code/src/main/java/io/almostrealism/profile/OperationProfileNode.java:188-460), installed on
the model by Qwen3.java:189-190 and written with java.beans.XMLEncoder (OperationProfileNode.save,
:767-778; OperationProfileNode.load reads it back with XMLDecoder, :824-838).  A node's own time is
its TimingMetric: `metricEntries` maps an entry name to accumulated seconds and `metricCounts` to
the number of recordings (OperationProfile.setMetricEntries / setMetricCounts,
base/code/src/main/java/io/almostrealism/profile/OperationProfile.java:182-212); a parent's total is
its own entries plus its children's totals.

Here the nodes are the decode step's kernel classes, timed by the library's launch-timing hook (each
class's launches carry start / stop HIP events recorded by their own dispatches,
ar_hip_qwen3_kernel_timing / ar_hip_qwen3_kernel_time): under the root, one node for the
persistent launch (every layer, the final norm, the logits and the greedy keys of a step) when the
model runs it, and one node per class of the same step as separate launches (the projections with
their fused norms and epilogues, attention with its split combine, the logits GEMV with argmax).
`to_xml` writes the tree in the XMLDecoder form OperationProfileNode.load reads: each node an
OperationProfileNode built by its no-argument constructor, then its key, name, metric entries and
counts and children set through the bean setters.
"""
from __future__ import annotations

import json
from xml.sax.saxutils import escape

from . import qwen3 as q

# The separate-launch step's classes, in step order: (class, node name, the reference features the
# class covers)
STEP_CLASSES = (
    (q.KT_QKV, "rmsnorm + dense qkv", "AttentionFeatures.java:830, 839, 868, 885"),
    (q.KT_ATTENTION, "qk-norm + rope + attention", "AttentionFeatures.java:842-921"),
    (q.KT_O, "dense o + residual", "AttentionFeatures.java:922"),
    (q.KT_GATE_UP, "rmsnorm + dense gate/up + swiglu", "FeedForwardFeatures.java:147-156"),
    (q.KT_DOWN, "dense down + residual", "FeedForwardFeatures.java:147-156"),
    (q.KT_LOGITS, "rmsnorm + logits + indexOfMax", "Qwen3.java:401-405, AggregationFeatures.java:111-121"),
)


def node(name: str, key: str | None = None, seconds: float | None = None, count: int | None = None,
         children: list | None = None) -> dict:
    """One profile node: its own metric (one entry under its name) when seconds is given."""
    n = {"key": key if key is not None else name, "name": name, "children": list(children or [])}
    if seconds is not None:
        n["metricEntries"] = {name: float(seconds)}
        n["metricCounts"] = {name: int(count or 0)}
    return n


def total_seconds(n: dict) -> float:
    """Self plus children, as OperationProfileNode.getTotalDuration adds them (:397-420)."""
    return sum(n.get("metricEntries", {}).values()) + sum(total_seconds(c) for c in n["children"])


def _time_class(am, which: int, steps: int) -> tuple[float, int]:
    am.kernel_timing(which)
    try:
        am.run(steps)
        ms, launches = am.kernel_time()
    finally:
        am.kernel_timing(q.KT_NONE)
    return ms / 1000.0, launches


def decode_profile(am, steps: int, name: str = "decode") -> dict:
    """Times `steps` decode steps per kernel class of model `am` (an AutoregressiveModel of
    common_amd.qwen3) and returns the tree.  Every class is timed over its own steps, so the model
    advances by steps x (1 + 6) positions when it runs the persistent step, steps x 6 otherwise; the
    caller leaves room for them in the cache.  The persistent setting is restored afterwards."""
    if steps < 1:
        raise ValueError("steps must be >= 1")
    children = []
    was_persistent = am.persistent
    try:
        if was_persistent:
            s, n = _time_class(am, q.KT_LAYERS, steps)
            children.append(node("decode_persistent (layers + final norm + logits + argmax keys)",
                                 key="decode_persistent", seconds=s, count=n))
            am.use_persistent(False)
        layer_nodes = []
        for which, label, _ in STEP_CLASSES:
            s, n = _time_class(am, which, steps)
            layer_nodes.append(node(label, key=f"step.{which}", seconds=s, count=n))
        children.append(node("separate launches per stage", key="separate_launches", children=layer_nodes))
    finally:
        if was_persistent:
            am.use_persistent(True)
    return node(f"{name}: {steps} steps per class", key=name, children=children)


def _value_xml(v, indent: str) -> str:
    if isinstance(v, bool):
        return f"{indent}<boolean>{'true' if v else 'false'}</boolean>\n"
    if isinstance(v, int):
        return f"{indent}<int>{v}</int>\n"
    if isinstance(v, float):
        return f"{indent}<double>{repr(v)}</double>\n"
    return f"{indent}<string>{escape(str(v))}</string>\n"


def _map_xml(prop: str, m: dict, indent: str) -> str:
    out = f'{indent}<void property="{prop}">\n{indent} <object class="java.util.HashMap">\n'
    for k, v in m.items():
        out += f'{indent}  <void method="put">\n' + _value_xml(str(k), indent + "   ") + _value_xml(v, indent + "   ")
        out += f"{indent}  </void>\n"
    return out + f"{indent} </object>\n{indent}</void>\n"


def _node_xml(n: dict, indent: str) -> str:
    out = f'{indent}<object class="io.almostrealism.profile.OperationProfileNode">\n'
    i2 = indent + " "
    for prop in ("key", "name"):
        if n.get(prop) is not None:
            out += f'{i2}<void property="{prop}">\n' + _value_xml(str(n[prop]), i2 + " ") + f"{i2}</void>\n"
    if "metricEntries" in n:
        out += _map_xml("metricEntries", {k: float(v) for k, v in n["metricEntries"].items()}, i2)
        out += _map_xml("metricCounts", {k: int(v) for k, v in n["metricCounts"].items()}, i2)
    if n["children"]:
        out += f'{i2}<void property="children">\n{i2} <object class="java.util.ArrayList">\n'
        for c in n["children"]:
            out += f'{i2}  <void method="add">\n' + _node_xml(c, i2 + "   ") + f"{i2}  </void>\n"
        out += f"{i2} </object>\n{i2}</void>\n"
    return out + f"{indent}</object>\n"


def to_xml(tree: dict) -> str:
    """The tree as the XMLDecoder document OperationProfileNode.load reads."""
    return ('<?xml version="1.0" encoding="UTF-8"?>\n<java version="17" class="java.beans.XMLDecoder">\n'
            + _node_xml(tree, " ") + "</java>\n")


def save(tree: dict, path: str) -> None:
    """Writes the XML form to `path` (and nothing else)."""
    with open(path, "w") as f:
        f.write(to_xml(tree))


def summary(tree: dict, indent: str = "") -> str:
    """Indented lines of name, total seconds and counts, like OperationProfileNode.summary's listing."""
    counts = sum(tree.get("metricCounts", {}).values())
    line = f"{indent}{tree['name']}: {1e3 * total_seconds(tree):.3f} ms" + (f" ({counts} launches)" if counts else "")
    return "\n".join([line] + [summary(c, indent + "  ") for c in tree["children"]])


def to_json(tree: dict) -> str:
    return json.dumps(tree)
