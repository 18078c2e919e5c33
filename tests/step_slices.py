"""Per-sequence blocks of a training step's launches, for node-local judging at the
full batch (tests/test_gpu_step_slices.py) and its CPU check (tests/test_step_slices.py).

A launch whose output carries the batch axis is evaluated for one sequence on that
sequence's blocks of its operands, with the block shapes of the same builder's
one-sequence graph (the twin) and the full graph's constants; a launch whose output
does not is evaluated whole."""
from typing import List, Sequence

import numpy as np

from oracle import bounds


def batch_axis(full_shape: Sequence[int], twin_shape: Sequence[int]) -> int:
    """The one dimension where the two shapes differ, or -1 where they are equal."""
    assert len(full_shape) == len(twin_shape)
    diff = [d for d in range(len(full_shape)) if full_shape[d] != twin_shape[d]]
    assert len(diff) <= 1, (full_shape, twin_shape)
    return diff[0] if diff else -1


def take_block(a: np.ndarray, shape: Sequence[int], p: int, q: int, b: int) -> np.ndarray:
    """Block b (of size q) along axis p of a flat row-major array of `shape`."""
    nd = np.asarray(a).reshape(shape)
    idx = [slice(None)] * len(shape)
    idx[p] = slice(b * q, (b + 1) * q)
    return np.ascontiguousarray(nd[tuple(idx)]).reshape(-1)


def twin_node(full, twin, node_id):
    """The full graph's node with the twin's shapes and the full graph's constants: body
    nodes keep their op, inputs, axes, permutations and constant values, and take the
    twin's shapes and shape attributes."""
    def merge(a, b):
        assert a["op"] == b["op"] and a["inputs"] == b["inputs"]
        attrs = dict(a["attrs"])
        if "shape" in b["attrs"]:
            attrs["shape"] = b["attrs"]["shape"]
        return dict(a, attrs=attrs, shape=b["shape"])

    n, t = full["nodes"][node_id], twin["nodes"][node_id]
    node = merge(n, t)
    if n["op"] == "fused":
        body = {"nodes": [merge(x, y) for x, y in zip(n["attrs"]["body"]["nodes"], t["attrs"]["body"]["nodes"])]}
        node["attrs"] = dict(node["attrs"], body=body)
    return node


def local(graph, node, operands: List[np.ndarray]):
    """(value, bound) of one launched node on its operand values (localReferenceFused,
    harness-m4.js:182-200)."""
    if node["op"] == "fused":
        g, out = node["attrs"]["body"], node["attrs"]["output"]
    else:
        g, out = bounds.one_op_graph(graph, node)
    r = bounds.reference_with_bounds(g, {f"a{k}": v for k, v in enumerate(operands)})
    return r["values"][out], r["bounds"][out]


def expectations(full, twin, launched, operand, sequences):
    """Yield (node id, sequence index or None, value, bound) for every launched node:
    per sequence where its output carries the batch axis, whole otherwise.
    `operand(i, s)` is node i's value: its block for sequence index s, or whole for None."""
    axis = [batch_axis(n["shape"], t["shape"]) for n, t in zip(full["nodes"], twin["nodes"])]
    for nid in launched:
        node = full["nodes"][nid]
        if axis[nid] >= 0:
            tn = twin_node(full, twin, nid)
            for s in range(len(sequences)):
                ops = [operand(i, s if axis[i] >= 0 else None) for i in node["inputs"]]
                v, e = local(twin, tn, ops)
                yield nid, s, v, e
        else:
            v, e = local(full, node, [operand(i, None) for i in node["inputs"]])
            yield nid, None, v, e
