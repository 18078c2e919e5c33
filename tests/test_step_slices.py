"""The per-sequence blocks that judge config 5's step at its full batch on the GPU
(tests/test_gpu_step_slices.py), checked on the CPU at B = 2 against the whole launches:
for every launch of the fused step whose output carries the batch axis, the oracle's
value and bound on one sequence's operand blocks, with the one-sequence twin's shapes
and the full graph's constants, equal that sequence's block of the value and bound of
the whole launch, bit for bit. A block taken along the wrong axis, a constant taken
from the twin (the loss scale 1/(B*T)), or a launch whose rows depended on another
sequence would break the equality."""
import numpy as np

from oracle import bounds, interp
from step_slices import batch_axis, expectations, local, take_block


def test_sequence_blocks_equal_the_whole_launch(tmp_path, tool):
    import tcmi_bridge
    B = 2
    tool("step-graph", {"model": "transformer", "B": B}, out=str(tmp_path / "full"))
    tool("step-graph", {"model": "transformer", "B": 1}, out=str(tmp_path / "twin"))
    fb, tb = tcmi_bridge.Bundle(tmp_path / "full"), tcmi_bridge.Bundle(tmp_path / "twin")
    c = fb.cases[0]
    full, twin = c["fused"], tb.cases[0]["fused"]
    inputs = {k: fb.arr(v) for k, v in c["inputs"].items()}
    with interp.blas_matmul():
        ref = bounds.reference_with_bounds(c["graph"], inputs)
    # The operands: float32 values of every fused node, as a GPU run would give them.
    vals = [ref["values"][o].astype(np.float32) for o in c["origin"]]
    del ref
    nodes, tnodes = full["nodes"], twin["nodes"]
    axis = [batch_axis(n["shape"], t["shape"]) for n, t in zip(nodes, tnodes)]
    launched = [i for i, n in enumerate(nodes) if n["op"] not in ("input", "const")]
    seqs = list(range(B))

    def operand(i, s):
        if s is None:
            return vals[i]
        return take_block(vals[i], nodes[i]["shape"], axis[i], tnodes[i]["shape"][axis[i]], s)

    whole = {}
    blocked = 0
    scales = set()
    for nid, s, v, e in expectations(full, twin, launched, operand, seqs):
        if s is None:
            continue
        if nid not in whole:
            whole[nid] = local(full, nodes[nid], [vals[i] for i in nodes[nid]["inputs"]])
        wv, we = whole[nid]
        q = tnodes[nid]["shape"][axis[nid]]
        assert np.array_equal(v, take_block(wv, nodes[nid]["shape"], axis[nid], q, s), equal_nan=True), (nid, s)
        assert np.array_equal(e, take_block(we, nodes[nid]["shape"], axis[nid], q, s), equal_nan=True), (nid, s)
        blocked += 1
        if nodes[nid]["op"] == "fused":
            for x in nodes[nid]["attrs"]["body"]["nodes"]:
                if x["op"] == "const" and isinstance(x["attrs"].get("value"), (int, float)):
                    scales.add(x["attrs"]["value"])
    assert blocked >= 2 * 300, blocked
    # The step's mean over B*T positions reaches some per-sequence launch as a constant.
    assert any(abs(v * B * 128 - 1) < 1e-12 or abs(v - B * 128) < 1e-9 for v in scales), sorted(scales)[:20]
    # The launches judged whole do not carry the batch, and some read operands that do.
    wholes = [i for i in launched if axis[i] < 0]
    assert wholes and any(axis[j] >= 0 for i in wholes for j in nodes[i]["inputs"])
