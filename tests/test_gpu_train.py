"""GPU parity of the training steps (benchmark configs 1 and 5, and the reference's own
transformer) through the fused trainer: node-local judging of every launch of the fused
step on the float32-rounded reference operands (the reference's teacher-forced check,
harness-m4.js:182-223 and :225-272), the first step's loss and new parameters against the
composed float32 budget, and the trainer's device-side feedback against the checked path
bit for bit (harness-m4.js:310-330)."""
import json
import pathlib
import sys

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import bounds
from step_slices import fused_values, judge_case

pytestmark = pytest.mark.gpu


def node_local(tool, tmp_path, req):
    import tcmi_bridge
    sg = tmp_path / "sg"
    tool("step-graph", req, out=str(sg))
    b = tcmi_bridge.Bundle(sg)
    c = b.cases[0]
    inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
    ref = bounds.reference_with_bounds(c["graph"], inputs)
    fused_vals = fused_values(c["fused"], c["origin"], ref["values"])
    np.concatenate([v.astype(np.float32) for v in fused_vals]).tofile(tmp_path / "values.f32")
    out = tmp_path / "local"
    print(f"gpu step: gpu-local {req}", flush=True)
    tool("gpu-local", dict(req, valuesFile=str(tmp_path / "values.f32")), out=str(out), timeout=600)
    g = tcmi_bridge.Bundle(out)
    gc = g.cases[0]
    assert gc["canaryIntact"]
    j, jp = judge_case(c["fused"], fused_vals, gc, g.arr)
    print(f"{req['model']}: node-local worst {j['worst']:.3g} over {j['elements']} elements, "
          f"unjudgeable {j['unjudgeable']}, by kind {j['byKind']}", file=sys.stderr)
    assert j["pass"], (j["first"], j["unjudged"])
    # The perf lowering: every node it launches (all but the shared reshapes, the
    # transposes its matmuls read in place, the broadcasts its consumers read through
    # their index maps, and the dead nodes no kept value depends on), on the same
    # reference operands.
    print(f"{req['model']}: perf lowering node-local worst {jp['worst']:.3g} over {jp['elements']} elements, "
          f"{jp['skipped']} nodes shared or folded, {jp['chains']} chains with their reductions", file=sys.stderr)
    assert jp["pass"], (jp["first"], jp["unjudged"])
    return j


def test_c1_step_node_local(tool, tmp_path):
    node_local(tool, tmp_path, {"model": "mlp"})


@pytest.mark.parametrize("attention", [False, True])
def test_reference_transformer_step_node_local(tool, tmp_path, attention):
    """With `attention`, each attention and its gradient fused (fusion/attention.js): the
    forward attention kernel and the gradient's dQ, dK and dV kernels (checked lowering),
    and the gradient's joint kernel (perf lowering), judged like every other launch."""
    meta = json.loads((GOLDEN / "transformer_init.json").read_text())
    j = node_local(tool, tmp_path, {"model": "transformer-ref", "V": meta["V"], "B": meta["batch"], "seed": meta["seed"],
                                    "firstBatch": meta["firstBatch"], "attention": attention})
    assert set(j["byKind"]) >= {"plain", "elementwise", "matmul-epilogue", "rowwise"}
    if attention:
        assert set(j["byKind"]) >= {"attention", "attention-grad"}, j["byKind"]


@pytest.mark.parametrize("attention", [False, True])
def test_c5_structure_step_node_local(tool, tmp_path, attention):
    """Config 5's full structure (V 96, d 256, H 4, L 4, ff 1024 ReLU, T 128) at batch 1;
    with `attention`, each attention and its gradient fused (fusion/attention.js)."""
    j = node_local(tool, tmp_path, {"model": "transformer", "B": 1, "attention": attention})
    if attention:
        assert j["byKind"]["attention"]["nodes"] == 4 and j["byKind"]["attention-grad"]["nodes"] == 12, j["byKind"]


@pytest.mark.parametrize("graph,arena", [(False, False), (False, True), (True, True)])
def test_c1_first_step_against_composed_budget(tool, graph, arena):
    """Step 0 of the fused trainer: loss and every new parameter within the composed budget
    of the whole step graph (inputs float32-rounded, bounds propagated node by node). With
    `arena`, the step's intermediate buffers share one allocation by live range; with
    `graph`, the step is the replay of a captured HIP graph."""
    import tcmi_bridge
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        tool("step-graph", {"model": "mlp"}, out=d)
        b = tcmi_bridge.Bundle(d)
        c = b.cases[0]
        inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
    r = tool("gpu-train", {"model": "mlp", "steps": 1, "returnParams": True, "graph": graph, "arena": arena})
    assert (r["arena"] is not None) == arena
    ref = bounds.reference_with_bounds(c["graph"], inputs)
    ids = [c["loss"]] + [c["outputs"][k] for k in r["params"]]
    gpu = [np.array([r["losses"][0]])] + [np.asarray(r["params"][k]) for k in r["params"]]
    j = bounds.judge_outputs([ref["values"][i] for i in ids], [ref["bounds"][i] for i in ids], gpu)
    assert j["pass"], j["first"]


# Capturing config 5's step over three streams ended the node process with a segmentation
# fault inside the runtime (config 1's captured and replayed correctly). The cause is not
# known, so capture of multi-stream programs is switched off (Program.capture refuses it).
MULTI_STREAM_CAPTURE_OFF = "multi-stream capture is switched off: capturing config 5's step over three streams segfaulted"


@pytest.mark.parametrize("graph,arena,streams", [(False, False, 1), (True, False, 1), (False, True, 1), (False, False, 3),
                                                 (True, False, 3)])
def test_c1_trainer_consistency_and_learning(tool, graph, arena, streams):
    """20 fused-trainer steps on one batch: each equals the checked path (runner.run of the
    plain lowering, one launch per node, with the new values fed back by the host) bit for
    bit — the trainer runs the perf lowering, whose matmuls read transposed operands in
    place — and the loss falls at every step. With `graph`, each step is the replay of a
    captured HIP graph (two graphs, the parameters' buffers exchanging roles), and every
    replay is checked against the eager path, with the host's synchronisation between.
    With `arena`, the step's intermediate buffers share one allocation by live range; with
    `streams`, independent launches run on several streams (eagerly: a program issued
    over several streams is not captured)."""
    if graph and streams > 1:
        pytest.skip(MULTI_STREAM_CAPTURE_OFF)
    r = tool("gpu-train", {"model": "mlp", "steps": 20, "consistency": True, "consistencySteps": 20, "sameBatch": True,
                           "graph": graph, "arena": arena, "streams": streams})
    assert r["identical"] is True
    assert (r["arena"] is not None) == arena
    losses = r["losses"]
    assert all(np.isfinite(losses))
    # Plain SGD at lr 0.1 on one batch: every step lowers the loss, by 0.2 over the 20.
    assert all(b < a for a, b in zip(losses, losses[1:])), losses
    assert losses[-1] < losses[0] - 0.2, losses


@pytest.mark.parametrize("graph,arena,streams,attention", [(False, False, 1, False), (True, False, 1, False),
                                                           (False, True, 1, False), (True, True, 1, False),
                                                           (False, False, 3, False), (True, False, 3, False),
                                                           (False, False, 1, True), (True, False, 1, True),
                                                           (False, True, 1, True), (True, True, 1, True)])
def test_c5_full_size_trainer(tool, graph, arena, streams, attention):
    """Config 5 at full size (B 64): the fused trainer's first 3 steps (perf lowering:
    transposes read in place by their matmuls, reshapes sharing buffers, identical
    independent launches batched into one dispatch) equal the checked path (plain
    lowering) bit for bit, and the initial loss is near ln(96) (small initial weights,
    uniform tokens). With `arena`, every buffer but the parameters, batch, loss and logits
    is placed by live range in one allocation (2.3 GB of node buffers in 0.9 GB), the
    members of a batch at one position, and the steps are still bit for bit the checked
    path's; so they are with the step's independent launches on three streams (each
    batch member then launched by itself). With `attention`, each attention and its
    gradient fused (fusion/attention.js): the trainer runs each gradient's dQ, dK and dV
    as one launch of their joint kernel, the checked path as three kernels, and the
    steps are still the same bits."""
    if graph and streams > 1:
        pytest.skip(MULTI_STREAM_CAPTURE_OFF)
    r = tool("gpu-train", {"model": "transformer", "B": 64, "steps": 3, "consistency": True, "consistencySteps": 3,
                           "graph": graph, "arena": arena, "streams": streams, "attention": attention}, timeout=600)
    assert r["identical"] is True
    assert r["folded"] > 0 and r["aliases"] > 0 and r["launches"] < r["checkedLaunches"]
    assert abs(r["losses"][0] - np.log(96)) < 0.1, r["losses"]
    assert r["batches"] >= 12, r["batches"]
    assert r["dispatches"] == (r["kernels"] - r["batchSaves"] if streams == 1 else r["kernels"]), r
    if arena:
        # With attention fused no [.., T, T] score tensor has a buffer: 1.0 GB of node
        # buffers instead of 1.3 GB, placed in 0.76 GB (what is left is mostly live at once).
        share = 0.78 if attention else 0.65
        assert r["arena"]["bytes"] < share * r["arena"]["unshared"] and r["arena"]["bytes"] < 0.85e9, r["arena"]
