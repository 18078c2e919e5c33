"""Attention fused in the training step (js/src/fusion/attention.js fuseAttentionTraining),
checked on the CPU: every attention of config 5's step and of the reference's transformer
becomes one forward 'attention' node and three 'attention-grad' nodes (dQ, dK, dV) whose
shared body recomputes the scores and P from Q and K. The transformed graph must hold the
original graph's values node for node in float64, bit for bit (each new node's body is
the ops of the nodes it replaces, in their order: a dropped term, a wrong transpose or a
dS formed from P where the softmax backward reads the exponentials would change bits);
the fusion contract's own counts must not move when the option is off; and the perf
lowering must run each gradient's three parts as one launch of their joint kernel. The
GPU side (node-local judging of both lowerings, the trainer bit for bit the checked path)
is in test_gpu_train.py and test_gpu_step_slices.py."""
import numpy as np
import pytest

from oracle import interp


def _bundle(tool, tmp_path, req):
    import tcmi_bridge
    d = tmp_path / "sg"
    tool("step-graph", req, out=str(d))
    return tcmi_bridge.Bundle(d)


@pytest.mark.parametrize("req,attentions", [({"model": "transformer", "B": 1}, 4), ({"model": "transformer-ref"}, 2)])
def test_fused_attention_step_holds_the_original_values(tool, tmp_path, req, attentions):
    b = _bundle(tool, tmp_path, dict(req, attention=True))
    c = b.cases[0]
    inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
    with interp.blas_matmul():
        orig = interp.evaluate(c["graph"], inputs)
        fused = interp.evaluate(c["fused"], inputs)
    kinds = {}
    for i, n in enumerate(c["fused"]["nodes"]):
        o = c["origin"][i]
        if o is None or o < 0:
            continue
        kind = n["attrs"]["kind"] if n["op"] == "fused" else n["op"]
        kinds[kind] = kinds.get(kind, 0) + 1
        assert np.array_equal(np.asarray(fused[i]), np.asarray(orig[o]), equal_nan=True), (i, n["op"], kind)
    assert kinds.get("attention") == attentions and kinds.get("attention-grad") == 3 * attentions, kinds
    parts = sorted(n["attrs"]["part"] for n in c["fused"]["nodes"] if n["op"] == "fused" and n["attrs"]["kind"] == "attention-grad")
    assert parts == sorted(["dq", "dk", "dv"] * attentions)


def test_contract_counts_do_not_move_when_the_option_is_off(tool, tmp_path):
    """The reference transformer's fused step keeps its published 450 launches (one per
    fused node, measurements.json m4.fusion) without the option, and loses the score
    launches with it."""
    off = _bundle(tool, tmp_path / "off", {"model": "transformer-ref"}).cases[0]
    on = _bundle(tool, tmp_path / "on", {"model": "transformer-ref", "attention": True}).cases[0]
    assert off["launchesChecked"] == 450
    assert on["launchesChecked"] < off["launchesChecked"] and on["launchesFused"] < off["launchesFused"]
    assert not any(n["op"] == "fused" and n["attrs"]["kind"].startswith("attention") for n in off["fused"]["nodes"])


def test_each_gradient_runs_as_one_launch(tool):
    """Config 5's step with the option: its four attention gradients are four joint
    launches (dQ, dK, dV in one dispatch each), and the batch checker, from the launch
    records alone, accepts them (the three parts of one gradient, in order, on the same
    operands)."""
    res = tool("batch-check", {"models": [{"model": "transformer", "B": 64, "attention": True}]})
    assert res[0]["check"]["ok"], res[0]
    r = tool("perf-lower", {"model": "transformer", "B": 64, "attention": True})
    joint = [b for b in r["batches"] if b.get("joint")]
    assert len(joint) == 4 and all(b["count"] == 3 for b in joint), joint
