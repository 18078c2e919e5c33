"""The reference's model-level GPU checks (src/gpu/harness-m4.js:225-330 and :383-392) on its
own transformer (V 16, T 64, d 64, H 4, L 2, ff 256 GELU, batch 4, Adam) at its four golden
runs (golden/spec-m3b.json golden-seed1..4, each 20 steps over its batch schedule):

  * teacher-forced (runTeacherForcedM4, :225-272): at every step t of every run, the
    parameters and Adam state of the float64 trajectory after step t - 1 (the oracle's
    trainCpu3b, pinned to torch in tests/test_golden_runs.py) and that step's batch go
    through the step graph; every launch of the fused step then reads those float32-rounded
    reference operands and is judged against its own float64 expectation within the
    float32 budget (node-local). The reference published 80/80 steps, worst 0.49999997,
    450 launches against 1308 unfused. Here both lowerings are judged: the checked one
    (one launch per fused node, as the reference's) and the perf lowering the trainer runs;
  * the fused forward pass at each run's initialisation on its first batch, node-locally
    (runForwardLocalM4, :275-306): LayerNorm, softmax, log-softmax and GELU-epilogue
    kernels the step's partition never forms. Published 4/4, worst 0.439, 48 launches
    against 212;
  * the trainer with Adam state (runConsistencyM4, :310-330): golden-seed1's first 3 steps
    through HipTrainer, parameters and Adam's moments and beta powers fed back on the
    device, equal to the checked path (runner.run, the host feeding every new value back)
    bit for bit: loss, every parameter and every state tensor. Published identical;
  * the sabotage rows (runSabotageM4's teacherForced and forward, :383-392): each of the
    reference's four kernel sabotages planted in this backend's kernels, run on the four
    forward passes and on golden-seed1's first two steps. The reference caught
    epilogue-before-bias and layernorm-tree-short in 4/4 forward passes and nothing else
    there; so must this backend.

The oracle's work per step (reference values with bounds, node-local expectations) runs in
a pool of forked workers, before and after the one GPU command per run."""
import json
import multiprocessing
import os
import sys
from concurrent.futures import ProcessPoolExecutor

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import bounds, trajectory
from step_slices import fused_values, judge_case

pytestmark = pytest.mark.gpu

META = json.loads((GOLDEN / "transformer_golden.json").read_text())
RUNS = META["golden"]
T = META["config"]["T"]
ROWS = META["synthetic"]["train"]

# What the pool's workers read: set in the parent before the pool forks.
_CTX = {}


def _pool():
    return ProcessPoolExecutor(max_workers=max(1, min(8, os.cpu_count() or 1)),
                               mp_context=multiprocessing.get_context("fork"))


def _numel(node):
    return int(np.prod(node["shape"])) if node["shape"] else 1


def _write_values(k):
    """Worker: value set k — the reference values of the graph on inputs k, carried to the
    fused graph's nodes — written as float32 at its place in the values file."""
    c = _CTX
    ref = bounds.reference_with_bounds(c["graph"], c["inputs"][k])
    vals = fused_values(c["fused"], c["origin"], ref["values"])
    out = np.memmap(c["file"], dtype=np.float32, mode="r+", offset=4 * k * c["per"], shape=(c["per"],))
    out[:] = np.concatenate([np.asarray(v, dtype=np.float64).reshape(-1) for v in vals]).astype(np.float32)
    out.flush()
    return k


def _judge(k):
    """Worker: value set k's GPU case judged node-locally, both lowerings."""
    import tcmi_bridge
    c = _CTX
    if c.get("bundle") is None:
        c["bundle"] = tcmi_bridge.Bundle(c["out"])
    g = c["bundle"]
    gc = g.cases[k]
    assert gc["set"] == k
    flat = np.memmap(c["file"], dtype=np.float32, mode="r", offset=4 * k * c["per"], shape=(c["per"],))
    vals, off = [], 0
    for node in c["fused"]["nodes"]:
        n = _numel(node)
        vals.append(np.asarray(flat[off: off + n], dtype=np.float64))
        off += n
    j, jp = judge_case(c["fused"], vals, gc, g.arr)
    slim = lambda r: None if r is None else {  # noqa: E731
        "pass": r["pass"], "worst": r["worst"], "unjudged": r["unjudged"], "unjudgeable": r["unjudgeable"],
        "elements": r["elements"], "byKind": r["byKind"], "first": r["first"]}
    return {"set": k, "canary": gc["canaryIntact"], "checked": slim(j), "perf": slim(jp)}


def _local_runs(tool, tmp_path, what, graph_req, inputs, gpu_req, sabotage=None, perf=True, chunk=5):
    """Value sets for `inputs` (one dict of raw inputs per set) on the graph of `graph_req`
    (step-graph or forward-graph), run on the GPU node-locally and judged, `chunk` sets per
    gpu-local command (a set of the reference transformer's step is 28 MB of operands and
    as much again of outputs; each chunk's files are removed once it is judged). Returns
    (graph case, per-set results)."""
    import shutil
    import tcmi_bridge
    sg = tmp_path / f"{what}-graph"
    tool(what, graph_req, out=str(sg))
    c = tcmi_bridge.Bundle(sg).cases[0]
    per = sum(_numel(n) for n in c["fused"]["nodes"])
    results = []
    for lo in range(0, len(inputs), chunk):
        part = inputs[lo: lo + chunk]
        file = tmp_path / f"{what}-values-{lo}.f32"
        np.memmap(file, dtype=np.float32, mode="w+", shape=(per * len(part),)).flush()
        out = tmp_path / f"{what}-{sabotage or 'honest'}-local-{lo}"
        _CTX.clear()
        _CTX.update(graph=c["graph"], fused=c["fused"], origin=c["origin"], inputs=part, file=str(file), per=per,
                    out=str(out), bundle=None)
        with _pool() as pool:
            list(pool.map(_write_values, range(len(part))))
        req = dict(gpu_req, valuesFile=str(file), sets=len(part), perf=perf)
        if sabotage:
            req["sabotage"] = sabotage
        print(f"gpu step: gpu-local {what} sets {lo}..{lo + len(part) - 1}, sabotage {sabotage}", flush=True)
        tool("gpu-local", req, out=str(out), timeout=900)
        with _pool() as pool:
            for r in pool.map(_judge, range(len(part))):
                r["set"] += lo
                results.append(r)
        file.unlink()
        shutil.rmtree(out)
    return c, results


def _batch(run, t):
    return trajectory.encode_batch([ROWS[i] for i in run["schedule"][t]], run["V"], T)


def _step_request(run):
    return {"model": "transformer-ref", "V": run["V"], "B": run["batch"], "seed": run["seed"]}


def _step_inputs(tool, tmp_path, run, steps):
    """The raw inputs of steps 0..steps-1 of a golden run, teacher-forced: the float64
    trajectory's parameters and state before each step, and the step's batch."""
    import tcmi_bridge
    d = tmp_path / "init"
    tool("step-graph", dict(_step_request(run), params64=True), out=str(d))
    c = tcmi_bridge.Bundle(d).cases[0]
    step = {k: c[k] for k in ("graph", "names", "stateNames", "outputs", "loss", "cotangent")}
    batches = [_batch(run, t) for t in range(steps)]
    tr = trajectory.train(step, c["params64"], c["state64"], batches[:-1])
    inputs = []
    for t in range(steps):
        feed = dict(c["params64"] if t == 0 else tr["params"][t - 1])
        feed.update(c["state64"] if t == 0 else tr["states"][t - 1])
        feed["x"], feed["y"] = batches[t]
        feed[c["cotangent"]] = [1.0]
        inputs.append(feed)
    return inputs


def _forward_inputs(tool, tmp_path):
    """The raw inputs of the four golden runs' forward passes at initialisation, on each
    run's first batch; and the forward graph's request."""
    import tcmi_bridge
    inputs = []
    for run in RUNS:
        d = tmp_path / f"fwd-init-{run['name']}"
        tool("forward-graph", dict(_step_request(run), params64=True), out=str(d))
        c = tcmi_bridge.Bundle(d).cases[0]
        feed = dict(c["params64"])
        feed["x"], feed["y"] = _batch(run, 0)
        inputs.append(feed)
    return inputs


def _summary(results, key):
    kinds = {}
    for r in results:
        for k, v in r[key]["byKind"].items():
            kinds[k] = max(kinds.get(k, 0.0), v["worst"])
    return {"passed": sum(1 for r in results if r[key]["pass"] and r["canary"]),
            "worst": max(r[key]["worst"] for r in results), "byKind": kinds}


@pytest.mark.parametrize("run", RUNS, ids=[r["name"] for r in RUNS])
def test_teacher_forced_node_local(tool, tmp_path, run):
    inputs = _step_inputs(tool, tmp_path, run, run["steps"])
    c, results = _local_runs(tool, tmp_path, "step-graph", _step_request(run), inputs, _step_request(run))
    checked, perf = _summary(results, "checked"), _summary(results, "perf")
    print(f"teacher-forced {run['name']}: checked lowering {checked['passed']}/{len(results)} steps, worst "
          f"{checked['worst']:.6g} by kind {checked['byKind']}; perf lowering {perf['passed']}/{len(results)}, "
          f"worst {perf['worst']:.6g}; {c['launchesChecked']} launches ({c['launchesFused']} in the perf lowering) "
          f"against {c['launchesUnfused']} unfused", file=sys.stderr)
    bad = [(r["set"], r["checked"]["first"], r["perf"]["first"]) for r in results
           if not (r["canary"] and r["checked"]["pass"] and r["perf"]["pass"])]
    assert not bad, bad
    assert len(results) == run["steps"] == 20
    # The reference's partition of its step: 450 launches, 1308 unfused (measurements.json m4).
    assert (c["launchesChecked"], c["launchesUnfused"]) == (450, 1308)


def test_forward_node_local(tool, tmp_path):
    inputs = _forward_inputs(tool, tmp_path)
    c, results = _local_runs(tool, tmp_path, "forward-graph", _step_request(RUNS[0]), inputs,
                             dict(_step_request(RUNS[0]), forward=True))
    checked, perf = _summary(results, "checked"), _summary(results, "perf")
    print(f"forward node-local: checked lowering {checked['passed']}/{len(results)}, worst {checked['worst']:.6g} "
          f"by kind {checked['byKind']}; perf lowering {perf['passed']}/{len(results)}, worst {perf['worst']:.6g}; "
          f"{c['launchesChecked']} launches ({c['launchesFused']} in the perf lowering) against "
          f"{c['launchesUnfused']} unfused", file=sys.stderr)
    bad = [(r["set"], r["checked"]["first"], r["perf"]["first"]) for r in results
           if not (r["canary"] and r["checked"]["pass"] and r["perf"]["pass"])]
    assert not bad, bad
    # The kernels the forward pass holds and the step's partition does not.
    assert set(checked["byKind"]) >= {"layernorm", "softmax", "log-softmax", "matmul-epilogue"}
    assert (c["launchesChecked"], c["launchesUnfused"]) == (48, 212)


# The reference's forward-pass sabotage row (measurements.json m4.gpu.sabotage[].checks.forward):
# passes caught by their values (its runLocal has no canaries), of 4.
FORWARD_CAUGHT = {"epilogue-before-bias": 4, "layernorm-tree-short": 4, "softmax-no-max": 0, "fused-bounds-off-by-one": 0}


@pytest.mark.parametrize("sabotage", list(FORWARD_CAUGHT))
def test_forward_sabotage_row(tool, tmp_path, sabotage):
    """Each kernel sabotage planted in the checked lowering of the four forward passes,
    judged node-locally. By values, as the reference counts, epilogue-before-bias and
    layernorm-tree-short must be caught in all four, as they were there. The off-by-one
    leaves every in-range value right, so its values pass; here the runner also carries
    canaries, which the reference's runLocal does not, and its write one past the end of
    the forward pass's fused elementwise output shows in all four. softmax-no-max is
    reported (the reference's scores are small, so no row overflows without the shift).
    Golden-seed1's first two teacher-forced steps under each, as in the reference's
    sabotage run, are reported beside it."""
    inputs = _forward_inputs(tool, tmp_path)
    _, results = _local_runs(tool, tmp_path, "forward-graph", _step_request(RUNS[0]), inputs,
                             dict(_step_request(RUNS[0]), forward=True), sabotage=sabotage, perf=False)
    by_values = [r["set"] for r in results if not r["checked"]["pass"]]
    by_canary = [r["set"] for r in results if not r["canary"]]
    step_inputs = _step_inputs(tool, tmp_path, RUNS[0], 2)
    _, steps = _local_runs(tool, tmp_path, "step-graph", _step_request(RUNS[0]), step_inputs, _step_request(RUNS[0]),
                           sabotage=sabotage, perf=False)
    step_values = [r["set"] for r in steps if not r["checked"]["pass"]]
    step_canary = [r["set"] for r in steps if not r["canary"]]
    print(f"sabotage {sabotage}: forward caught by values {len(by_values)}/4 (reference {FORWARD_CAUGHT[sabotage]}/4), "
          f"by canaries {len(by_canary)}/4; teacher-forced steps caught by values {len(step_values)}/2 (reference 0/2), "
          f"by canaries {len(step_canary)}/2; first {[r['checked']['first'] for r in results][:1]}", file=sys.stderr)
    if sabotage in ("epilogue-before-bias", "layernorm-tree-short"):
        assert len(by_values) == 4, [r["checked"]["first"] for r in results]
    if sabotage == "fused-bounds-off-by-one":
        assert not by_values and len(by_canary) == 4


def test_adam_trainer_consistency(tool):
    """Golden-seed1's first 3 steps on its schedule's batches: the fused trainer (perf
    lowering, parameters and Adam state fed back on the device) equal to the checked path
    bit for bit, eagerly and replayed as HIP graphs in the liveness arena."""
    run = RUNS[0]
    batches = [[ROWS[i] for i in run["schedule"][t]] for t in range(3)]
    for graph, arena in [(False, False), (True, True)]:
        r = tool("gpu-train", dict(_step_request(run), batches=batches, steps=3, consistency=True, consistencySteps=3,
                                   graph=graph, arena=arena))
        print(f"adam consistency (graph {graph}, arena {arena}): identical {r['identical']}, losses {r['losses']}",
              file=sys.stderr)
        assert r["identical"] is True
        # The first loss is the run's initial loss within the float32 budget's order.
        assert abs(r["losses"][0] - run["initLoss"]) < 1e-4 * run["initLoss"], r["losses"]
