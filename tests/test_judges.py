"""The two judges every full-size GPU verdict goes through, pinned by planted errors:
judge_outputs (src/fusion/workloads.js:351-374, the kept outputs of configs 2-4 and
the trainers' first steps) and judge_local (src/gpu/harness-m4.js:202-223, node by
node over a fused graph). Each planted mistake is one the judge must catch: a value
just outside the 2E budget (and one just inside it that must pass), NaN, a wrong value
in the last element of the last output or node, a fused node and a plain node, a
missing or short GPU array, and an unjudgeable fraction just above the 1% rule (and one
just below it that must pass)."""
import numpy as np
import pytest

from oracle import bounds


def _g(nodes):
    return {"nodes": nodes}


def _in(name, shape):
    return {"op": "input", "inputs": [], "attrs": {"name": name, "shape": shape}, "shape": shape}


def _node(op, inputs, out_shape, **attrs):
    return {"op": op, "inputs": inputs, "attrs": attrs, "shape": out_shape}


def _three_outputs():
    """exp(x), x * y and x / y over 64 elements: three kept outputs with non-zero bounds."""
    n = 64
    g = _g([_in("x", [n]), _in("y", [n]), _node("exp", [0], [n]), _node("mul", [0, 1], [n]), _node("div", [0, 1], [n])])
    rng = np.random.default_rng(7)
    r = bounds.reference_with_bounds(g, {"x": rng.normal(size=n), "y": rng.uniform(1, 2, size=n)})
    ids = [2, 3, 4]
    vals, bnds = [r["values"][i] for i in ids], [r["bounds"][i] for i in ids]
    assert all(np.all(b > 0) for b in bnds)
    return vals, bnds


def test_judge_outputs_budget_edges_and_nan():
    vals, bnds = _three_outputs()
    exact = [v.astype(np.float32) for v in vals]
    assert bounds.judge_outputs(vals, bnds, exact)["pass"]
    for k in range(3):
        for i in (0, 31, 63):
            inside = [v.copy() for v in vals]
            inside[k][i] += 1.99 * bnds[k][i]
            ok = bounds.judge_outputs(vals, bnds, inside)
            assert ok["pass"] and 0.99 < ok["worst"] < 1.0, (k, i, ok)
            outside = [v.copy() for v in vals]
            outside[k][i] -= 2.01 * bnds[k][i]
            bad = bounds.judge_outputs(vals, bnds, outside)
            assert not bad["pass"] and bad["first"]["output"] == k and bad["first"]["index"] == i, (k, i, bad)
            nan = [v.copy() for v in vals]
            nan[k][i] = np.nan
            bad = bounds.judge_outputs(vals, bnds, nan)
            assert not bad["pass"] and bad["first"]["output"] == k and bad["worst"] == np.inf


def test_judge_outputs_last_element_of_last_output():
    vals, bnds = _three_outputs()
    gpu = [v.copy() for v in vals]
    gpu[-1][-1] += 2.01 * bnds[-1][-1]
    bad = bounds.judge_outputs(vals, bnds, gpu)
    assert not bad["pass"] and bad["first"]["output"] == 2 and bad["first"]["index"] == 63


def test_judge_outputs_refuses_missing_and_short_outputs():
    vals, bnds = _three_outputs()
    gpu = [v.copy() for v in vals]
    # One output fewer: the zip would silently drop the last one.
    bad = bounds.judge_outputs(vals, bnds, gpu[:2])
    assert not bad["pass"] and bad["first"]["reason"] == "length"
    # A size-1 array would broadcast against the full reference.
    bad = bounds.judge_outputs(vals, bnds, gpu[:2] + [gpu[2][:1]])
    assert not bad["pass"] and bad["first"] == {"output": 2, "reason": "length"}
    bad = bounds.judge_outputs(vals, bnds, gpu[:2] + [gpu[2][:-1]])
    assert not bad["pass"] and bad["first"]["reason"] == "length"


@pytest.mark.parametrize("cancelled,passes", [(99, True), (101, False)])
def test_judge_outputs_one_percent_rule(cancelled, passes):
    """a / (b - 1) with b = 1 at `cancelled` of 10000 elements: those quotients are
    infinite with an unbounded error, so they are unjudgeable. 0.99 % passes, 1.01 % is
    unjudged and fails, whatever the other elements say."""
    n = 10000
    g = _g([_in("a", [n]), _in("b", [n]), _node("const", [], [n], shape=[n], value=1),
            _node("sub", [1, 2], [n]), _node("div", [0, 3], [n])])
    rng = np.random.default_rng(3)
    b = rng.uniform(2, 3, size=n)
    b[rng.permutation(n)[:cancelled]] = 1.0
    r = bounds.reference_with_bounds(g, {"a": rng.uniform(1, 2, size=n), "b": b})
    v, e = r["values"][4], r["bounds"][4]
    gpu = v.astype(np.float32)
    j = bounds.judge_outputs([v], [e], [gpu])
    assert j["unjudgeable"] == cancelled and j["elements"] == n
    assert j["pass"] is passes and j["unjudged"] is (not passes)
    # Within the rule, a judgeable element off by 2.01 E still fails.
    if passes:
        i = int(np.flatnonzero(np.isfinite(e))[-1])
        moved = v.copy()
        moved[i] += 2.01 * e[i]
        assert not bounds.judge_outputs([v], [e], [moved])["pass"]


def _fused_mlp_tail(tool):
    """relu(x·w + b) (a fused matmul epilogue), its column sum (a plain launch) and
    exp(-s) (a fused elementwise chain), fused by the host's fuse(), with the oracle's
    node-local expectation for every launched node."""
    g = _g([_in("x", [4, 8]), _in("w", [8, 6]), _in("b", [6]),
            _node("matmul", [0, 1], [4, 6]), _node("broadcast", [2], [4, 6], shape=[4, 6]),
            _node("add", [3, 4], [4, 6]), _node("relu", [5], [4, 6]),
            _node("sum", [6], [6], axis=0, keepDims=False), _node("neg", [7], [6]), _node("exp", [8], [6])])
    f = tool("fuse", {"graphs": [{"name": "tail", "graph": g, "keep": [9]}]})[0]
    fused = f["graph"]
    rng = np.random.default_rng(11)
    ref = bounds.reference_with_bounds(g, {"x": rng.normal(size=32), "w": rng.normal(size=48), "b": rng.normal(size=6)})
    vals = [ref["values"][o] for o in f["origin"]]
    expected, bound = bounds.local_reference_fused(fused, vals)
    kinds = {i: (n["attrs"]["pattern"] if n["op"] == "fused" else n["op"]) for i, n in enumerate(fused["nodes"]) if i in expected}
    assert sorted(kinds.values()) == ["elementwise", "matmul-epilogue", "sum"], kinds
    return fused, expected, bound, kinds


def test_judge_local_planted_errors(tool):
    fused, expected, bound, kinds = _fused_mlp_tail(tool)
    gpu = {k: v.astype(np.float32) for k, v in expected.items()}
    ok = bounds.judge_local(fused, gpu, expected, bound)
    assert ok["pass"] and ok["elements"] == 24 + 6 + 6 and set(ok["byKind"]) == {"matmul-epilogue", "plain", "elementwise"}
    for node_id, kind in kinds.items():
        e = bound[node_id]
        i = int(np.argmax(e))
        assert e[i] > 0
        inside = dict(gpu)
        inside[node_id] = expected[node_id].copy()
        inside[node_id][i] += 1.99 * e[i]
        assert bounds.judge_local(fused, inside, expected, bound)["pass"], kind
        outside = dict(gpu)
        outside[node_id] = expected[node_id].copy()
        outside[node_id][i] -= 2.01 * e[i]
        bad = bounds.judge_local(fused, outside, expected, bound)
        assert not bad["pass"] and bad["first"]["node"] == node_id and bad["first"]["index"] == i, kind
        nan = dict(gpu)
        nan[node_id] = expected[node_id].copy()
        nan[node_id][i] = np.nan
        assert not bounds.judge_local(fused, nan, expected, bound)["pass"], kind
    # The last element of the last launched node.
    last = max(expected)
    moved = dict(gpu)
    moved[last] = expected[last].copy()
    moved[last][-1] += 2.01 * bound[last][-1]
    bad = bounds.judge_local(fused, moved, expected, bound)
    assert not bad["pass"] and bad["first"]["node"] == last and bad["first"]["index"] == expected[last].size - 1


def test_judge_local_refuses_missing_and_short_nodes(tool):
    fused, expected, bound, kinds = _fused_mlp_tail(tool)
    gpu = {k: v.astype(np.float32) for k, v in expected.items()}
    for node_id in expected:
        missing = {k: v for k, v in gpu.items() if k != node_id}
        bad = bounds.judge_local(fused, missing, expected, bound)
        assert not bad["pass"] and bad["first"]["node"] == node_id and bad["first"]["reason"] == "missing"
        short = dict(gpu)
        short[node_id] = gpu[node_id][:-1]
        bad = bounds.judge_local(fused, short, expected, bound)
        assert not bad["pass"] and bad["first"]["reason"] == "length"


@pytest.mark.parametrize("cancelled,passes", [(99, True), (101, False)])
def test_judge_local_one_percent_rule(cancelled, passes):
    """10000 elements over two launched nodes, `cancelled` of them with an unbounded
    expectation (spread over both nodes): 0.99 % passes, 1.01 % is unjudged."""
    graph = _g([_in("a", [6000]), _node("exp", [0], [6000]), _node("neg", [0], [4000])])
    rng = np.random.default_rng(5)
    expected = {1: rng.normal(size=6000), 2: rng.normal(size=4000)}
    bound = {1: np.full(6000, 1e-6), 2: np.full(4000, 1e-6)}
    flat = rng.permutation(10000)[:cancelled]
    for f in flat:
        node, i = (1, f) if f < 6000 else (2, f - 6000)
        bound[node][i] = np.inf
    gpu = {k: v.copy() for k, v in expected.items()}
    j = bounds.judge_local(graph, gpu, expected, bound)
    assert j["unjudgeable"] == cancelled and j["elements"] == 10000
    assert j["pass"] is passes and j["unjudged"] is (not passes)


def test_local_reference_fused_equals_the_whole_graph_on_exact_operands(tool):
    """With operands that float32 holds exactly (small integers, so the matmul, bias, relu
    and column sum are exact too), each launched node's node-local expectation is the
    whole graph's float64 value of the node it stands for, bit for bit: the body is
    evaluated on the right operands, in the right order, and its output node is the one
    read. The sum's bound is the plain op's own, the chain's the composed body's."""
    g = _g([_in("x", [4, 8]), _in("w", [8, 6]), _in("b", [6]),
            _node("matmul", [0, 1], [4, 6]), _node("broadcast", [2], [4, 6], shape=[4, 6]),
            _node("add", [3, 4], [4, 6]), _node("relu", [5], [4, 6]),
            _node("sum", [6], [6], axis=0, keepDims=False), _node("neg", [7], [6]), _node("exp", [8], [6])])
    f = tool("fuse", {"graphs": [{"name": "tail", "graph": g, "keep": [9]}]})[0]
    rng = np.random.default_rng(13)
    ref = bounds.reference_with_bounds(g, {"x": rng.integers(-3, 4, size=32), "w": rng.integers(-3, 4, size=48),
                                           "b": rng.integers(-3, 4, size=6)})
    vals = [ref["values"][o] for o in f["origin"]]
    expected, bound = bounds.local_reference_fused(f["graph"], vals)
    assert len(expected) == 3
    for node_id, v in expected.items():
        o = f["origin"][node_id]
        assert np.array_equal(v, ref["values"][o]), (node_id, o)
    # The matmul epilogue and the column sum are exact: their bounds are rounding-only
    # (gamma terms) and non-negative; exp's is positive everywhere.
    chain = max(expected)
    assert np.all(bound[chain] > 0)
    assert f["graph"]["nodes"][chain]["attrs"]["pattern"] == "elementwise"


def test_judge_fused_refuses_a_node_no_original_holds(tool):
    """A fused node whose origin is -1 (the transposed operand the trainer's lowering forms
    for a product formed transposed) has no reference value: judge_fused refuses it with
    reason 'origin' instead of reading the last node's reference. The trainer's fused step
    marks such nodes -1 and no longer maps the product's original id to them."""
    import tcmi_bridge
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        tool("step-graph", {"model": "transformer-ref"}, out=d)
        c = tcmi_bridge.Bundle(d).cases[0]
    formed = [i for i, o in enumerate(c["origin"]) if o < 0]
    assert formed and all(c["fused"]["nodes"][i]["op"] == "transpose" for i in formed)
    g = {"nodes": [{"op": "input", "inputs": [], "attrs": {"name": "a"}, "shape": [2]},
                   {"op": "neg", "inputs": [0], "attrs": {}, "shape": [2]}]}
    ref = bounds.reference_with_bounds(g, {"a": [1.0, 2.0]})
    gpu = [np.array([1.0, 2.0]), np.array([-1.0, -2.0])]
    assert bounds.judge_fused(g, [0, 1], gpu, ref)["pass"]
    j = bounds.judge_fused(g, [0, -1], gpu, ref)
    assert not j["pass"] and j["first"]["reason"] == "origin" and j["first"]["node"] == 1
