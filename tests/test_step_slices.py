"""The per-sequence blocks that judge config 5's step at its full batch on the GPU
(tests/test_gpu_step_slices.py), checked on the CPU at B = 2 against the whole launches:
for every launch of the fused step whose output carries the batch axis, the oracle's
value and bound on one sequence's operand blocks, with the one-sequence twin's shapes
and the full graph's constants, equal that sequence's block of the value and bound of
the whole launch, bit for bit. A block taken along the wrong axis, a constant taken
from the twin (the loss scale 1/(B*T)), or a launch whose rows depended on another
sequence would break the equality."""
import numpy as np
import pytest

from oracle import bounds, interp
from step_slices import (absorb_producers, absorbed_producers, batch_axis, expectations, fold_reductions, fused_values,
                         local, restate, take_block)


@pytest.mark.parametrize("attention", [False, True])
def test_sequence_blocks_equal_the_whole_launch(tmp_path, tool, attention):
    """With `attention`, the step with attention and its gradient fused
    (fusion/attention.js): its attention and attention-grad nodes are blocked the same way."""
    import tcmi_bridge
    B = 2
    tool("step-graph", {"model": "transformer", "B": B, "attention": attention}, out=str(tmp_path / "full"))
    tool("step-graph", {"model": "transformer", "B": 1, "attention": attention}, out=str(tmp_path / "twin"))
    fb, tb = tcmi_bridge.Bundle(tmp_path / "full"), tcmi_bridge.Bundle(tmp_path / "twin")
    c = fb.cases[0]
    full, twin = c["fused"], tb.cases[0]["fused"]
    inputs = {k: fb.arr(v) for k, v in c["inputs"].items()}
    with interp.blas_matmul():
        ref = bounds.reference_with_bounds(c["graph"], inputs)
    # The operands: float32 values of every fused node, as a GPU run would give them.
    vals = [v.astype(np.float32) for v in fused_values(full, c["origin"], ref["values"])]
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
    assert blocked >= 2 * (250 if attention else 300), blocked
    if attention:
        kinds = {nodes[n]["attrs"]["kind"] for n in whole if nodes[n]["op"] == "fused"}
        assert {"attention", "attention-grad"} <= kinds, kinds
    # The step's mean over B*T positions reaches some per-sequence launch as a constant.
    assert any(abs(v * B * 128 - 1) < 1e-12 or abs(v - B * 128) < 1e-9 for v in scales), sorted(scales)[:20]
    # The launches judged whole do not carry the batch, and some read operands that do.
    wholes = [i for i in launched if axis[i] < 0]
    assert wholes and any(axis[j] >= 0 for i in wholes for j in nodes[i]["inputs"])


def test_folded_row_reductions_are_the_chain_on_the_reduction(tool):
    """The perf lowering takes config 5's row reductions (LayerNorm's sums, softmax's row
    sums) into the row-statistics chains that read them. The checkers' restatement of such
    a launch (fold_reductions) evaluated in float64 on a chain's operands equals the
    reduction evaluated first and the chain's own body applied to its value, bit for bit,
    value and bound: the fold changes where the reduction runs, not what is computed. The
    same holds where the launch also forms the reduction's operand from its producer's
    operands (the producer evaluated first on the unfolded side). Chains run as launches of
    their own or inside the launches that form them (their records carry the folds)."""
    d = tool("perf-lower", {"model": "transformer", "B": 1})
    graph, folds = d["graph"], {int(k): v for k, v in d["rowFolds"].items()}
    folds.update({f["value"]: f["rowFolds"] for fs in d["formed"].values() for f in fs if f.get("rowFolds")})
    assert len(folds) >= 20
    reds = {f["reduction"] for fs in folds.values() for f in fs}
    assert reds <= set(d["folded"]) and all(graph["nodes"][r]["op"] in ("sum", "max") for r in reds)
    rng = np.random.default_rng(3)
    producers = [k for k, fs in folds.items() if any("producer" in f for f in fs)]
    assert len(producers) >= 6
    # Column sums taken into their one reader (a bias's update), at batch 1 one-pass sums.
    columns = [k for k, fs in folds.items() if any(f.get("columns") for f in fs)]
    assert len(columns) >= 6
    for k, fs in list(folds.items())[:12] + [(k, folds[k]) for k in producers[:12] + columns[:8]]:
        node, ins = fold_reductions(graph, k, fs)
        # Positive operands keep the deviation chains' square roots real.
        ops = [rng.uniform(0.5, 2.0, size=interp.size(graph["nodes"][i]["shape"])).astype(np.float32) for i in ins]
        v, e = local(graph, node, ops)
        # The same launch the unfolded way: each reduction's producer by itself (where the
        # launch forms the reduction's operand too), each reduction, then the chain.
        chain_ops = []
        by_red = {f["reduction"]: f for f in fs}
        for pos, i in enumerate(graph["nodes"][k]["inputs"]):
            if i in by_red:
                red, f = graph["nodes"][i], by_red[i]
                if "producer" in f:
                    pv, pe = local(graph, graph["nodes"][f["producer"]], [ops[q] for q in f["producerPos"]])
                    rg, rout = bounds.one_op_graph(graph, red)
                    r = bounds.reference_with_bounds(rg, {}, carried={"a0": (pv, pe)})
                    rv, re_ = r["values"][rout], r["bounds"][rout]
                else:
                    rv, re_ = local(graph, red, [ops[pos]])
                chain_ops.append((rv, re_))
            else:
                chain_ops.append((ops[pos].astype(np.float64), np.zeros(ops[pos].size)))
        chain = graph["nodes"][k]
        if chain["op"] == "fused":
            body, out = chain["attrs"]["body"], chain["attrs"]["output"]
        else:
            body, out = bounds.one_op_graph(graph, chain)
        carried = {f"a{p}": ce for p, ce in enumerate(chain_ops)}
        r = bounds.reference_with_bounds(body, {}, carried=carried)
        assert np.array_equal(v, r["values"][out]) and np.all(np.isfinite(v)), k
        assert np.array_equal(e, r["bounds"][out]), k


def _unabsorbed(graph, nid, records, ops):
    """(value, bound) of node `nid` evaluated the unabsorbed way: each absorbed producer
    evaluated first, on its own operands (its producerPos of the launch's operands), then
    the node's own body on those values and its other operands."""
    node = graph["nodes"][nid]
    at = {p: a for a in records or [] for p in a["pos"]}
    carried = {}
    for p in range(len(node["inputs"])):
        a = at.get(p)
        carried[f"a{p}"] = ops[p] if a is None else _unabsorbed(graph, a["producer"], a.get("absorbed"),
                                                                 [ops[q] for q in a["producerPos"]])
    if node["op"] == "fused":
        body, out = node["attrs"]["body"], node["attrs"]["output"]
    else:
        body, out = bounds.one_op_graph(graph, node)
    r = bounds.reference_with_bounds(body, {}, carried=carried)
    return r["values"][out], r["bounds"][out]


def test_absorbed_producers_are_formed_as_computed(tool):
    """The trainer's lowering lets an elementwise launch form an elementwise producer that
    only it reads (the producer's other consumer dead), where it would have loaded it. The
    checkers' restatement of such a launch (absorb_producers), evaluated in float64 on the
    launch's operands, equals each producer evaluated first and the reader's own body
    applied to its value, bit for bit, value and bound."""
    d = tool("perf-lower", {"model": "transformer", "B": 1})
    graph, took = d["graph"], {int(k): v for k, v in d["absorbed"].items()}
    assert len(took) >= 6
    assert absorbed_producers(took) <= set(d["folded"])
    rng = np.random.default_rng(4)
    for k, records in took.items():
        node, ins = absorb_producers(graph, k, records)
        ops = [rng.uniform(0.5, 2.0, size=interp.size(graph["nodes"][i]["shape"])).astype(np.float32) for i in ins]
        v, e = local(graph, node, ops)
        rv, re_ = _unabsorbed(graph, k, records, [(o.astype(np.float64), np.zeros(o.size)) for o in ops])
        assert np.array_equal(v, rv) and np.all(np.isfinite(v)), k
        assert np.array_equal(e, re_), k


def _perf_lowered(tool, req):
    if "c3" not in req:
        return tool("perf-lower", req)
    g = tool("config-graphs", {"c3": [{"fn": req["c3"], "R": 8, "C": 16}]})["c3"][0]["gradient"]
    return tool("perf-lower", {"graph": g["graph"], "keep": g["keep"], "fuse": {}})


def _carried(graph, i, carried):
    """(value, bound) of node i: carried, or a broadcast or reshape of a carried node."""
    if i in carried:
        return carried[i]
    n = graph["nodes"][i]
    src = n["inputs"][0]
    v, e = _carried(graph, src, carried)
    if n["op"] == "broadcast":
        s0 = graph["nodes"][src]["shape"]
        return interp.k_broadcast(v, s0, n["shape"]), interp.k_broadcast(e, s0, n["shape"])
    assert n["op"] == "reshape", n["op"]
    return v, e


def _run_carried(graph, node, ins, carried):
    if node["op"] == "fused":
        body, out = node["attrs"]["body"], node["attrs"]["output"]
    else:
        body, out = bounds.one_op_graph(graph, node)
    r = bounds.reference_with_bounds(body, {}, carried={f"a{p}": _carried(graph, i, carried) for p, i in enumerate(ins)})
    return r["values"][out], r["bounds"][out]


@pytest.mark.parametrize("req", [{"model": "transformer", "B": 1}, {"model": "transformer", "B": 1, "attention": True},
                                 {"model": "mlp"}, {"c3": "softmax"}, {"c3": "logSoftmax"}])
def test_formed_values_are_the_values_then_the_reader(tool, req):
    """The perf lowering lets a launch form the values it reads — row values (LayerNorm's
    means, a backward's row statistics) and full-size values (LayerNorm's centred rows,
    softmax's exponentials) — from what their own launches would have read, recursively.
    The checkers' restatement of such a launch (form_values), evaluated in float64 on the
    launch's operands, equals each value's own launch evaluated first, in the record's
    order, and the reader's own launch applied to them, bit for bit, value and bound. The
    formed values launch nothing, and a config-3 gradient is two launches: the forward
    reading x, the backward reading x and dy."""
    d = _perf_lowered(tool, req)
    graph = d["graph"]
    formed = {int(k): v for k, v in d["formed"].items()}
    folds = {int(k): v for k, v in d["rowFolds"].items()}
    took = {int(k): v for k, v in d["absorbed"].items()}
    values = {f["value"] for fs in formed.values() for f in fs}
    assert values <= set(d["folded"]) and not values & {x["node"] for x in d["launches"]}
    if "c3" in req:
        assert len(d["launches"]) == 2 and len(formed) == 2, d["launches"]
    elif req["model"] == "transformer":
        assert len(values) >= 40, len(values)
    rng = np.random.default_rng(5)
    for k, records in formed.items():
        node, ins = restate(graph, k, folds.get(k), took.get(k), records)
        ops = [rng.uniform(0.5, 2.0, size=interp.size(graph["nodes"][i]["shape"])).astype(np.float32) for i in ins]
        v, e = local(graph, node, ops)
        assert np.all(np.isfinite(v)), k
        # The unformed way: each value's own launch on the values before it, then the reader.
        carried = {i: (o.astype(np.float64), np.zeros(o.size)) for i, o in zip(ins, ops)}
        for f in records:
            vnode, vins = restate(graph, f["value"], f.get("rowFolds"), f.get("absorbed"))
            carried[f["value"]] = _run_carried(graph, vnode, vins, carried)
        rnode, rins = restate(graph, k, folds.get(k), took.get(k))
        rv, re_ = _run_carried(graph, rnode, rins, carried)
        assert np.array_equal(v, rv), k
        assert np.array_equal(e, re_), k
