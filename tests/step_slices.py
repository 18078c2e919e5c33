"""Per-sequence blocks of a training step's launches, for node-local judging at the
full batch (tests/test_gpu_step_slices.py) and its CPU check (tests/test_step_slices.py).

A launch whose output carries the batch axis is evaluated for one sequence on that
sequence's blocks of its operands, with the block shapes of the same builder's
one-sequence graph (the twin) and the full graph's constants; a launch whose output
does not is evaluated whole."""
from typing import List, Sequence

import numpy as np

from oracle import bounds, interp


def fused_values(fused, origin, values):
    """The value of every node of a fused step graph: its original node's value, or, for a
    node no original node holds (origin -1: the transposed operand the trainer's lowering
    forms for a product it forms transposed), its own op on the values before it."""
    out = []
    for i, o in enumerate(origin):
        if o >= 0:
            out.append(values[o])
            continue
        node = fused["nodes"][i]
        assert node["op"] == "transpose", node["op"]
        out.append(interp.kernel(node, [out[j] for j in node["inputs"]], fused))
    return out


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


def _producer_body(graph, p):
    """The body nodes and output index of node `p` (a producer or a chain): a fused node's
    own body, or its one op on inputs a0.. (the node's operands in order)."""
    if p["op"] == "fused":
        return p["attrs"]["body"]["nodes"], p["attrs"]["output"]
    ins = [{"op": "input", "inputs": [], "attrs": {"name": f"a{k}", "shape": graph["nodes"][i]["shape"]},
            "shape": graph["nodes"][i]["shape"]} for k, i in enumerate(p["inputs"])]
    return ins + [{"op": p["op"], "inputs": list(range(len(ins))), "attrs": p["attrs"], "shape": p["shape"]}], len(ins)


def fold_reductions(graph, node_id, folds):
    """A launch of the perf lowering that took row reductions into a chain, fused or a
    single op (its record's rowFolds: [{reduction, pos}], with producer and producerPos
    where the reduction's operand is formed in the launch too, or columns where the
    reduction is a column sum taken into its one reader): the chain as a fused node,
    each body input at `pos` (the reduction's value) replaced by the reduction itself,
    applied to a new input a{pos[0]} — or to the producer's body on inputs
    a{producerPos[j]} — and the launch's operand node ids (the reduction's operand in
    those positions, or the producer's operands). Restated here from the lowering's rule,
    so a wrong fold there fails the judge."""
    node = graph["nodes"][node_id]
    if not folds:
        return node, list(node["inputs"])
    at = {p: f for f in folds for p in f["pos"]}
    if node["op"] == "fused":
        body, chain_out, attrs = node["attrs"]["body"]["nodes"], node["attrs"]["output"], node["attrs"]
    else:
        # A single-op chain: its op on inputs a0.. (the node's operands in order).
        body, chain_out = _producer_body(graph, node)
        attrs = {"kind": "elementwise", "pattern": "elementwise"}
    out, where, reduced = [], {}, {}
    for bid, b in enumerate(body):
        f = at.get(int(b["attrs"]["name"][1:])) if b["op"] == "input" else None
        if f is not None:
            red = graph["nodes"][f["reduction"]]
            if f["reduction"] not in reduced and f.get("columns"):
                # A column sum (a sum over a non-last axis) taken into its one reader: the
                # sum itself, as the graph states it, on a new input of its operand's shape.
                src = graph["nodes"][red["inputs"][0]]["shape"]
                assert red["op"] == "sum" and int(np.prod(src[red["attrs"]["axis"] + 1:])) > 1
                out.append({"op": "input", "inputs": [], "attrs": {"name": f"a{f['pos'][0]}", "shape": src}, "shape": src})
                out.append({"op": red["op"], "inputs": [len(out) - 1], "attrs": red["attrs"], "shape": red["shape"]})
                reduced[f["reduction"]] = len(out) - 1
            if f["reduction"] not in reduced:
                # The operand as [outer, n] rows reduced along them (the reduced axis is the
                # last non-trivial one), then the reduction's own shape.
                src = graph["nodes"][red["inputs"][0]]["shape"]
                axis = red["attrs"]["axis"]
                rows = [int(np.prod(src[:axis])), src[axis]]
                if "producer" in f:
                    p = graph["nodes"][f["producer"]]
                    assert red["inputs"][0] == f["producer"] and p["shape"] == rows
                    pnodes, pout = _producer_body(graph, p)
                    pmap = {}
                    for pid, pn in enumerate(pnodes):
                        if pn["op"] == "input":
                            name = f"a{f['producerPos'][int(pn['attrs']['name'][1:])]}"
                            out.append(dict(pn, attrs=dict(pn["attrs"], name=name)))
                        else:
                            out.append(dict(pn, inputs=[pmap[i] for i in pn["inputs"]]))
                        pmap[pid] = len(out) - 1
                    operand = pmap[pout]
                else:
                    out.append({"op": "input", "inputs": [], "attrs": {"name": f"a{f['pos'][0]}", "shape": rows},
                                "shape": rows})
                    operand = len(out) - 1
                out.append({"op": red["op"], "inputs": [operand], "attrs": {"axis": 1, "keepDims": True},
                            "shape": [rows[0], 1]})
                if red["shape"] != [rows[0], 1]:
                    out.append({"op": "reshape", "inputs": [len(out) - 1], "attrs": {"shape": red["shape"]},
                                "shape": red["shape"]})
                reduced[f["reduction"]] = len(out) - 1
            where[bid] = reduced[f["reduction"]]
        else:
            out.append(dict(b, inputs=[where[i] for i in b["inputs"]]))
            where[bid] = len(out) - 1
    inputs = list(node["inputs"])
    for f in folds:
        for p in f["pos"]:
            assert inputs[p] == f["reduction"]
            inputs[p] = graph["nodes"][f["reduction"]]["inputs"][0]
        if "producer" in f:
            pins = graph["nodes"][f["producer"]]["inputs"]
            for p in f["pos"]:
                inputs[p] = pins[0]
            for j, p in enumerate(f["producerPos"]):
                inputs.extend([None] * (p + 1 - len(inputs)))
                inputs[p] = pins[j]
    assert None not in inputs
    attrs = dict(attrs, body={"nodes": out}, output=where[chain_out])
    return dict(node, op="fused", attrs=attrs, inputs=inputs), inputs


def _absorbed_body(graph, node_id, absorbed):
    """(body nodes, output index, operand node ids) of node `node_id` with the producers in
    `absorbed` formed inside its body: each input at `pos` replaced by the producer's own
    body (with what that producer absorbed, restated the same way) on inputs
    a{producerPos[j]}, the producer's operands taking those positions."""
    node = graph["nodes"][node_id]
    body, out = _producer_body(graph, node)
    inputs = list(node["inputs"])
    if not absorbed:
        return body, out, inputs
    at = {p: a for a in absorbed for p in a["pos"]}
    nodes, where, formed = [], {}, {}
    for bid, b in enumerate(body):
        a = at.get(int(b["attrs"]["name"][1:])) if b["op"] == "input" else None
        if a is not None:
            key = a["producer"]
            if key not in formed:
                assert node["inputs"][a["pos"][0]] == a["producer"]
                pbody, pout, _ = _absorbed_body(graph, a["producer"], a.get("absorbed"))
                pmap = {}
                for pid, pn in enumerate(pbody):
                    if pn["op"] == "input":
                        name = f"a{a['producerPos'][int(pn['attrs']['name'][1:])]}"
                        nodes.append(dict(pn, attrs=dict(pn["attrs"], name=name)))
                    else:
                        nodes.append(dict(pn, inputs=[pmap[i] for i in pn["inputs"]]))
                    pmap[pid] = len(nodes) - 1
                formed[key] = pmap[pout]
            where[bid] = formed[key]
        else:
            nodes.append(dict(b, inputs=[where[i] for i in b["inputs"]]))
            where[bid] = len(nodes) - 1
    for a in absorbed:
        _, _, pins = _absorbed_body(graph, a["producer"], a.get("absorbed"))
        assert len(pins) == len(a["producerPos"])
        for p in a["pos"]:
            inputs[p] = pins[0]
        for j, p in enumerate(a["producerPos"]):
            inputs.extend([None] * (p + 1 - len(inputs)))
            inputs[p] = pins[j]
    assert None not in inputs
    return nodes, where[out], inputs


def absorbed_producers(absorbed):
    """Every producer node id in a {reader: [absorbed records]} map, nested ones included."""
    out = set()

    def walk(records):
        for a in records or []:
            out.add(a["producer"])
            walk(a.get("absorbed"))
    for records in absorbed.values():
        walk(records)
    return out


def absorb_producers(graph, node_id, absorbed):
    """A launch of the perf lowering that absorbed elementwise producers (its record's
    absorbed: [{producer, pos, producerPos, absorbed?}]): the reader as a fused node whose
    body forms each producer's value where it would have loaded it, and the launch's
    operand node ids. Restated here from the lowering's rule, so a wrong absorption there
    fails the judge."""
    node = graph["nodes"][node_id]
    nodes, out, inputs = _absorbed_body(graph, node_id, absorbed)
    attrs = {"kind": "elementwise", "pattern": node["attrs"].get("pattern", "elementwise"), "body": {"nodes": nodes},
             "output": out}
    return dict(node, op="fused", attrs=attrs, inputs=inputs), inputs


def _reaches(graph, i, values):
    """Whether node i is one of `values`, or a broadcast or reshape of one."""
    n = graph["nodes"][i]
    return i in values or (n["op"] in ("broadcast", "reshape") and _reaches(graph, n["inputs"][0], values))


def form_values(graph, node_id, formed, folds=None, absorbed=None):
    """A launch of the perf lowering that forms values it reads (its record's formed:
    [{value, rowFolds?, absorbed?}], every value formed inside it): the launch restated
    without them (with its own row folds or absorbed producers), every operand that is one
    of those values — directly, or a broadcast or reshape of one — replaced by that value's
    own launch restated the same way, on its operands in turn (each value once, reshaped to
    where it is read). The launch's operands are the nodes left to read, in order of first
    use. Restated here from the lowering's rule, by node ids: a value formed from the
    wrong operands, or a record naming a value the launch does not read, fails."""
    nodes = graph["nodes"]
    recs = {f["value"]: f for f in formed}
    out, ins, memo = [], [], {}

    def value(i, shape):
        if i not in memo:
            n = nodes[i]
            if i in recs:
                memo[i] = inline(*restate(graph, i, recs[i].get("rowFolds"), recs[i].get("absorbed")))
            elif _reaches(graph, i, recs):
                src = value(n["inputs"][0], nodes[n["inputs"][0]]["shape"])
                out.append({"op": n["op"], "inputs": [src], "attrs": n["attrs"], "shape": n["shape"]})
                memo[i] = len(out) - 1
            else:
                out.append({"op": "input", "inputs": [], "attrs": {"name": f"a{len(ins)}", "shape": n["shape"]},
                            "shape": n["shape"]})
                ins.append(i)
                memo[i] = len(out) - 1
        v = memo[i]
        if list(out[v]["shape"]) != list(shape):
            out.append({"op": "reshape", "inputs": [v], "attrs": {"shape": list(shape)}, "shape": list(shape)})
            v = len(out) - 1
        return v

    def inline(node, node_ins):
        body, bout = _producer_body(graph, node)
        where = {}
        for bid, b in enumerate(body):
            if b["op"] == "input":
                where[bid] = value(node_ins[int(b["attrs"]["name"][1:])], b["shape"])
            else:
                out.append(dict(b, inputs=[where[x] for x in b["inputs"]]))
                where[bid] = len(out) - 1
        return where[bout]

    node, node_ins = restate(graph, node_id, folds, absorbed)
    o = inline(node, node_ins)
    assert set(recs) <= set(memo), (node_id, sorted(set(recs) - set(memo)))
    attrs = dict(node["attrs"]) if node["op"] == "fused" else {"kind": "elementwise", "pattern": "elementwise"}
    attrs = dict(attrs, body={"nodes": out}, output=o)
    return dict(node, op="fused", attrs=attrs, inputs=ins), ins


def formed_values(formed):
    """The values that the launches of {reader: [formed records]} form, and the reductions
    and producers folded into those values' own launches (their row folds and absorbed
    producers)."""
    values, reductions, producers = set(), set(), set()
    for records in formed.values():
        for f in records:
            values.add(f["value"])
            for x in f.get("rowFolds") or []:
                reductions.add(x["reduction"])
                if "producer" in x:
                    producers.add(x["producer"])
            producers |= absorbed_producers({0: f.get("absorbed") or []})
    return values, reductions, producers


def restate(graph, node_id, folds=None, absorbed=None, formed=None):
    """The launch of node `node_id` as the perf lowering runs it: its row folds or its
    absorbed producers restated (a launch has at most one of them), then the values it
    forms, or the node itself."""
    if formed:
        return form_values(graph, node_id, formed, folds, absorbed)
    if absorbed:
        assert not folds
        return absorb_producers(graph, node_id, absorbed)
    return fold_reductions(graph, node_id, folds)


def merge_twin(n, t):
    """Node `n` of the full graph with the shapes of its twin `t` (the same node of the
    one-sequence graph) and the full graph's constants: body nodes keep their op, inputs,
    axes, permutations and constant values, and take the twin's shapes and shape
    attributes."""
    def merge(a, b):
        assert a["op"] == b["op"] and a["inputs"] == b["inputs"]
        attrs = dict(a["attrs"])
        if "shape" in b["attrs"]:
            attrs["shape"] = b["attrs"]["shape"]
        return dict(a, attrs=attrs, shape=b["shape"])

    node = merge(n, t)
    if n["op"] == "fused":
        body = {"nodes": [merge(x, y) for x, y in zip(n["attrs"]["body"]["nodes"], t["attrs"]["body"]["nodes"])]}
        node["attrs"] = dict(node["attrs"], body=body)
    return node


def twin_node(full, twin, node_id):
    """The full graph's node with the twin's shapes and the full graph's constants."""
    return merge_twin(full["nodes"][node_id], twin["nodes"][node_id])


def local(graph, node, operands: List[np.ndarray]):
    """(value, bound) of one launched node on its operand values (localReferenceFused,
    harness-m4.js:182-200)."""
    if node["op"] == "fused":
        g, out = node["attrs"]["body"], node["attrs"]["output"]
    else:
        g, out = bounds.one_op_graph(graph, node)
    r = bounds.reference_with_bounds(g, {f"a{k}": v for k, v in enumerate(operands)})
    return r["values"][out], r["bounds"][out]


def expectations(full, twin, launched, operand, sequences, row_folds=None, absorbed=None, formed=None):
    """Yield (node id, sequence index or None, value, bound) for every launched node:
    per sequence where its output carries the batch axis, whole otherwise.
    `operand(i, s)` is node i's value: its block for sequence index s, or whole for None.
    `row_folds` ({node id: [{reduction, pos}]}, a perf lowering's): those launches are the
    chain with its row reductions taken in, on the reductions' operands; `absorbed`
    ({node id: [{producer, pos, producerPos}]}): those launches form their producers;
    `formed` ({node id: [formed records]}): those launches form the values they read."""
    axis = [batch_axis(n["shape"], t["shape"]) for n, t in zip(full["nodes"], twin["nodes"])]
    row_folds = row_folds or {}
    absorbed = absorbed or {}
    formed = formed or {}
    for nid in launched:
        folds = row_folds.get(nid) or row_folds.get(str(nid))
        took = absorbed.get(nid) or absorbed.get(str(nid))
        rows = formed.get(nid) or formed.get(str(nid))
        node, ins = restate(full, nid, folds, took, rows)
        if axis[nid] >= 0:
            tn = merge_twin(node, restate(twin, nid, folds, took, rows)[0])
            for s in range(len(sequences)):
                ops = [operand(i, s if axis[i] >= 0 else None) for i in ins]
                v, e = local(twin, tn, ops)
                yield nid, s, v, e
        else:
            v, e = local(full, node, [operand(i, None) for i in ins])
            yield nid, None, v, e


def judge_case(fused, fused_vals, gc, arr):
    """Node-local judgement of one gpu-local case (tool.js gpuLocal): every launch of the
    checked lowering against its float64 expectation on the reference operands
    `fused_vals` (localReferenceFused + judgeLocal, harness-m4.js:182-223), and, where the
    case holds it, every launch of the perf lowering — whose skipped nodes must be exactly
    its shared reshapes, in-place transposes and broadcasts, folded reductions and
    producers, relus applied on load and dead nodes, and whose folded launches are judged
    as the launches they are. `arr` reads a bundle array. Returns (checked, perf or None)."""
    expected, bound = bounds.local_reference_fused(fused, fused_vals)
    gpu = {int(k): arr(v) for k, v in gc["gpu"].items()}
    assert set(gpu) == set(expected)
    j = bounds.judge_local(fused, gpu, expected, bound)
    if "gpuPerf" not in gc:
        return j, None
    perf = {int(k): arr(v) for k, v in gc["gpuPerf"].items()}
    skipped = set(expected) - set(perf)
    assert skipped == {a for a, _ in gc["aliases"]} | set(gc["folded"]) | set(gc["dead"])
    # Reductions folded into their row-statistics chains, and the producers of their
    # operands formed in the same launches, are the other launches it skips.
    folds = {int(k): v for k, v in gc["rowFolds"].items()}
    took = {int(k): v for k, v in gc["absorbed"].items()}
    rows = {int(k): v for k, v in gc.get("formed", {}).items()}
    reductions = {f["reduction"] for fs in folds.values() for f in fs}
    producers = {f["producer"] for fs in folds.values() for f in fs if "producer" in f}
    producers |= absorbed_producers(took)
    # Values formed by their readers, with what their own launches would fold or absorb.
    values, value_reductions, value_producers = formed_values(rows)
    assert all(fused["nodes"][i]["op"] not in ("matmul", "input", "const") for i in values)
    reductions |= {i for i in values if fused["nodes"][i]["op"] in ("sum", "max")} | value_reductions
    producers |= value_producers
    # Relus the matmuls reading them apply as they load their operand.
    on_load = {o["node"] for ops in gc["loadOps"].values() for o in ops}
    nodes = fused["nodes"]
    assert all(nodes[i]["op"] == "relu" for i in on_load)
    assert all(nodes[i]["op"] in ("reshape", "transpose", "broadcast")
               for i in skipped - set(gc["dead"]) - reductions - producers - on_load - values)
    assert all(nodes[i]["op"] in ("sum", "max") for i in reductions)
    assert all(nodes[i]["op"] not in ("sum", "max", "matmul") for i in producers)
    # A chain with its reductions folded in is judged as the launch it is: the reductions and
    # the chain on the reductions' operands.
    pexp, pbound = {}, {}
    for k in perf:
        if k in folds or k in took or k in rows:
            node, ins = restate(fused, k, folds.get(k), took.get(k), rows.get(k))
            pexp[k], pbound[k] = local(fused, node, [fused_vals[i] for i in ins])
        else:
            pexp[k], pbound[k] = expected[k], bound[k]
    jp = bounds.judge_local(fused, perf, pexp, pbound)
    jp["skipped"], jp["chains"], jp["formed"] = len(skipped), len(folds), len(values)
    return j, jp
