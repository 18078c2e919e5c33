"""The host side (JavaScript, run under node) against the reference's recorded
structure: builder graphs node for node, the fusion pass's counts on the
reference's own transformer, the direct-case catalogue, bitwise semantic
preservation of fusion (judged by the float64 oracle), and that every graph
lowers with every load proved in bounds."""
import json

import numpy as np
import pytest

from oracle import interp

ELEMENTWISE = ("add", "sub", "mul", "div", "neg", "exp", "log", "relu", "tanh", "sqrt", "step", "stopGradient")


def test_builder_graphs_equal_reference_cases(golden_cases, tool):
    ref = {c["name"]: c for c in golden_cases}
    built = tool("builder-cases")
    assert len(built) == 12
    for b in built:
        assert b["graph"] == ref[b["name"]]["graph"], b["name"]
        assert b["outputs"] == ref[b["name"]]["outputs"], b["name"]


def test_fusion_counts_on_reference_transformer(m4_counts, tool):
    """measurements.json m4.fusion: forward 212 -> 48 and step 1308 -> 450 launches, by pattern,
    with 2 and 0 activation epilogues; the pass sabotage throws on both (m4.passSabotage.model)."""
    got = {g["graph"]: g for g in tool("model-fusion")}
    for want in m4_counts["fusion"]:
        g = got[want["graph"]]
        for k in ("launchesBefore", "launchesAfter", "byPattern", "epilogues", "epiloguesWithActivation"):
            assert g[k] == want[k], (want["graph"], k, g[k], want[k])
        assert g["unfusedLaunches"] == want["launchesBefore"] and g["fusedLaunches"] == want["launchesAfter"]
    # The reference recorded the pass sabotage failing at node 157 (forward) and 597 (step):
    # "fuse: node 157 used before it is built" (m4.passSabotage.model).
    import re
    for graph, node in (("forward", 157), ("step", 597)):
        msg = got[graph]["passSabotageError"]
        assert msg.startswith("fuse:") and [int(x) for x in re.findall(r"\d+", msg)] == [node], msg


def test_direct_catalogue_is_the_references(m4_counts, tool):
    cat = tool("direct-catalogue")
    want = [(d["name"], d["kind"], d["pattern"]) for d in m4_counts["direct"]]
    assert [(c["name"], c["kind"], c["pattern"]) for c in cat] == want
    by = {}
    for c in cat:
        # Every case fuses into exactly the one kernel it is meant to test.
        assert len(c["launched"]) == 1, c["name"]
        assert c["launched"][0]["op"] == "fused" and c["launched"][0]["kind"] == c["kind"], c["name"]
        assert c["launched"][0]["pattern"] == c["pattern"], c["name"]
        by[c["pattern"]] = by.get(c["pattern"], 0) + 1
    assert by == {k: v["cases"] for k, v in m4_counts["gpuDirect"]["byPattern"].items()}


def _semantics(original, fused, origin, inputs):
    a = interp.evaluate(original, inputs)
    b = interp.evaluate(fused, inputs)
    for nid in range(len(fused["nodes"])):
        x, y = a[origin[nid]], b[nid]
        if x.size != y.size or not np.array_equal(x.view(np.int64), y.view(np.int64)):
            return False
    return True


def test_fusion_preserves_semantics_bitwise(golden_cases, tool):
    """checkSemantics (fuse.js:311-330): the fused graph evaluates bitwise equal at every
    surviving node, on every golden case's forward and gradient graph."""
    grads = tool("grad", {"cases": [{"name": c["name"], "graph": c["graph"], "outputs": c["outputs"]} for c in golden_cases]})
    reqs, feeds = [], []
    for c, g in zip(golden_cases, grads):
        reqs.append({"name": c["name"] + "/fwd", "graph": c["graph"], "keep": c["outputs"]})
        feeds.append(c["inputs"])
        feed = dict(c["inputs"])
        for n, cot in zip(g["cotangents"], c["cotangents"]):
            feed[n] = cot
        reqs.append({"name": c["name"] + "/grad", "graph": g["graph"], "keep": c["outputs"] + g["grads"]})
        feeds.append(feed)
    fused = tool("fuse", {"graphs": reqs})
    n_fused = 0
    for r, f, feed in zip(reqs, fused, feeds):
        assert "error" not in f, (r["name"], f.get("error"))
        assert _semantics(r["graph"], f["graph"], f["origin"], feed), r["name"]
        for node in f["graph"]["nodes"]:
            if node["op"] == "fused":
                n_fused += 1
                assert len(node["inputs"]) <= 6
    assert n_fused > 50


def test_fusion_sabotage_is_caught_by_semantics(golden_cases, tool):
    """The pass sabotage ('fusion-absorbs-shared') either throws or changes some value."""
    reqs = [{"name": c["name"], "graph": c["graph"], "keep": c["outputs"], "sabotage": "fusion-absorbs-shared"}
            for c in golden_cases]
    honest = tool("fuse", {"graphs": [dict(r, sabotage=None) for r in reqs]})
    bad = tool("fuse", {"graphs": reqs})
    caught = 0
    for c, h, b in zip(golden_cases, honest, bad):
        if "error" in b:
            caught += 1
        elif b["graph"] != h["graph"] and not _semantics(c["graph"], b["graph"], b["origin"], c["inputs"]):
            caught += 1
    assert caught >= 1


def test_recompute_option_recomputes(tool):
    """A producer feeding a broadcast is stored once by default and recomputed with
    recompute: true (m4-fusion.test.js:55-63), semantics preserved either way."""
    nodes = [{"op": "input", "inputs": [], "attrs": {"name": "y", "shape": [16, 256]}, "shape": [16, 256]},
             {"op": "input", "inputs": [], "attrs": {"name": "p", "shape": [256]}, "shape": [256]}]
    cyc = ["tanh", "exp", "neg", "exp", "sqrt", "log"]
    for k in range(16):
        nodes.append({"op": cyc[k % 6], "inputs": [len(nodes) - 1 if k else 1], "attrs": {}, "shape": [256]})
    nodes.append({"op": "broadcast", "inputs": [len(nodes) - 1], "attrs": {"shape": [16, 256]}, "shape": [16, 256]})
    nodes.append({"op": "add", "inputs": [0, len(nodes) - 1], "attrs": {}, "shape": [16, 256]})
    g = {"nodes": nodes}
    plain, re = tool("fuse", {"graphs": [{"name": "a", "graph": g, "keep": [len(nodes) - 1]},
                                          {"name": "b", "graph": g, "keep": [len(nodes) - 1], "recompute": True}]})
    count = lambda f: sum(1 for n in f["graph"]["nodes"] if n["op"] == "fused")
    assert count(plain) == 2 and count(re) == 1
    rng = np.random.default_rng(1)
    feed = {"y": rng.uniform(-2, 2, 16 * 256), "p": rng.uniform(-2, 2, 256)}
    assert _semantics(g, plain["graph"], plain["origin"], feed)
    assert _semantics(g, re["graph"], re["origin"], feed)


def test_every_golden_graph_lowers_with_loads_proved_in_bounds(golden_cases, tool):
    """lowerMI355X proves every gather and operand load in bounds or throws; every golden
    graph, fused and unfused, must lower."""
    for c in golden_cases:
        for fz in (None, {"keep": c["outputs"]}):
            req = {"graph": c["graph"]}
            if fz:
                req["fuse"] = fz
            out = tool("lower", req)
            assert len(out["launches"]) >= 1
            for l in out["launches"]:
                assert len(l["params"]) <= 48
                for k in l["kernels"]:
                    assert all(g >= 1 for g in k["grid"]) and k["block"][0] in (64, 256)


def test_c2_programs_are_fully_judgeable(tool):
    """Config 2's generator keeps every element of every program (forward and gradient)
    judgeable: finite values inside float32's range and finite bounds."""
    from oracle import bounds
    progs = tool("chain-graphs", {"seeds": list(range(16)), "R": 32, "C": 1024})
    rng = np.random.default_rng(7)
    for p in progs:
        feed = {"x0": rng.standard_normal(32 * 1024), "x1": rng.standard_normal(32 * 1024),
                "r": rng.standard_normal(1024), "d0": rng.standard_normal(32 * 1024)}
        for kind in ("forward", "gradient"):
            v = p[kind]
            ref = bounds.streaming_reference(v["graph"], feed, v["keep"])
            vals = [ref[k][0] for k in v["keep"]]
            bnds = [ref[k][1] for k in v["keep"]]
            assert bounds.unjudgeable_count(vals, bnds) == 0, (p["seed"], kind, p["ops"])
            assert 8 <= len(p["ops"]) <= 16


def test_generated_kernels_read_no_parameter_block(golden_cases, tool):
    """Every size a kernel uses is a constant of its text: no generated source reads the
    parameter block (a layout mismatch there once sent a split-K matmul out of bounds)."""
    import re
    graphs = [{"graph": c["graph"]} for c in golden_cases[:40]]
    graphs.append({"graph": golden_cases[0]["graph"], "fuse": {"keep": golden_cases[0]["outputs"]}})
    progs = tool("chain-graphs", {"seeds": [0, 1], "R": 64, "C": 1024})
    for p in progs:
        graphs.append({"graph": p["gradient"]["graph"], "fuse": {"keep": p["gradient"]["keep"]}})
    for req in graphs:
        out = tool("lower", dict(req, sources=True))
        for l in out["launches"]:
            for k in l["kernels"]:
                assert not re.search(r"\.P\[", k["source"]), k["name"]


def _mixed_radix(n, factors):
    """Offsets of indices 0..n-1 over factors [[extent, stride], ...] (outer to inner)."""
    x = np.arange(n, dtype=np.int64)
    off = np.zeros(n, dtype=np.int64)
    inner = 1
    for e, st in reversed(factors):
        off += ((x // inner) % e) * st
        inner *= e
    assert inner == n or n == 1, (n, factors)
    return off


def _chain_value(graph, operand, source, src_value):
    """The operand's value from its source through the transpose/reshape chain between them
    (and the relu a view applies on load), by the oracle's kernels."""
    from oracle import interp
    chain = []
    cur = operand
    while cur != source:
        node = graph["nodes"][cur]
        assert node["op"] in ("transpose", "reshape", "relu"), node["op"]
        chain.append(node)
        cur = node["inputs"][0]
    v = src_value
    for node in reversed(chain):
        v = interp.kernel(node, [v], graph)
    return v


@pytest.mark.parametrize("req", [{"model": "mlp"}, {"model": "transformer", "B": 2}, {"model": "transformer-ref"}])
def test_perf_lowering_views_address_the_operands(tool, req):
    """The perf lowering skips only reshapes (sharing their input's buffer), transposes
    whose every consumer is a matmul operand slot, broadcasts read by bodies, and the
    nodes no kept value depends on (dead); each matmul operand it reads in place
    is addressed by its strided view exactly as the transpose chain would have laid it out
    (checked element by element on distinct values), and the load mode matches the view."""
    d = tool("perf-lower", req)
    g = d["graph"]
    nodes = g["nodes"]
    for a, src in d["aliases"]:
        assert nodes[a]["op"] == "reshape" and nodes[src]["op"] != "reshape"
    # Folded: transposes read in place by matmuls, broadcasts read through their index map,
    # and row reductions taken into the row-statistics chains that read them.
    reductions = {f["reduction"] for fs in d["rowFolds"].values() for f in fs}
    producers = {f["producer"] for fs in d["rowFolds"].values() for f in fs if "producer" in f}
    absorbed = set()
    # Values formed by their readers: an elementwise, gather, rowwise or row-statistics value
    # or a last-axis reduction (with what its own launch folds or absorbs) that every
    # launch reading it forms.
    formed, formers, value_absorbs = set(), {}, []
    for reader, records in d["formed"].items():
        for f in records:
            formed.add(f["value"])
            formers.setdefault(f["value"], set()).add(int(reader))
            for x in f.get("rowFolds") or []:
                reductions.add(x["reduction"])
                if "producer" in x:
                    producers.add(x["producer"])
            if f.get("absorbed"):
                value_absorbs.append((f["absorbed"], f["value"]))

    takers = {}

    def walk(records, reader):
        for a in records:
            # An absorbed producer: an elementwise node its reader reads at `pos`, kept by
            # nobody; every live reader of it forms it (checked below).
            p = nodes[a["producer"]]
            assert all(nodes[reader]["inputs"][q] == a["producer"] for q in a["pos"])
            assert p["op"] in ELEMENTWISE or (p["op"] == "fused" and p["attrs"]["kind"] == "elementwise")
            assert a["producer"] not in d["keep"] and a["producerPos"][0] == a["pos"][0]
            takers.setdefault(a["producer"], set()).add(reader)
            absorbed.add(a["producer"])
            walk(a.get("absorbed", []), a["producer"])
    consumers = {}
    for n_id, n in enumerate(nodes):
        for i in n["inputs"]:
            consumers.setdefault(i, set()).add(n_id)
    for reader, records in d["absorbed"].items():
        walk(records, int(reader))
    for records, value in value_absorbs:
        walk(records, value)
    # A producer formed in place is formed by every live reader of it (a launch, or a
    # producer formed in place in turn): nothing reads a buffer it would have written.
    for prod, by in takers.items():
        assert consumers[prod] - set(d["dead"]) == by, (prod, by)
    if req["model"] != "mlp":
        assert absorbed
    # Relus applied by the matmuls that read them, as they load them: every launched reader
    # of such a relu reads it as a matmul operand through a view that names it.
    on_load = {}
    for reader, ops in d["loadOps"].items():
        for o in ops:
            assert nodes[o["node"]]["op"] == "relu" and o["op"] == "relu" and o["source"] == nodes[o["node"]]["inputs"][0]
            on_load.setdefault(o["node"], set()).add(int(reader))
    if req["model"] == "transformer":
        assert len(on_load) == 4
    for relu, readers in on_load.items():
        assert relu not in d["keep"]
        for l in d["launches"]:
            named = any(v.get("opNode") == relu for v in (l["views"] or {}).values())
            assert named == (l["node"] in readers), (relu, l["node"])
    assert all(nodes[i]["op"] in ("transpose", "broadcast")
               for i in set(d["folded"]) - reductions - producers - absorbed - set(on_load) - formed)
    # A formed value is kept by nobody, and formed by exactly the launches that stand for its
    # live consumers: a launched consumer itself; for one that launches nothing (a
    # broadcast read in place, a reshape sharing a buffer, a folded reduction or producer,
    # another formed value), the launches standing for its own consumers.
    launched = {x["node"] for x in d["launches"]}
    aliased = {a for a, _ in d["aliases"]}

    def standing(c):
        if c in launched:
            return {c}
        assert c in d["folded"] or c in aliased, c
        return set().union(*[standing(x) for x in consumers.get(c, set()) - set(d["dead"])])
    for v, by in formers.items():
        assert v not in d["keep"] and (nodes[v]["op"] in ("sum", "max", "fused", "broadcast", "transpose")
                                       or nodes[v]["op"] in ELEMENTWISE)
        assert not any(src == v and a in d["keep"] for a, src in d["aliases"]), v
        readers = set().union(*[standing(c) for c in consumers[v] - set(d["dead"])])
        assert readers == by, (v, readers, by)
    if req["model"] == "transformer":
        assert len(formed) >= 40, len(formed)
    # A folded broadcast is read by elementwise, rowwise or epilogue bodies only (never
    # by a reduction, a gather or as a matmul operand), through the broadcast's source.
    for chain, fs in d["rowFolds"].items():
        c = nodes[int(chain)]
        assert (c["op"] == "fused" and c["attrs"]["kind"] == "elementwise") or c["op"] in ELEMENTWISE
        for f in fs:
            r = nodes[f["reduction"]]
            assert r["op"] in ("sum", "max") and r["shape"] != nodes[r["inputs"][0]]["shape"]
            assert f["reduction"] not in d["keep"] and all(c["inputs"][p] == f["reduction"] for p in f["pos"])
            # Every launched consumer of a folded reduction takes it in.
            assert all(str(u) in d["rowFolds"] or u in formed for u in consumers[f["reduction"]] if u not in d["dead"])
            if "producer" in f:
                # A producer formed in the launch: an elementwise node of the reduction's
                # 2-D operand shape, read by the reduction alone, kept by nobody.
                p = nodes[f["producer"]]
                assert r["inputs"][0] == f["producer"] and consumers[f["producer"]] == {f["reduction"]}
                assert f["producer"] not in d["keep"] and len(p["shape"]) == 2
                assert p["op"] in ELEMENTWISE or (p["op"] == "fused" and p["attrs"]["kind"] == "elementwise")
                assert f["producerPos"][0] == f["pos"][0] and len(f["producerPos"]) == len(p["inputs"])
    if req["model"] != "mlp":
        assert producers
    for i in d["folded"]:
        # A broadcast read in place (one that is formed by its readers is checked above).
        if nodes[i]["op"] == "broadcast" and i not in formed:
            for c in consumers[i]:
                assert nodes[c]["op"] == "fused" or nodes[c]["op"] in ELEMENTWISE, nodes[c]["op"]
    # Dead nodes: exactly those no kept node depends on (liveness recomputed here).
    live = set()
    for n_id in range(len(nodes) - 1, -1, -1):
        if n_id in d["keep"] or nodes[n_id]["op"] in ("input", "const") or consumers.get(n_id, set()) & live:
            live.add(n_id)
    assert set(d["dead"]) == {n_id for n_id in range(len(nodes)) if n_id not in live}
    launched = {l["node"] for l in d["launches"]}
    skipped = {a for a, _ in d["aliases"]} | set(d["folded"]) | set(d["dead"])
    assert launched.isdisjoint(skipped)
    assert launched | skipped == {n_id for n_id, n in enumerate(nodes) if n["op"] not in ("input", "const")}
    checked = mapped = 0
    for l in d["launches"]:
        for i in l["inputs"]:
            assert i not in skipped, (l["node"], i)
        for slot, v in (l["views"] or {}).items():
            shape = nodes[v["operand"]]["shape"]
            src_shape = nodes[v["source"]]["shape"]
            src = np.arange(int(np.prod(src_shape)), dtype=np.float64)
            want = _chain_value(g, v["operand"], v["source"], src).reshape(shape)
            view = v["view"]
            R, C = shape[-2], shape[-1]
            nb = int(np.prod(shape[:-2]))
            # Every index decoded over the view's mixed-radix factors: the flattened batch
            # index over view["batch"], the row and column over their own factors (or the
            # single strides sr and sc), outer to inner.
            rf = view.get("r") or [[R, view["sr"]]]
            cf = view.get("c") or [[C, view["sc"]]]
            idx = (_mixed_radix(nb, view["batch"])[:, None, None] + _mixed_radix(R, rf)[None, :, None]
                   + _mixed_radix(C, cf)[None, None, :]).reshape(shape)
            assert np.array_equal(src[idx], want), (l["node"], slot)
            mode = l["modes"][0 if slot == "a" else 1]
            strides4 = all(st % 4 == 0 for e, st in view["batch"] + rf[:-1] + cf[:-1] if e > 1)
            if cf[-1][1] == 1 and cf[-1][0] % 4 == 0 and C % 4 == 0 and strides4 and all(st % 4 == 0 for e, st in rf if e > 1):
                assert mode == 0
            elif rf[-1][1] == 1 and rf[-1][0] % 4 == 0 and R % 4 == 0 and strides4 and all(st % 4 == 0 for e, st in cf if e > 1):
                assert mode == 1
            if "r" in view:
                mapped += 1
            checked += 1
    if req["model"] != "mlp":
        assert checked > 10
    if req["model"] == "transformer":
        # The heads merged back into rows (and the head gradients on their way back) are read
        # through mapped views, not materialised.
        assert mapped >= 8
    # Every matmul splits K exactly as in the plain lowering (the same order of the K sum).
    splits = [l["split"] for l in d["launches"] if l["split"] is not None]
    assert splits, "no matmul's K split was read from its kernel"
    for l in d["launches"]:
        assert l["split"] == l["plainSplit"], (l["node"], l["split"], l["plainSplit"])


def test_perf_lowering_keeps_the_split_of_config4_backward(tool):
    """Config 4's gradient graphs at full size: the transposed weight-gradient matmuls read in
    place keep the plain lowering's K split, so their bits are the same."""
    graphs = tool("config-graphs", {"c4": [{"act": "relu", "M": M, "K": K, "N": N}
                                           for M, K, N in ((512, 512, 512), (4096, 4096, 4096), (8192, 1024, 4096))]})["c4"]
    for g in graphs:
        d = tool("perf-lower", {"graph": g["gradient"]["graph"], "keep": g["gradient"]["keep"]})
        nodes = d["graph"]["nodes"]
        assert sum(nodes[i]["op"] == "transpose" for i in d["folded"]) == 2   # transpose(W), transpose(X)
        # Only the weight gradient over M = 8192 rows (a long K for few output tiles) splits.
        chunks = sorted(l["split"][0] for l in d["launches"] if l["split"] is not None)
        assert chunks == ([1, 1, 4] if g["M"] == 8192 else [1, 1, 1]), (g["M"], chunks)
        for l in d["launches"]:
            assert l["split"] == l["plainSplit"], (g["M"], g["K"], g["N"], l["node"])


def test_row_fold_takes_in_a_producer_only_with_a_full_size_body(tool):
    """A row reduction's elementwise producer joins the reduction's rowwise launch only when
    every value of its body is full size (besides its operands, constants and their
    broadcasts): the rowwise kernel tells a row's value from an element's by size, so with as
    many rows as their length a computed vector of the row length would be read at the row
    index. The GPU corpus run with recompute found it (program 25's gradient: exp and log of
    a [1, 3] vector broadcast over [3, 3], read at the row index). Here the same graph fused
    plainly leaves the vector's exp and log a launch of their own and the producer folds;
    with recompute they move into the producer, which then stays a launch."""
    def node(op, inputs, out_shape, **attrs):
        return {"op": op, "inputs": inputs, "attrs": attrs, "shape": out_shape}
    nodes = [node("input", [], [1, 3], name="v", shape=[1, 3]), node("input", [], [3, 3], name="m", shape=[3, 3]),
             node("exp", [0], [1, 3]), node("log", [2], [1, 3]), node("broadcast", [3], [3, 3], shape=[3, 3]),
             node("mul", [1, 4], [3, 3]), node("neg", [5], [3, 3]),
             node("sum", [6], [3, 1], axis=1, keepDims=True), node("neg", [7], [3, 1]), node("exp", [8], [3, 1])]
    for recompute in (False, True):
        d = tool("perf-lower", {"graph": {"nodes": nodes}, "keep": [9], "fuse": {"recompute": recompute}})
        g = d["graph"]["nodes"]
        (chain, folds), = d["rowFolds"].items()
        (f,) = folds
        assert g[f["reduction"]]["op"] == "sum"
        producer = g[f["reduction"]]["inputs"][0]
        body = g[producer]["attrs"]["body"]["nodes"]
        assert [b["op"] for b in body if b["op"] in ("exp", "log")] == (["exp", "log"] if recompute else [])
        assert ("producer" in f) != recompute and (producer in d["folded"]) != recompute
        assert (producer in [l["node"] for l in d["launches"]]) == recompute


def test_column_reduction_takes_in_a_producer_only_where_its_maps_fit(tool):
    """A column reduction forms its operand's producer in place (the trainer's lowering),
    the producer's index maps appended to the launch's five size words. With four
    transposed rank-4 operands the maps fit one argument block (41 of 48 words) and the
    producer is taken in; with five (50 words) it is not: the producer stays a launch of
    its own and the reduction reads its value. Counting only the producer's words would
    pass the second at lowering and fail it at launch."""
    def graph(k):
        nodes, acc = [], None
        for j in range(k):
            nodes.append({"op": "input", "inputs": [], "attrs": {"name": f"x{j}", "shape": [2, 3, 4, 8]}, "shape": [2, 3, 4, 8]})
            nodes.append({"op": "transpose", "inputs": [len(nodes) - 1], "attrs": {"perm": [3, 2, 1, 0]}, "shape": [8, 4, 3, 2]})
            t = len(nodes) - 1
            if acc is not None:
                nodes.append({"op": "add", "inputs": [acc, t], "attrs": {}, "shape": [8, 4, 3, 2]})
                t = len(nodes) - 1
            acc = t
        nodes.append({"op": "sum", "inputs": [acc], "attrs": {"axis": 0}, "shape": [4, 3, 2]})
        return {"nodes": nodes}, len(nodes) - 1
    for k, taken in ((4, True), (5, False)):
        g, s = graph(k)
        d = tool("perf-lower", {"graph": g, "keep": [s], "fuse": {}, "absorb": True})
        kinds = [x["kind"] for x in d["launches"]]
        assert ("fused-elementwise" not in kinds) == taken, kinds
        assert bool(d["absorbed"]) == taken
        assert all(x["params"] <= 48 for x in d["launches"])


def _product_shape(nodes, n):
    """(batch dims, M, K, N) of a plain matmul node or of an epilogue group's matmul, or None."""
    if n["op"] == "matmul":
        a, b = (nodes[i]["shape"] for i in n["inputs"])
    elif n["op"] == "fused" and n["attrs"]["kind"] == "epilogue":
        body = n["attrs"]["body"]["nodes"]
        mm = next(x for x in body if x["op"] == "matmul")
        a, b = (body[i]["shape"] for i in mm["inputs"])
    else:
        return None
    return (tuple(a[:-2]), a[-2], a[-1], b[-1])


def _splits_by_product(d):
    """{(shape, read by a node): [chunks of each launch]} of a perf-lower result."""
    nodes = d["graph"]["nodes"]
    read = {i for n in nodes for i in n["inputs"]}
    out = {}
    for l in d["launches"]:
        shape = _product_shape(nodes, nodes[l["node"]])
        if shape is not None and l["split"] is not None:
            out.setdefault((shape, l["node"] in read), []).append(l["split"][0])
    return out


def test_k_split_shares_the_chip_only_among_products_no_node_reads(tool):
    """A product whose value no node reads (a weight gradient with its update epilogue) may
    share one dispatch with the others of its shape, so its K split aims at the chip over all
    of them; a product that a node reads splits as it would alone. Config 5's step at batch
    64: the 16 fused attention-projection weight gradients (256 x 8192 x 256, nothing reads
    them) split alike, into fewer chunks than the same products of the unfused step, which
    the separate updates read; those split as the product does alone in a graph of its own."""
    fused = _splits_by_product(tool("perf-lower", {"model": "transformer", "B": 64}))
    unfused = _splits_by_product(tool("perf-lower", {"model": "transformer", "B": 64, "unfused": True}))
    wgrad = ((), 256, 8192, 256)
    assert len(fused[(wgrad, False)]) == 16 and len(set(fused[(wgrad, False)])) == 1
    assert (wgrad, True) not in fused
    assert len(unfused[(wgrad, True)]) == 16 and (wgrad, False) not in unfused
    nodes = [{"op": "input", "inputs": [], "attrs": {"name": "a", "shape": [256, 8192]}, "shape": [256, 8192]},
             {"op": "input", "inputs": [], "attrs": {"name": "b", "shape": [8192, 256]}, "shape": [8192, 256]},
             {"op": "matmul", "inputs": [0, 1], "attrs": {}, "shape": [256, 256]}]
    alone = _splits_by_product(tool("perf-lower", {"graph": {"nodes": nodes}, "keep": [2]}))[(wgrad, False)]
    assert set(unfused[(wgrad, True)]) == set(alone)
    assert fused[(wgrad, False)][0] < alone[0]


@pytest.mark.parametrize("config,V,B,layers", [("reference", 16, 2, 2), ("c5", 96, 1, 4)])
def test_attention_fusion_preserves_semantics(tool, config, V, B, layers):
    """The attention extension (fuse(..., {attention: true}), off by default): every
    attention of the transformer's forward pass (matmul(Q, Kt) -> the softmax group ->
    matmul(P, V)) becomes one fused node, the float64 interpreter evaluates the fused
    graph bitwise equal at every surviving node, and the contract's own fusion of the
    same graph is unchanged by the option being available."""
    fw = tool("transformer-forward", {"config": config, "V": V, "B": B})
    plain, att = tool("fuse", {"graphs": [{"name": "p", "graph": fw["graph"], "keep": fw["keep"]},
                                          {"name": "a", "graph": fw["graph"], "keep": fw["keep"], "attention": True}]})
    kinds = lambda f: [n["attrs"]["kind"] for n in f["graph"]["nodes"] if n["op"] == "fused"]
    assert kinds(att).count("attention") == layers
    assert "attention" not in kinds(plain)
    assert kinds(plain).count("rowwise") - kinds(att).count("rowwise") == layers   # each softmax group absorbed
    launched = lambda f: sum(1 for n in f["graph"]["nodes"] if n["op"] not in ("input", "const"))
    assert launched(plain) - launched(att) == 2 * layers
    assert _semantics(fw["graph"], att["graph"], att["origin"], fw["inputs"])
    for n in att["graph"]["nodes"]:
        if n["op"] == "fused" and n["attrs"]["kind"] == "attention":
            ops = [b["op"] for b in n["attrs"]["body"]["nodes"]]
            assert ops.count("matmul") == 2 and ops.count("max") == 1 and ops.count("exp") == 1


def test_attention_fusion_leaves_training_steps_and_golden_cases_alone(golden_cases, tool):
    """In a training step the probabilities also feed the backward pass, so no attention
    fuses there; on every golden case the option keeps fusion semantics bitwise."""
    fw = tool("transformer-forward", {"config": "reference", "V": 16, "B": 1})
    g = tool("grad", {"cases": [{"name": "t", "graph": fw["graph"], "outputs": [fw["keep"][1]]}]})[0]
    step = tool("fuse", {"graphs": [{"name": "s", "graph": g["graph"], "keep": [fw["keep"][1]] + g["grads"], "attention": True}]})[0]
    assert not any(n["op"] == "fused" and n["attrs"]["kind"] == "attention" for n in step["graph"]["nodes"])
    reqs = [{"name": c["name"], "graph": c["graph"], "keep": c["outputs"], "attention": True} for c in golden_cases]
    fused = tool("fuse", {"graphs": reqs})
    for c, f in zip(golden_cases, fused):
        assert "error" not in f, (c["name"], f.get("error"))
        assert _semantics(c["graph"], f["graph"], f["origin"], c["inputs"]), c["name"]


def test_recomputed_epilogue_reads_its_product_through_the_workspace(tool):
    """A group formed with recomputation can reach its matmul through a transpose
    (x·w, scaled, transposed, added to a residual): the store of element i needs the
    product at another index, which the epilogue's accumulator does not hold. The
    lowering forms the product in the workspace first (the split-K form, one chunk) and
    the second kernel reads element j's sum there; the plain matmul of the same shape
    keeps its one-kernel form. (Corpus program 89's gradient has such a group; the GPU
    test of recomputed corpus programs judges it.)"""
    def inp(name, shape):
        return {"op": "input", "inputs": [], "attrs": {"name": name, "shape": shape}, "shape": shape}
    g = {"nodes": [inp("x", [2, 4, 4]), inp("w", [2, 4, 2]), inp("s", [2, 4, 2]), inp("r", [2, 4, 2]),
                   {"op": "matmul", "inputs": [0, 1], "attrs": {}, "shape": [2, 4, 2]},
                   {"op": "mul", "inputs": [4, 2], "attrs": {}, "shape": [2, 4, 2]},
                   {"op": "transpose", "inputs": [5], "attrs": {"perm": [2, 1, 0]}, "shape": [2, 4, 2]},
                   {"op": "add", "inputs": [3, 6], "attrs": {}, "shape": [2, 4, 2]}]}
    plain = tool("lower", {"graph": g, "fuse": {"keep": [7]}, "sources": True})
    rec = tool("lower", {"graph": g, "fuse": {"keep": [7], "recompute": True}, "sources": True})
    # Without recomputation the transpose is a load of a stored product.
    assert [l["kind"] for l in plain["launches"]] == ["fused-epilogue", "fused-elementwise"]
    assert all("gemm_product_at" not in k["source"] for l in plain["launches"] for k in l["kernels"])
    (epi,) = [l for l in rec["launches"] if l["kind"] == "fused-epilogue"]
    assert len(rec["launches"]) == 1 and len(epi["kernels"]) == 2
    part, red = epi["kernels"]
    assert ", true, " in part["source"] and "gemm_product_at" in red["source"] and red["name"].endswith("_red")
    assert rec["workspace"] >= 2 * 4 * 2 * 4


def test_chain_maps_address_random_transpose_reshape_chains(tool):
    """The mixed-radix index maps of the perf lowering's mapped views (lower.js chainMap),
    against numpy on distinct values: random chains of transposes and reshapes over random
    shapes: where a map is given (about two thirds of them; the others hold a reshape that
    cuts a factor where neither extent divides the other), every element of the chain's
    value is found at the offset the map gives."""
    rng = np.random.default_rng(5)
    cases = []
    for _ in range(300):
        rank = int(rng.integers(2, 5))
        shape = [int(rng.choice([1, 2, 3, 4, 5, 6, 8])) for _ in range(rank)]
        chain, cur = [], list(shape)
        for _ in range(int(rng.integers(1, 5))):
            if rng.random() < 0.5:
                perm = [int(p) for p in rng.permutation(len(cur))]
                chain.append(["transpose", perm])
                cur = [cur[p] for p in perm]
            else:
                n = int(np.prod(cur))
                dims = []
                while n > 1:
                    d = int(rng.choice([f for f in range(2, n + 1) if n % f == 0]))
                    dims.append(d)
                    n //= d
                cur = dims or [1]
                chain.append(["reshape", cur])
        cases.append({"shape": shape, "chain": chain})
    res = tool("chain-map", {"cases": cases})
    mapped = 0
    for c, r in zip(cases, res):
        src = np.arange(int(np.prod(c["shape"]))).reshape(c["shape"])
        v = src
        for op, arg in c["chain"]:
            v = np.transpose(v, arg) if op == "transpose" else v.reshape(arg)
        assert list(v.shape) == r["shape"]
        if r["map"] is None:
            continue
        mapped += 1
        idx = np.zeros(v.shape, dtype=np.int64)
        for axis, factors in enumerate(r["map"]):
            sh = [1] * v.ndim
            sh[axis] = v.shape[axis]
            idx = idx + _mixed_radix(v.shape[axis], factors).reshape(sh)
        assert np.array_equal(src.reshape(-1)[idx], v), c
    assert mapped >= 150


@pytest.mark.parametrize("workload", ["step-V16-B8", "step-V75-B16"])
def test_formed_kernels_declare_each_name_once(tool, workload):
    """A rowwise kernel emits its row-tier statements (values computed once per row) phase
    by phase into the row loop's scope, so a name made from how many such lines are pending
    can come back in a later phase: the unfused training steps of the workload sweep,
    lowered with their row values formed by the launches reading them, once declared one
    row load twice (a compile error on the GPU). Every name a kernel declares is declared
    once (in a batched kernel whose members run different bodies, once in each member's
    case, a scope of its own)."""
    import re
    d = tool("perf-lower", {"workload": workload, "sources": True})
    assert d["formed"], "the case forms no values"
    for name, text in d["sources"].items():
        for src in re.split(r"\n\s*case \d+u: \{", text):
            declared = re.findall(r"\bconst float (\w+) =", src)
            loops = src.count("for (int s = 0;")
            # Names inside the element loops repeat per loop (their own scopes); row-tier
            # names (R...) and reduction results are declared once in the row loop.
            row = [x for x in declared if x.startswith("R") or x.startswith("red")]
            assert len(row) == len(set(row)), (name, sorted(x for x in row if row.count(x) > 1))
            assert loops > 0 or not row


def test_formation_prices_repeated_transcendentals(tool):
    """The perf lowering forms a value in its readers where its launch estimate (bytes at
    6 TB/s plus op-priced vector work plus a launch cost, added) does not rise. In config
    2's program 0 gradient at full size, the forward chain's last value (two exp and two
    tanh per element) is read by four launches: repeating it in each would cost more than
    its write and read-backs, so it stays a launch, and the cheaper values before it are
    formed in the launches that read them. With a flat count of repeated ops instead,
    all four readers once repeated the chain (28 us for a 100.7 MB kernel on the GPU)."""
    g = tool("config-graphs", {"c2": [{"seed": 0, "R": 8192, "C": 1024}]})["c2"][0]["gradient"]
    d = tool("perf-lower", {"graph": g["graph"], "keep": g["keep"], "fuse": {}})
    nodes = d["graph"]["nodes"]
    launched = {x["node"] for x in d["launches"]}
    formed = {f["value"] for fs in d["formed"].values() for f in fs}

    def ops(i):
        n = nodes[i]
        return [b["op"] for b in n["attrs"]["body"]["nodes"]] if n["op"] == "fused" else [n["op"]]
    readers = {}
    for i, n in enumerate(nodes):
        for x in n["inputs"]:
            readers.setdefault(x, set()).add(i)
    # A launch computes its own body and the values its record says it forms.
    def tanhs(i):
        return ops(i).count("tanh") + sum(ops(f["value"]).count("tanh") for f in d["formed"].get(str(i), []))
    chain = [i for i in launched if tanhs(i) >= 2 and len(readers.get(i, ())) >= 3]
    assert chain, "the shared transcendental chain is not a launch"
    assert formed, "nothing formed"
    # No launch repeats the chain: the launches reading the chain's value read it.
    for i in chain:
        assert i not in formed and all(str(r) not in d["formed"] or i not in {f["value"] for f in d["formed"][str(r)]}
                                       for r in readers[i])
