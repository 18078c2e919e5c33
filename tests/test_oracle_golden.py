"""The oracle pinned before it is trusted: the float64 interpreter against the
reference's PyTorch goldens and closed forms, the float32 bound against the
closed forms the reference's own tests state (test/gpu-bounds.test.js:35-114),
and the judges against planted errors."""
import json
import math

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import bounds, interp

TOL = 1e-12


def tensor_error(ours, ref):
    """The reference's v1 metric (src/testing/golden.js:24-34): max |a-b| / max |b|."""
    ours = np.asarray(ours, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ours.size != ref.size:
        return math.inf
    d = np.abs(ours - ref)
    if np.any(np.isnan(d)):
        return math.inf
    diff = float(d.max()) if d.size else 0.0
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    return 0.0 if diff == 0 else diff / max(scale, 1e-300)


def test_interpreter_forward_matches_torch_float64(golden_cases):
    for c in golden_cases:
        vals = interp.evaluate(c["graph"], c["inputs"])
        for k, out in enumerate(c["outputs"]):
            err = tensor_error(vals[out], c["torchOutputs"][k])
            assert err <= TOL, f"{c['name']} output {k}: {err}"


def test_interpreter_and_host_autodiff_match_torch_gradients(golden_cases, tool):
    """The host's grad() (JS) builds each case's gradient graph; the oracle evaluates it.
    random-9 (x0/x0, an exact zero gradient as rounding residue) is the one failure the
    reference records (test/golden.test.js:23-36); pinned to exactly that."""
    out = tool("grad", {"cases": [{"name": c["name"], "graph": c["graph"], "outputs": c["outputs"]} for c in golden_cases]})
    failing = []
    for c, g in zip(golden_cases, out):
        feed = dict(c["inputs"])
        for name, cot in zip(g["cotangents"], c["cotangents"]):
            feed[name] = cot
        vals = interp.evaluate(g["graph"], feed)
        names = [n["attrs"]["name"] for n in c["graph"]["nodes"] if n["op"] == "input"]
        errs = [tensor_error(vals[gid], c["torchGrads"][nm]) for nm, gid in zip(names, g["grads"])]
        if max(errs, default=0) > TOL:
            failing.append((c["name"], max(errs)))
            if c["name"] == "random-9":
                gd = max(float(np.abs(np.asarray(vals[gid]) - np.asarray(c["torchGrads"][nm])).max())
                         for nm, gid in zip(names, g["grads"]))
                assert gd < 1e-15
    assert [f[0] for f in failing] == ["random-9"], failing


def test_composites_match_torch_native(golden_cases):
    comps = [c for c in golden_cases if c["kind"] == "composite"]
    assert len(comps) == 9
    for c in comps:
        vals = interp.evaluate(c["graph"], c["inputs"])
        assert tensor_error(vals[c["outputs"][0]], c["torchNative"]["output"]) <= TOL, c["name"]


def _g(nodes):
    return {"nodes": nodes}


def _in(name, shape):
    return {"op": "input", "inputs": [], "attrs": {"name": name, "shape": shape}, "shape": shape}


def test_interpreter_closed_forms():
    """test/interp.test.js: matmul by hand, batched matmul, sums, maxes, softmax at 800."""
    g = _g([_in("a", [2, 3]), _in("b", [3, 2]), {"op": "matmul", "inputs": [0, 1], "attrs": {}, "shape": [2, 2]}])
    v = interp.evaluate(g, {"a": [1, 2, 3, 4, 5, 6], "b": [7, 8, 9, 10, 11, 12]})
    assert list(v[2]) == [58, 64, 139, 154]
    g = _g([_in("x", [2, 3]), {"op": "sum", "inputs": [0], "attrs": {"axis": 0, "keepDims": False}, "shape": [3]},
            {"op": "max", "inputs": [0], "attrs": {"axis": 1, "keepDims": True}, "shape": [2, 1]}])
    v = interp.evaluate(g, {"x": [1, -2, 3, 4, 5, -6]})
    assert list(v[1]) == [5, 3, -3] and list(v[2]) == [3, 5]
    # max ignores NaN as the reference's `v > acc ? v : acc` does.
    v = interp.evaluate(g, {"x": [float("nan"), 1, 2, 3, float("nan"), 0]})
    assert list(v[2]) == [2, 3]
    # a 3-cycle transpose and its inverse.
    g = _g([_in("x", [2, 3, 4]), {"op": "transpose", "inputs": [0], "attrs": {"perm": [2, 0, 1]}, "shape": [4, 2, 3]}])
    x = np.arange(24.0)
    v = interp.evaluate(g, {"x": x})
    assert np.array_equal(v[1], np.transpose(x.reshape(2, 3, 4), (2, 0, 1)).reshape(-1))


def test_sequential_summation_order_is_the_references():
    """Sums add first to last: (1e16 + 1) - 1e16 + ... differs from pairwise/sorted sums."""
    x = [1e16, 1.0, -1e16, 1.0]
    g = _g([_in("x", [4]), {"op": "sum", "inputs": [0], "attrs": {"axis": 0, "keepDims": False}, "shape": []}])
    assert interp.evaluate(g, {"x": x})[1][0] == ((1e16 + 1.0) + -1e16) + 1.0 == 1.0


def _single(op_nodes, inputs):
    g = _g(op_nodes)
    r = bounds.reference_with_bounds(g, inputs)
    return r["values"][-1], r["bounds"][-1]


U, EPS = 2.0 ** -24, 2.0 ** -23


def gamma(n):
    return n * U / (1 - n * U)


def close(a, b):
    assert abs(a - b) <= 1e-12 * abs(b), (a, b)


def test_bound_closed_forms():
    """Each per-op constant of the float32 budget (gpu-bounds.test.js:35-62)."""
    ab = lambda op, s=[1]: [_in("a", s), _in("b", s), {"op": op, "inputs": [0, 1], "attrs": {}, "shape": s}]
    un = lambda op, s: [_in("x", s), {"op": op, "inputs": [0], "attrs": {}, "shape": s}]
    v, e = _single(ab("add"), {"a": [1.5], "b": [2.25]})
    close(e[0], U * 3.75)
    v, e = _single(ab("div"), {"a": [1], "b": [3]})
    close(e[0], 2.5 * EPS * abs(v[0]))
    v, e = _single(un("exp", [1]), {"x": [2]})
    close(e[0], (3 + 2 * 2) * EPS * math.exp(2))
    v, e = _single(un("log", [2]), {"x": [1.5, 100]})
    close(e[0], 2.0 ** -21)
    close(e[1], 3 * EPS * abs(v[1]))
    v, e = _single(un("tanh", [2]), {"x": [0.5, 30]})
    close(e[0], 1e-5)
    close(e[1], (9.5 + 4 * 30) * EPS)
    v, e = _single([_in("x", [4]), {"op": "sum", "inputs": [0], "attrs": {"axis": 0, "keepDims": False}, "shape": []}],
                   {"x": [1, -2, 3, -4]})
    close(e[0], gamma(4) * 10)
    v, e = _single([_in("a", [1, 2]), _in("b", [2, 1]), {"op": "matmul", "inputs": [0, 1], "attrs": {}, "shape": [1, 1]}],
                   {"a": [1, -2], "b": [3, 4]})
    close(e[0], gamma(2) * (3 + 8))
    v, e = _single([_in("x", [2, 3]), {"op": "transpose", "inputs": [0], "attrs": {"perm": [1, 0]}, "shape": [3, 2]}],
                   {"x": [1, 2, 3, 4, 5, 6]})
    assert list(e) == [0] * 6
    v, e = _single([_in("x", [3]), {"op": "max", "inputs": [0], "attrs": {"axis": 0, "keepDims": False}, "shape": []}],
                   {"x": [1, 7, 3]})
    assert list(e) == [0]


def test_bound_inputs_rounded_and_subnormal_flush():
    g = _g([_in("x", [1]), {"op": "const", "inputs": [], "attrs": {"shape": [], "value": 0.1}, "shape": []},
            {"op": "broadcast", "inputs": [1], "attrs": {"shape": [1]}, "shape": [1]},
            {"op": "add", "inputs": [0, 2], "attrs": {}, "shape": [1]}])
    r = bounds.reference_with_bounds(g, {"x": [0.1]})
    f = float(np.float32(0.1))
    assert r["inputs"]["x"][0] == f and r["values"][3][0] == f + f
    v, e = _single([_in("a", [1]), _in("b", [1]), {"op": "mul", "inputs": [0, 1], "attrs": {}, "shape": [1]}],
                   {"a": [1e-20], "b": [1e-20]})
    assert v[0] != 0 and abs(v[0]) < 2.0 ** -126 and e[0] >= 2.0 ** -126


def test_bound_step_flip_and_unbounded_division():
    # x + 1e-8 - 1e-8 carries rounding error; step at 1e-17 may flip (bound 1), at 1 not.
    g = _g([_in("x", [2]),
            {"op": "const", "inputs": [], "attrs": {"shape": [], "value": 1e-8}, "shape": []},
            {"op": "broadcast", "inputs": [1], "attrs": {"shape": [2]}, "shape": [2]},
            {"op": "add", "inputs": [0, 2], "attrs": {}, "shape": [2]},
            {"op": "sub", "inputs": [3, 2], "attrs": {}, "shape": [2]},
            {"op": "step", "inputs": [4], "attrs": {}, "shape": [2]}])
    r = bounds.reference_with_bounds(g, {"x": [1e-17, 1]})
    assert list(r["bounds"][5]) == [1, 0]
    g = _g([_in("a", [1]), _in("b", [1]),
            {"op": "const", "inputs": [], "attrs": {"shape": [1], "value": 1}, "shape": [1]},
            {"op": "sub", "inputs": [1, 2], "attrs": {}, "shape": [1]},
            {"op": "div", "inputs": [0, 3], "attrs": {}, "shape": [1]}])
    r = bounds.reference_with_bounds(g, {"a": [1], "b": [1]})
    assert r["bounds"][4][0] == math.inf
    assert bounds.unjudgeable_count(r["values"], r["bounds"]) >= 1


def test_bound_random9_cancelled_gradient(tool):
    """x / x has gradient exactly zero; its bound is set by g/x and -g*x/(x*x)
    (gpu-bounds.test.js:70-84): between 3 and 12 EPS * |g/x|."""
    g = _g([_in("x", [3]), {"op": "div", "inputs": [0, 0], "attrs": {}, "shape": [3]}])
    G = tool("grad", {"cases": [{"name": "r9", "graph": g, "outputs": [1]}]})[0]
    xs, gs = [0.3, -1.7, 1.2], [0.5, -0.25, 1]
    r = bounds.reference_with_bounds(G["graph"], {"x": xs, "d0": gs})
    gid = G["grads"][0]
    assert list(r["values"][gid]) == [0, 0, 0]
    for b, x, gg in zip(r["bounds"][gid], xs, gs):
        term = abs(float(np.float32(gg)) / float(np.float32(x)))
        assert 3 * EPS * term < b < 12 * EPS * term


def test_judge_catches_planted_errors():
    g = _g([_in("x", [2]), {"op": "add", "inputs": [0, 0], "attrs": {}, "shape": [2]}])
    r = bounds.reference_with_bounds(g, {"x": [1, 2]})
    ok = bounds.judge(g, [r["values"][0], r["values"][1].astype(np.float32)], r["values"], r["bounds"])
    assert ok["pass"]
    moved = r["values"][0].copy()
    moved[1] += 1e-12
    bad = bounds.judge(g, [moved, r["values"][1]], r["values"], r["bounds"])
    assert not bad["pass"] and bad["first"]["node"] == 0
    # A value off by more than 2E fails; within it passes.
    e = r["bounds"][1][0]
    assert not bounds.judge(g, [r["values"][0], r["values"][1] + 2.01 * e], r["values"], r["bounds"])["pass"]
    assert bounds.judge(g, [r["values"][0], r["values"][1] + 1.99 * e], r["values"], r["bounds"])["pass"]
    # NaN never passes.
    assert not bounds.judge(g, [r["values"][0], np.array([np.nan, 4.0])], r["values"], r["bounds"])["pass"]


def test_transformer_init_matches_torch_m3b(tool):
    """The reference transformer (V 16, B 4, T 64, d 64, L 2, GELU) at golden-seed1's
    initialisation on its first batch: the host builder + autodiff + the oracle's float64
    evaluation against golden/torch-m3b.f64 (logits, loss, every gradient) at 1e-10, and
    the parameters drawn by the host's RNG hash to the spec's initSha."""
    import hashlib
    import struct
    meta = json.loads((GOLDEN / "transformer_init.json").read_text())
    blob = np.fromfile(GOLDEN / "transformer_init.f64", dtype="<f8")
    t = tool("transformer-init", {"V": meta["V"], "batch": meta["batch"], "seed": meta["seed"], "firstBatch": meta["firstBatch"]})
    h = hashlib.sha256()
    for name in t["names"]:
        a = t["params"][name]
        h.update(struct.pack(f"<{len(a)}d", *a))
    assert h.hexdigest() == meta["initSha"]
    feed = dict(t["params"])
    feed["x"], feed["y"] = t["x"], t["y"]
    feed[t["cotangent"]] = [1.0]
    vals = interp.evaluate(t["graph"], feed)
    ten = lambda k: blob[meta["tensors"][k][0]: meta["tensors"][k][0] + meta["tensors"][k][1]]
    assert tensor_error(vals[t["logits"]], ten("logits")) <= 1e-10
    assert abs(vals[t["loss"]][0] - meta["loss"]) <= 1e-10 * abs(meta["loss"])
    for name, gid in zip(t["names"], t["grads"]):
        assert tensor_error(vals[gid], ten(f"grad/{name}")) <= 1e-10, name


def test_blas_matmul_block_stays_within_the_order_bound(golden_cases):
    """interp.blas_matmul(): the large products of the full-size training steps summed in
    the BLAS's order. Against the ordered sum, each element differs by at most
    2*gamma64(K)*sum|a||b| (two float64 orders of one sum, each within gamma64(K) of the
    exact value), and every golden case still matches torch float64 at 1e-12 with
    every product sent to the BLAS."""
    rng = np.random.default_rng(17)
    u64 = 2.0 ** -53
    for (bt, m, k, n) in [(1, 3, 1, 5), (1, 17, 7, 9), (2, 64, 256, 96), (1, 128, 1024, 64), (4, 32, 4096, 8)]:
        a = rng.normal(size=bt * m * k) * rng.choice([1e-3, 1, 1e3], size=bt * m * k)
        b = rng.normal(size=bt * k * n)
        sa, sb = ([bt, m, k] if bt > 1 else [m, k]), ([bt, k, n] if bt > 1 else [k, n])
        ordered = interp.k_matmul(a, b, sa, sb)
        with interp.blas_matmul(0):
            fast = interp.k_matmul(a, b, sa, sb)
        mass = interp.k_matmul(np.abs(a), np.abs(b), sa, sb)
        g = k * u64 / (1 - k * u64)
        assert np.all(np.abs(fast - ordered) <= 2 * g * mass), (bt, m, k, n)
        # The ordered sum really is p ascending: equal to an explicit loop on one element.
        A, B = a.reshape(bt, m, k), b.reshape(bt, k, n)
        acc = 0.0
        for p in range(k):
            acc = acc + A[-1, -1, p] * B[-1, p, -1]
        assert ordered[-1] == acc
    with interp.blas_matmul(0):
        for c in golden_cases:
            vals = interp.evaluate(c["graph"], c["inputs"])
            for j, out in enumerate(c["outputs"]):
                assert tensor_error(vals[out], c["torchOutputs"][j]) <= TOL, (c["name"], j)
