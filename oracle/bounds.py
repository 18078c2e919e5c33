"""The float32 error budget — TEST INFRASTRUCTURE ONLY (the checker, never the product).

Restates src/gpu/bounds.js of abho7/tensor-compiler-webgpu: a float64 value for
every node, computed from float32-rounded inputs and constants, and beside it a
first-order bound E on the error a float32 evaluation may make, propagated node
by node from the per-op accuracy the reference pre-registered (bounds.js:25-55;
derived from the WGSL specification: exp (3+2|x|) ulp, log 3 ulp or 2^-21
absolute, tanh max(1e-5, ...), div 2.5 ulp, sqrt 4.5 ulp, flush-to-zero allowed).
A GPU value passes when |gpu - ref| <= S * E with S = 2 (judge, bounds.js:155-171).

Also restated: unjudgeable (:139-148), the fused judge judgeFused and the
node-local pair localReferenceFused / judgeLocal (src/gpu/harness-m4.js:46-60,
182-223), the streaming outputs judge judgeOutputs (src/fusion/workloads.js:351-374).

Parity pins (tests/test_oracle_golden.py): the closed forms of
test/gpu-bounds.test.js:35-114 (add U*3.75, div 2.5*EPS*|r|, exp (3+2*2)*EPS*e^2,
log 2^-21 at 1.5 and 3*EPS*|r| at 100, tanh 1e-5 at 0.5 and (9.5+4*30)*EPS at 30,
sum gamma(4)*10, matmul gamma(2)*11, transpose/max 0, step flip 1, division by a
cancelled value unbounded), each chosen so a dropped term or wrong constant fails.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import numpy as np

from . import interp

S = 2.0
U = 2.0 ** -24
EPS = 2.0 ** -23
TAU = 2.0 ** -126
F32_MAX = 3.4028234663852886e38


def gamma(n: float) -> float:
    return (n * U) / (1 - n * U)


def fround(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float64)


def ftz(r: np.ndarray) -> np.ndarray:
    return np.where((r != 0) & (np.abs(r) < TAU), TAU, 0.0)


def _elementwise_bound(op: str, r, args, errs):
    a = np.abs
    if op in ("add", "sub"):
        return errs[0] + errs[1] + U * a(r)
    if op == "mul":
        x, y = args
        ex, ey = errs
        return a(y) * ex + a(x) * ey + ex * ey + U * a(r)
    if op == "div":
        x, y = args
        ex, ey = errs
        m = a(y)
        bad = (ey >= m) | (m < 2.0 ** -126) | (m > 2.0 ** 126)
        with np.errstate(all="ignore"):
            v = (ex + a(r) * ey) / (m - ey) + 2.5 * EPS * a(r)
        return np.where(bad, np.inf, v)
    if op in ("neg", "relu", "stopGradient"):
        return errs[0].copy()
    if op == "exp":
        x, ex = args[0], errs[0]
        grow = np.exp(ex)
        return a(r) * (grow - 1) + (3 + 2 * (a(x) + ex)) * EPS * a(r) * grow
    if op == "log":
        x, ex = args[0], errs[0]
        bad = ~(x > 0) | (ex >= x)
        with np.errstate(all="ignore"):
            inherited = -np.log1p(-ex / x)
            v = inherited + np.maximum(2.0 ** -21, 3 * EPS * (a(r) + inherited))
        return np.where(bad, np.inf, v)
    if op == "tanh":
        x, ex = args[0], errs[0]
        return ex + np.maximum(1e-5, (9.5 + 4 * (a(x) + ex)) * EPS)
    if op == "sqrt":
        x, ex = args[0], errs[0]
        with np.errstate(all="ignore"):
            inherited = np.where(x > 0, np.minimum(np.sqrt(ex), ex / np.sqrt(np.where(x > 0, x, 1.0))), np.sqrt(ex))
        return np.where(x < 0, np.inf, inherited + 4.5 * EPS * a(r))
    if op == "step":
        x, ex = args[0], errs[0]
        return np.where((ex > 0) & (a(x) <= ex), 1.0, 0.0)
    raise ValueError(f"no bound rule for '{op}'")


def _structured_bound(node, args, errs, graph):
    op = node["op"]
    nodes = graph["nodes"]
    if op == "sum":
        in_shape = nodes[node["inputs"][0]]["shape"]
        n = in_shape[node["attrs"]["axis"]]
        inherited = interp.k_sum(errs[0], in_shape, node["attrs"]["axis"])
        mass = interp.k_sum(np.abs(args[0]), in_shape, node["attrs"]["axis"])
        return inherited + gamma(n) * mass
    if op == "max":
        in_shape = nodes[node["inputs"][0]]["shape"]
        return interp.k_max(errs[0], in_shape, node["attrs"]["axis"])
    if op == "matmul":
        a_shape = nodes[node["inputs"][0]]["shape"]
        b_shape = nodes[node["inputs"][1]]["shape"]
        K = a_shape[-1]
        mm = lambda p, q: interp.k_matmul(p, q, a_shape, b_shape)
        aa, bb = np.abs(args[0]), np.abs(args[1])
        ea, eb = errs
        return mm(aa, eb) + mm(ea, bb) + mm(ea, eb) + gamma(K) * mm(aa, bb)
    if op in ("broadcast", "reshape", "transpose"):
        return interp.kernel(node, [errs[0]], graph)
    return None


def reference_with_bounds(graph, raw_inputs: Dict[str, Sequence[float]], carried: Optional[Dict] = None):
    """{values, bounds, inputs} per node (bounds.js:91-136).

    `carried` maps input names to (value, bound): an input that is an earlier
    step's output taken at its float64 value with that step's bound.
    """
    carried = carried or {}
    values: List[np.ndarray] = []
    bounds: List[np.ndarray] = []
    used: Dict[str, np.ndarray] = {}
    with np.errstate(all="ignore"):
        for node in graph["nodes"]:
            op = node["op"]
            if op == "input" and node["attrs"]["name"] in carried:
                v, e = carried[node["attrs"]["name"]]
                value = np.asarray(v, dtype=np.float64).reshape(-1).copy()
                bound = np.asarray(e, dtype=np.float64).reshape(-1).copy()
                used[node["attrs"]["name"]] = value
            elif op == "input":
                name = node["attrs"]["name"]
                if name not in raw_inputs:
                    raise KeyError(f"no value for input '{name}'")
                raw = np.asarray(raw_inputs[name], dtype=np.float64).reshape(-1)
                if raw.size != interp.size(node["shape"]):
                    raise ValueError(f"input '{name}' has {raw.size} values, needs {interp.size(node['shape'])}")
                value = fround(raw)
                used[name] = value
                bound = ftz(value)
            elif op == "const":
                value = fround(interp.kernel(node, [], graph))
                bound = ftz(value)
            else:
                args = [values[i] for i in node["inputs"]]
                errs = [bounds[i] for i in node["inputs"]]
                value = interp.kernel(node, args, graph)
                bound = _structured_bound(node, args, errs, graph)
                if bound is None:
                    bound = _elementwise_bound(op, value, args, errs)
                bound = bound + ftz(value)
            values.append(value)
            bounds.append(bound)
    return {"values": values, "bounds": bounds, "inputs": used}


def _node_step(graph, node, values, bounds_, raw_inputs, used):
    op = node["op"]
    if op == "input":
        name = node["attrs"]["name"]
        raw = np.asarray(raw_inputs[name], dtype=np.float64).reshape(-1)
        if raw.size != interp.size(node["shape"]):
            raise ValueError(f"input '{name}' has {raw.size} values, needs {interp.size(node['shape'])}")
        value = fround(raw)
        used[name] = value
        return value, ftz(value)
    if op == "const":
        value = fround(interp.kernel(node, [], graph))
        return value, ftz(value)
    args = [values[i] for i in node["inputs"]]
    errs = [bounds_[i] for i in node["inputs"]]
    value = interp.kernel(node, args, graph)
    bound = _structured_bound(node, args, errs, graph)
    if bound is None:
        bound = _elementwise_bound(op, value, args, errs)
    return value, bound + ftz(value)


def streaming_reference(graph, raw_inputs, outputs):
    """reference_with_bounds for `outputs` only, holding just the live values
    (src/fusion/workloads.js:275-301 streamingReference): {id: (value, bound)}.
    Gives exactly reference_with_bounds' values and bounds for those ids."""
    last_use = [-1] * len(graph["nodes"])
    for nid, n in enumerate(graph["nodes"]):
        for i in n["inputs"]:
            last_use[i] = nid
    keep = set(outputs)
    values: Dict[int, np.ndarray] = {}
    bnds: Dict[int, np.ndarray] = {}
    used: Dict[str, np.ndarray] = {}
    out = {}
    with np.errstate(all="ignore"):
        for nid, node in enumerate(graph["nodes"]):
            v, e = _node_step(graph, node, values, bnds, raw_inputs, used)
            values[nid], bnds[nid] = v, e
            if nid in keep:
                out[nid] = (v, e)
            for i in set(node["inputs"]):
                if last_use[i] == nid and i not in keep:
                    values.pop(i, None)
                    bnds.pop(i, None)
            if last_use[nid] == -1 and nid not in keep:
                values.pop(nid, None)
                bnds.pop(nid, None)
    return out


def unjudgeable_count(values, bounds) -> int:
    n = 0
    for v, e in zip(values, bounds):
        n += int(np.count_nonzero(~np.isfinite(v) | (np.abs(v) > F32_MAX) | ~np.isfinite(e)))
    return n


def _ratios(g: np.ndarray, r: np.ndarray, e: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    with np.errstate(all="ignore"):
        d = np.abs(g - r)
        ratio = d / (S * e)
        ratio = np.where(d == 0, 0.0, np.where(np.isnan(d), np.inf, ratio))
        # d > 0 with e == 0: d / 0 = inf already.
    return ratio


def judge(graph, gpu, values, bounds, only=None):
    """Node-by-node judgement (bounds.js:155-171): {pass, worst, first}."""
    worst, first = 0.0, None
    for node_id, node in enumerate(graph["nodes"]):
        if only is not None and node_id not in only:
            continue
        ratio = _ratios(gpu[node_id], values[node_id], bounds[node_id])
        if ratio.size:
            w = float(np.max(ratio))
            worst = max(worst, w)
            if first is None and w > 1:
                i = int(np.argmax(ratio > 1))
                first = {"node": node_id, "op": node["op"], "index": i, "gpu": float(gpu[node_id][i]),
                         "ref": float(values[node_id][i]), "bound": float(bounds[node_id][i]), "ratio": float(ratio[i])}
    return {"pass": first is None, "worst": worst, "first": first}


def judge_fused(fused_graph, origin, gpu, ref):
    """Every surviving node of a fused graph against its original node's reference (harness-m4.js:46-60)."""
    worst, first = 0.0, None
    for node_id, node in enumerate(fused_graph["nodes"]):
        o = origin[node_id]
        # A node no original node holds (origin -1: a transposed operand formed for a
        # product formed transposed) has no reference value here; refuse it rather than
        # read ref[-1], which Python would take as the last node.
        if o is None or o < 0:
            return {"pass": False, "worst": np.inf, "first": {"node": node_id, "origin": o, "op": node["op"],
                                                              "reason": "origin"}}
        g, r, e = np.asarray(gpu[node_id]), ref["values"][o], ref["bounds"][o]
        if g.size != r.size:
            return {"pass": False, "worst": np.inf, "first": {"node": node_id, "origin": o, "op": node["op"], "reason": "length"}}
        ratio = _ratios(g, r, e)
        if ratio.size:
            w = float(np.max(ratio))
            worst = max(worst, w)
            if first is None and w > 1:
                i = int(np.argmax(ratio > 1))
                first = {"node": node_id, "origin": o, "op": node["op"], "pattern": node["attrs"].get("pattern"),
                         "index": i, "gpu": float(g[i]), "ref": float(r[i]), "bound": float(e[i]), "ratio": float(ratio[i])}
    return {"pass": first is None, "worst": worst, "first": first}


def one_op_graph(graph, node):
    """The graph of `node` alone, its operands as inputs a0, a1, ... (harness-m3b.js:65-77)."""
    nodes = [{"op": "input", "inputs": [], "attrs": {"name": f"a{k}", "shape": list(graph["nodes"][i]["shape"])},
              "shape": list(graph["nodes"][i]["shape"])} for k, i in enumerate(node["inputs"])]
    nodes.append({"op": node["op"], "inputs": list(range(len(node["inputs"]))), "attrs": node["attrs"],
                  "shape": list(node["shape"])})
    return {"nodes": nodes}, len(nodes) - 1


def local_reference_fused(graph, values):
    """Per launched node: its body's (or its one op's) float64 result and bound on float32-rounded
    operand values (harness-m4.js:182-200)."""
    expected: Dict[int, np.ndarray] = {}
    bound: Dict[int, np.ndarray] = {}
    for node_id, node in enumerate(graph["nodes"]):
        if node["op"] in ("input", "const"):
            continue
        if node["op"] == "fused":
            g, out = node["attrs"]["body"], node["attrs"]["output"]
        else:
            g, out = one_op_graph(graph, node)
        r = reference_with_bounds(g, {f"a{k}": values[i] for k, i in enumerate(node["inputs"])})
        expected[node_id] = r["values"][out]
        bound[node_id] = r["bounds"][out]
    return expected, bound


def _refused(node_id, node, reason, elements):
    return {"pass": False, "unjudged": False, "worst": np.inf, "unjudgeable": 0, "elements": elements, "byKind": {},
            "first": {"node": node_id, "op": node["op"], "pattern": node["attrs"].get("pattern"), "reason": reason}}


def judge_local(graph, gpu, expected, bound):
    """Node-local judgement with the 1% unjudgeable rule (harness-m4.js:202-223)."""
    worst, first = 0.0, None
    unjudgeable = elements = 0
    by_kind: Dict[str, Dict[str, float]] = {}
    for node_id in sorted(expected):
        node = graph["nodes"][node_id]
        r, e = expected[node_id], bound[node_id]
        # A launched node with no GPU value, or one of another length, fails outright
        # (the reference indexes gpu[node.id][i] for every i; a missing or short array
        # reads undefined, which never passes).
        if node_id not in gpu:
            return _refused(node_id, node, "missing", elements)
        g = np.asarray(gpu[node_id], dtype=np.float64)
        if g.size != r.size:
            return _refused(node_id, node, "length", elements)
        kind = node["attrs"]["pattern"] if node["op"] == "fused" else "plain"
        k = by_kind.setdefault(kind, {"nodes": 0, "worst": 0.0})
        k["nodes"] += 1
        elements += r.size
        bad = ~np.isfinite(r) | (np.abs(r) > F32_MAX) | ~np.isfinite(e)
        unjudgeable += int(np.count_nonzero(bad))
        ratio = np.where(bad, 0.0, _ratios(g, r, e))
        if ratio.size:
            w = float(np.max(ratio))
            worst = max(worst, w)
            k["worst"] = max(k["worst"], w)
            if first is None and w > 1:
                i = int(np.argmax(ratio > 1))
                first = {"node": node_id, "op": node["op"], "pattern": node["attrs"].get("pattern"), "index": i,
                         "gpu": float(g[i]), "ref": float(r[i]), "bound": float(e[i]), "ratio": float(ratio[i])}
    unjudged = unjudgeable > 0.01 * elements
    return {"pass": first is None and not unjudged, "unjudged": unjudged, "worst": worst, "first": first,
            "unjudgeable": unjudgeable, "elements": elements, "byKind": by_kind}


def judge_outputs(values, bounds, gpu):
    """Outputs judged with the 1% unjudgeable rule (workloads.js:351-374)."""
    worst, first = 0.0, None
    unjudgeable = elements = 0
    if len(gpu) != len(values) or len(bounds) != len(values):
        return {"pass": False, "unjudged": False, "worst": np.inf, "unjudgeable": 0, "elements": 0,
                "first": {"output": min(len(gpu), len(values)), "reason": "length"}}
    for k, (r, e, g) in enumerate(zip(values, bounds, gpu)):
        g = np.asarray(g, dtype=np.float64)
        if g.size != r.size:
            return {"pass": False, "unjudged": False, "worst": np.inf, "unjudgeable": unjudgeable,
                    "elements": elements, "first": {"output": k, "reason": "length"}}
        elements += r.size
        bad = ~np.isfinite(r) | (np.abs(r) > F32_MAX) | ~np.isfinite(e)
        unjudgeable += int(np.count_nonzero(bad))
        ratio = np.where(bad, 0.0, _ratios(g, r, e))
        if ratio.size:
            w = float(np.max(ratio))
            worst = max(worst, w)
            if first is None and w > 1:
                i = int(np.argmax(ratio > 1))
                first = {"output": k, "index": i, "gpu": float(g[i]), "ref": float(r[i]), "bound": float(e[i]),
                         "ratio": float(ratio[i])}
    unjudged = unjudgeable > 0.01 * elements
    return {"pass": first is None and not unjudged, "unjudged": unjudged, "worst": worst,
            "unjudgeable": unjudgeable, "elements": elements, "first": first}
