"""GPU parity of the matmul's operand views: every combination of a row-major and a
transposed operand (autodiff's transpose(W) and transpose(X) forms, and both at once),
unbatched and batched, at ragged sizes (not multiples of the tile) and at sizes that
force the per-element load path (extents not multiples of 4), with a bias + activation
epilogue. Each graph runs fused in the plain lowering (transposes materialised by a
gather) and in the perf lowering (the matmul reads the transposed operand in place);
both are judged against the float64 oracle within the float32 budget, the perf
lowering's output must equal the plain one's bit for bit, and the load modes the
kernels use are the ones the layout calls for."""
import sys

import numpy as np
import pytest

from oracle import bounds

pytestmark = pytest.mark.gpu

# (name, batch dims, M, K, N); the K and N of "odd" and "odd-batched" exercise the
# per-element path; "wide-split" takes the 2 x 4-wavefront tiles with a ragged last
# column tile and a K split, "wide-odd" those tiles with N not a multiple of 4.
SHAPES = [("ragged", [], 100, 72, 132), ("tiles", [], 256, 512, 192), ("batched", [3], 40, 64, 56),
          ("odd", [], 33, 17, 29), ("odd-batched", [2], 9, 30, 11), ("wide-split", [], 1000, 2100, 260),
          ("wide-odd", [], 4100, 96, 262)]


def _graph(tool, bd, M, K, N, ta, tb, act):
    """matmul(op(A), op(B)) + bias -> act, op a last-two-axes transpose when requested."""
    r = len(bd) + 2
    perm = list(range(r - 2)) + [r - 1, r - 2]
    nodes = []

    def add(op, inputs, attrs, shape):
        nodes.append({"op": op, "inputs": inputs, "attrs": attrs, "shape": shape})
        return len(nodes) - 1

    a_shape = bd + ([K, M] if ta else [M, K])
    b_shape = bd + ([N, K] if tb else [K, N])
    a = add("input", [], {"name": "A", "shape": a_shape}, a_shape)
    b = add("input", [], {"name": "B", "shape": b_shape}, b_shape)
    bias = add("input", [], {"name": "bias", "shape": [N]}, [N])
    if ta:
        a = add("transpose", [a], {"perm": perm}, bd + [M, K])
    if tb:
        b = add("transpose", [b], {"perm": perm}, bd + [K, N])
    mm = add("matmul", [a, b], {}, bd + [M, N])
    bb = add("broadcast", [bias], {"shape": bd + [M, N]}, bd + [M, N])
    s = add("add", [mm, bb], {}, bd + [M, N])
    y = add(act, [s], {}, bd + [M, N])
    return {"nodes": nodes}, y, {"A": a_shape, "B": b_shape, "bias": [N]}


def test_matmul_operand_views(tmp_path, tool):
    import tcmi_bridge
    rng = np.random.default_rng(7)
    reqs, meta = [], []
    for name, bd, M, K, N in SHAPES:
        for ta in (False, True):
            for tb in (False, True):
                act = "tanh" if (ta ^ tb) else "relu"
                g, y, shapes = _graph(tool, bd, M, K, N, ta, tb, act)
                inputs = {k: (rng.standard_normal(int(np.prod(s))) / np.sqrt(K)).astype(np.float32).tolist()
                          for k, s in shapes.items()}
                reqs.append({"name": f"{name}-{'T' if ta else 'N'}{'T' if tb else 'N'}", "graph": g, "inputs": inputs,
                             "keep": [y], "perf": True})
                meta.append((ta, tb, K, M, N, y))
    print(f"gpu step: gpu-graphs, {len(reqs)} matmul view cases", flush=True)
    tool("gpu-graphs", {"graphs": reqs}, out=str(tmp_path), timeout=300)
    b = tcmi_bridge.Bundle(tmp_path)
    for c, req, (ta, tb, K, M, N, y) in zip(b.cases, reqs, meta):
        ref = bounds.reference_with_bounds(req["graph"], {k: np.asarray(v) for k, v in req["inputs"].items()})
        fused_nodes = c["fused"]["nodes"]
        gpu = [b.arr(c["gpuFused"][str(i)]) for i in range(len(fused_nodes))]
        j = bounds.judge_fused(c["fused"], c["origin"], gpu, ref)
        assert j["pass"], (c["name"], j["first"])
        assert all(c["canaryFused"]) and c["canaryPerf"], c["name"]
        (yf,) = [int(k) for k in c["gpuPerf"]]
        perf = b.arr(c["gpuPerf"][str(yf)])
        plain = b.arr(c["gpuFused"][str(yf)])
        jp = bounds.judge_outputs([ref["values"][y]], [ref["bounds"][y]], [perf])
        assert jp["pass"], (c["name"], "perf", jp["first"])
        assert np.array_equal(perf.view(np.uint32), plain.view(np.uint32)), c["name"]
        assert len(c["perfFolded"]) == int(ta) + int(tb), c["name"]
        (modes,) = c["perfModes"]
        want_a = (1 if M % 4 == 0 else 2) if ta else (0 if K % 4 == 0 else 2)
        want_b = (1 if K % 4 == 0 else 2) if tb else (0 if N % 4 == 0 else 2)
        assert modes == [want_a, want_b], (c["name"], modes, [want_a, want_b])
        print(f"{c['name']}: modes {modes} worst {j['worst']:.3g}", file=sys.stderr)


def _mapped_case(name, src_shape, chain, role, other, act):
    """matmul over an operand formed from input `S` by `chain` ([("transpose", perm) or
    ("reshape", shape)], in order) in operand slot `role` ("a": X·W, "b": Y·X), the other
    operand an input of shape `other`, plus bias and `act`."""
    nodes = []

    def add(op, inputs, attrs, shape):
        nodes.append({"op": op, "inputs": inputs, "attrs": attrs, "shape": shape})
        return len(nodes) - 1

    x = add("input", [], {"name": "S", "shape": src_shape}, src_shape)
    shape = list(src_shape)
    for op, arg in chain:
        if op == "transpose":
            shape = [shape[p] for p in arg]
            x = add("transpose", [x], {"perm": arg}, shape)
        elif op == "relu":
            x = add("relu", [x], {}, shape)
        else:
            shape = list(arg)
            x = add("reshape", [x], {"shape": shape}, shape)
    o = add("input", [], {"name": "O", "shape": other}, other)
    a, b = (x, o) if role == "a" else (o, x)
    M, N = nodes[a]["shape"][-2], nodes[b]["shape"][-1]
    mm = add("matmul", [a, b], {}, [M, N])
    bias = add("input", [], {"name": "bias", "shape": [N]}, [N])
    bb = add("broadcast", [bias], {"shape": [M, N]}, [M, N])
    y = add(act, [add("add", [mm, bb], {}, [M, N])], {}, [M, N])
    shapes = {"S": src_shape, "O": other, "bias": [N]}
    return {"name": name, "graph": {"nodes": nodes}, "keep": [y], "perf": True}, shapes, y


# (name, source shape, chain, slot, other operand's shape, transposes read in place, modes):
# the heads of an attention merged back into rows ([B, H, T, dh] -> [B, T, H, dh] ->
# [B·T, H·dh]) read as A, as B and transposed (the weight gradient's form), the key
# gradient's double transpose, a head size that is not a multiple of 4 (per-element
# loads), a reshape that cuts the transposed layout where no mixed-radix map exists
# (its transpose stays a launch), and relus applied on load; "transposes read in place"
# counts every node the perf lowering folds (the relus too).
MAPPED = [
    ("heads-a", [2, 3, 20, 8], [("transpose", [0, 2, 1, 3]), ("reshape", [40, 24])], "a", [24, 36], 1, [0, 0]),
    ("heads-b", [2, 3, 20, 8], [("transpose", [0, 2, 1, 3]), ("reshape", [40, 24])], "b", [36, 40], 1, [0, 0]),
    ("heads-ta", [2, 3, 20, 8], [("transpose", [0, 2, 1, 3]), ("reshape", [40, 24]), ("transpose", [1, 0])], "a",
     [40, 16], 2, [1, 0]),
    ("key-double", [2, 3, 8, 20], [("transpose", [0, 1, 3, 2]), ("transpose", [0, 2, 1, 3]), ("reshape", [40, 24])],
     "a", [24, 12], 2, [1, 0]),
    ("odd-heads", [2, 3, 20, 5], [("transpose", [0, 2, 1, 3]), ("reshape", [40, 15])], "a", [15, 9], 1, [2, 2]),
    ("unmappable", [6, 4], [("transpose", [1, 0]), ("reshape", [3, 8])], "a", [8, 5], 0, [0, 2]),
    # A relu read only as a matmul operand: applied as the matmul loads it (the relu and
    # the transposes after it launch nothing), directly, transposed through mapped views,
    # and with per-element loads.
    ("relu-a", [40, 24], [("relu", None)], "a", [24, 12], 1, [0, 0]),
    ("relu-b", [40, 24], [("relu", None)], "b", [20, 40], 1, [0, 0]),
    ("relu-heads-ta", [2, 3, 20, 8], [("relu", None), ("transpose", [0, 2, 1, 3]), ("reshape", [40, 24]),
                                      ("transpose", [1, 0])], "a", [40, 16], 3, [1, 0]),
    ("relu-odd", [9, 7], [("relu", None), ("transpose", [1, 0])], "b", [5, 7], 2, [2, 2]),
]


def test_matmul_mapped_views(tmp_path, tool):
    """Operands read through a chain of transposes and reshapes (a mapped view: the row or
    column index steps over several strides): plain and perf lowerings within the budget,
    equal bit for bit, the transposes read in place where a map exists, and the load modes
    the map allows."""
    import tcmi_bridge
    rng = np.random.default_rng(11)
    reqs, meta = [], []
    for name, src, chain, role, other, folded, modes in MAPPED:
        req, shapes, y = _mapped_case(name, src, chain, role, other, "relu" if role == "a" else "tanh")
        req["inputs"] = {k: (rng.standard_normal(int(np.prod(s))) / 4).astype(np.float32).tolist() for k, s in shapes.items()}
        reqs.append(req)
        meta.append((y, folded, modes))
    print(f"gpu step: gpu-graphs, {len(reqs)} mapped view cases", flush=True)
    tool("gpu-graphs", {"graphs": reqs}, out=str(tmp_path), timeout=300)
    b = tcmi_bridge.Bundle(tmp_path)
    for c, req, (y, folded, modes) in zip(b.cases, reqs, meta):
        ref = bounds.reference_with_bounds(req["graph"], {k: np.asarray(v) for k, v in req["inputs"].items()})
        gpu = [b.arr(c["gpuFused"][str(i)]) for i in range(len(c["fused"]["nodes"]))]
        j = bounds.judge_fused(c["fused"], c["origin"], gpu, ref)
        assert j["pass"], (c["name"], j["first"])
        assert all(c["canaryFused"]) and c["canaryPerf"], c["name"]
        (yf,) = [int(k) for k in c["gpuPerf"]]
        perf = b.arr(c["gpuPerf"][str(yf)])
        jp = bounds.judge_outputs([ref["values"][y]], [ref["bounds"][y]], [perf])
        assert jp["pass"], (c["name"], "perf", jp["first"])
        assert np.array_equal(perf.view(np.uint32), b.arr(c["gpuFused"][str(yf)]).view(np.uint32)), c["name"]
        assert len(c["perfFolded"]) == folded, (c["name"], c["perfFolded"])
        assert c["perfModes"] == [modes], (c["name"], c["perfModes"])
        print(f"{c['name']}: modes {c['perfModes']} worst {j['worst']:.3g}", file=sys.stderr)
