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
