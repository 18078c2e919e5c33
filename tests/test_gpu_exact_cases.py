"""GPU special cases whose results the mathematics fixes exactly, independent of the
float32 budget: a product with an identity or a one-hot operand has one nonzero term
per output, so every path of the matmul kernel (tiles, ragged edges, per-element loads,
K groups, the K split and its chunk sums, operands read through transposed views,
batches) must return the other operand's values bit for bit; and softmax and
logSoftmax subtract the row maximum, so a row shifted by +800 (config 3's shifted rows)
must give its unshifted twin's result within the two rows' budgets. Each graph runs in
the plain lowering and in the perf lowering the bench times."""
import numpy as np
import pytest

from oracle import bounds

pytestmark = pytest.mark.gpu


def _nodes():
    nodes = []

    def add(op, inputs, attrs, shape):
        nodes.append({"op": op, "inputs": inputs, "attrs": attrs, "shape": shape})
        return len(nodes) - 1
    return nodes, add


def _identity_case(name, bd, M, K, N, ta, tb, rng):
    """matmul(op(X), op(S)): X [.., M, K] (its transpose read back through a view when
    ta), S [K, N] the first N columns of the K x K identity (stored transposed when tb),
    so the product is X's first N columns."""
    nodes, add = _nodes()
    r = len(bd) + 2
    perm = list(range(r - 2)) + [r - 1, r - 2]
    x_shape = bd + ([K, M] if ta else [M, K])
    s_shape = bd + ([N, K] if tb else [K, N])
    x = add("input", [], {"name": "X", "shape": x_shape}, x_shape)
    i = add("input", [], {"name": "S", "shape": s_shape}, s_shape)
    if ta:
        x = add("transpose", [x], {"perm": perm}, bd + [M, K])
    if tb:
        i = add("transpose", [i], {"perm": perm}, bd + [K, N])
    y = add("matmul", [x, i], {}, bd + [M, N])
    xs = rng.standard_normal(int(np.prod(x_shape))).astype(np.float32)
    sel = np.eye(K, N, dtype=np.float32)
    sel = np.ascontiguousarray(sel.T if tb else sel)
    sel = np.broadcast_to(sel, tuple(bd) + sel.shape).ravel()
    xm = xs.reshape(x_shape)
    if ta:
        xm = np.swapaxes(xm, -1, -2)
    want = np.ascontiguousarray(xm[..., :N]).ravel()
    return ({"name": name, "graph": {"nodes": nodes}, "inputs": {"X": xs.tolist(), "S": sel.tolist()}, "keep": [y],
             "perf": True}, y, want)


def test_identity_and_one_hot_products_are_exact(tmp_path, tool):
    import tcmi_bridge
    rng = np.random.default_rng(11)
    reqs, expect = [], []
    # (name, batch dims, M, K, N): ragged tiles, per-element loads (extents not multiples
    # of 4), K groups (a few 32 x 32 tiles over K >= 256), a K split (K >= 2048, its
    # chunks summed by the second kernel), a batch.
    for name, bd, M, K, N in [("ragged", [], 100, 72, 72), ("odd", [], 33, 29, 27), ("kgroups", [], 64, 512, 64),
                              ("split", [], 96, 2304, 128), ("batched", [3], 40, 64, 64)]:
        for ta in (False, True):
            for tb in (False, True):
                req, y, want = _identity_case(f"identity-{name}-{'T' if ta else 'N'}{'T' if tb else 'N'}", bd, M, K, N, ta, tb,
                                              rng)
                reqs.append(req)
                expect.append((y, want))
    # One-hot rows times an embedding table: row t of the product is row token[t] of E.
    nodes, add = _nodes()
    T, V, D = 500, 96, 256
    tokens = rng.integers(0, V, T)
    oh = np.zeros((T, V), dtype=np.float32)
    oh[np.arange(T), tokens] = 1
    e = rng.standard_normal(V * D).astype(np.float32)
    x = add("input", [], {"name": "x", "shape": [T, V]}, [T, V])
    w = add("input", [], {"name": "E", "shape": [V, D]}, [V, D])
    y = add("matmul", [x, w], {}, [T, D])
    reqs.append({"name": "one-hot", "graph": {"nodes": nodes}, "inputs": {"x": oh.ravel().tolist(), "E": e.tolist()},
                 "keep": [y], "perf": True})
    expect.append((y, e.reshape(V, D)[tokens].ravel()))
    print(f"gpu step: gpu-graphs, {len(reqs)} exact product cases", flush=True)
    tool("gpu-graphs", {"graphs": reqs}, out=str(tmp_path), timeout=300)
    b = tcmi_bridge.Bundle(tmp_path)
    for c, (y, want) in zip(b.cases, expect):
        assert all(c["canaryFused"]) and c["canaryPerf"], c["name"]
        (yf,) = [int(k) for k in c["gpuPerf"]]
        perf = b.arr(c["gpuPerf"][str(yf)])
        plain = b.arr(c["gpuFused"][str(yf)])
        assert np.array_equal(plain.view(np.uint32), want.view(np.uint32)), c["name"]
        assert np.array_equal(perf.view(np.uint32), want.view(np.uint32)), c["name"]


@pytest.mark.parametrize("fn", ["softmax", "logSoftmax"])
def test_shifted_rows_match_their_unshifted_twins(tmp_path, tool, fn):
    """Rows R/2 .. R-1 of the input are rows 0 .. R/2-1 plus 800 (exactly representable
    here: the values are multiples of 2^-8 of magnitude below 32): each pair of outputs
    agrees within the sum of the two rows' float32 budgets, in both lowerings."""
    import tcmi_bridge
    rng = np.random.default_rng(5)
    R, C = 64, 4096
    half = (np.round(rng.standard_normal((R // 2, C)) * 2 * 256) / 256).astype(np.float32)
    x = np.concatenate([half, half + np.float32(800)])
    assert np.array_equal(x[R // 2:] - np.float32(800), half)      # the shift is exact
    (g,) = tool("config-graphs", {"c3": [{"fn": fn, "R": R, "C": C}]})["c3"]
    fwd = g["forward"]
    (y,) = fwd["keep"]
    req = {"name": f"shift-{fn}", "graph": fwd["graph"], "inputs": {"x": x.ravel().tolist()}, "keep": [y], "perf": True}
    print(f"gpu step: gpu-graphs, {fn} shifted rows", flush=True)
    tool("gpu-graphs", {"graphs": [req]}, out=str(tmp_path), timeout=300)
    b = tcmi_bridge.Bundle(tmp_path)
    (c,) = b.cases
    ref = bounds.reference_with_bounds(req["graph"], {"x": x.ravel().astype(np.float64)})
    bound = ref["bounds"][y].reshape(R, C)
    assert all(c["canaryFused"]) and c["canaryPerf"]
    (yf,) = [int(k) for k in c["gpuPerf"]]
    for got in (b.arr(c["gpuPerf"][str(yf)]), b.arr(c["gpuFused"][str(yf)])):
        g = got.astype(np.float64).reshape(R, C)
        gap = np.abs(g[: R // 2] - g[R // 2:])
        allowed = 2 * (bound[: R // 2] + bound[R // 2:])
        assert np.all(gap <= allowed), (fn, float(np.max(gap - allowed)))
        assert np.all(np.isfinite(g))
