"""The slices through which the GPU tests of configs 3 and 4 are judged at full
size are exact: for the graphs the builder makes, the oracle's values and bounds
of a slice of the full graph's outputs equal, bit for bit, those of the graph
built at the slice's size on the sliced inputs — rows for softmax/logSoftmax
(forward and gradient) and for y, dX of the matmul epilogue; columns for its y,
dW and dbias. A planted mistake in the slicing (a shifted row) must show."""
import numpy as np
import pytest

from oracle import bounds


def _graphs(tool, c3, c4):
    return tool("config-graphs", {"c3": c3, "c4": c4})


def _ref(graph, inputs, ids):
    out = bounds.streaming_reference(graph, inputs, ids)
    return [out[i] for i in ids]


def test_c3_row_slices_exact(tool):
    R, C, rows = 12, 16, [0, 3, 4, 11]
    rng = np.random.default_rng(5)
    x = (2 * rng.standard_normal(R * C)).astype(np.float32)
    x[3 * C:4 * C] += 800
    dy = rng.standard_normal(R * C).astype(np.float32)
    full = _graphs(tool, [{"fn": f, "R": R, "C": C} for f in ("softmax", "logSoftmax")], [])["c3"]
    sub = _graphs(tool, [{"fn": f, "R": len(rows), "C": C} for f in ("softmax", "logSoftmax")], [])["c3"]
    take = lambda a: a.reshape(R, C)[rows].reshape(-1)
    for fg, sg in zip(full, sub):
        for kind in ("forward", "gradient"):
            ins = {"x": x} if kind == "forward" else {"x": x, "d0": dy}
            sins = {k: take(v) for k, v in ins.items()}
            a = _ref(fg[kind]["graph"], ins, fg[kind]["keep"])
            b = _ref(sg[kind]["graph"], sins, sg[kind]["keep"])
            assert fg[kind]["keep"] == sg[kind]["keep"]
            for (va, ea), (vb, eb) in zip(a, b):
                assert np.array_equal(take(va), vb) and np.array_equal(take(ea), eb), (fg["fn"], kind)
            # A planted slicing mistake (row 4's inputs in place of row 3's) is seen.
            bad = {k: v.reshape(R, C)[[0, 4, 4, 11]].reshape(-1) for k, v in ins.items()}
            vbad = _ref(sg[kind]["graph"], bad, sg[kind]["keep"])[0][0]
            assert not np.array_equal(take(a[0][0]), vbad)


def test_c4_row_and_column_slices_exact(tool):
    M, K, N = 6, 5, 7
    rows, cols = [0, 2, 5], [1, 4, 6]
    rng = np.random.default_rng(6)
    X = rng.standard_normal(M * K).astype(np.float32)
    W = rng.standard_normal(K * N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    dY = rng.standard_normal(M * N).astype(np.float32)
    acts = ("relu", "tanh")
    full = _graphs(tool, [], [{"act": a, "M": M, "K": K, "N": N} for a in acts])["c4"]
    by_rows = _graphs(tool, [], [{"act": a, "M": len(rows), "K": K, "N": N} for a in acts])["c4"]
    by_cols = _graphs(tool, [], [{"act": a, "M": M, "K": K, "N": len(cols)} for a in acts])["c4"]
    r2 = lambda a, w: a.reshape(-1, w)[rows].reshape(-1)
    c2 = lambda a, w: a.reshape(-1, w)[:, cols].reshape(-1)
    for fg, rg, cg in zip(full, by_rows, by_cols):
        g = fg["gradient"]
        ins = {"X": X, "W": W, "bias": bias, "d0": dY}
        y, dx, dw, db = _ref(g["graph"], ins, g["keep"])
        yr, dxr = _ref(rg["gradient"]["graph"], {"X": r2(X, K), "W": W, "bias": bias, "d0": r2(dY, N)},
                       rg["gradient"]["keep"][:2])
        yc, _, dwc, dbc = _ref(cg["gradient"]["graph"], {"X": X, "W": c2(W, N), "bias": bias[cols], "d0": c2(dY, N)},
                               cg["gradient"]["keep"])
        for (v, e), (vs, es), sl in ((y, yr, lambda a: r2(a, N)), (dx, dxr, lambda a: r2(a, K)),
                                     (y, yc, lambda a: c2(a, N)), (dw, dwc, lambda a: c2(a, N)),
                                     (db, dbc, lambda a: a[cols])):
            assert np.array_equal(sl(v), vs) and np.array_equal(sl(e), es), fg["act"]
