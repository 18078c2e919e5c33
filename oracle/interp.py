"""Float64 reference interpreter for the tensor IR — TEST INFRASTRUCTURE ONLY.

This module is the oracle the MI355X backend is judged against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only
as the checker (or as the timed CPU baseline); no product code path calls it.

It restates src/interp.js of abho7/tensor-compiler-webgpu (KERNELS :48-128,
evaluate :136-157) in numpy, keeping the properties that make its values
bitwise reproducible there:
  * every reduction sums (or maxes) its terms first to last along the axis
    (interp.js:34-45) — done here one slice at a time, vectorised across the
    other axes, so each output sees exactly the reference's sequence of adds;
  * matmul accumulates p = 0..K-1 from 0 with a separate multiply and add per
    term (interp.js:67-84) — done as rank-1 updates, which gives the same
    per-output sequence of roundings as the reference's i-j-p loop;
  * max keeps `v > acc ? v : acc` from -inf (NaN never replaces acc);
  * relu/step compare with `> 0` (relu(NaN) = 0, step(NaN) = 0).
Graphs are the reference's JSON form: {"nodes": [{op, inputs, attrs, shape}]}.
A `fused` node (src/fusion/fuse.js:295-302, FUSED_KERNELS) is evaluated by
evaluating its body graph on its operands.

Parity pins (tests/test_oracle_golden.py): golden/torch.json float64 outputs and
gradients of the reference's 112 cases within 1e-12 (random-9 excepted as the
reference itself records), the closed forms of test/interp.test.js, and the
transformer init logits/gradients of golden/torch-m3b.f64 within 1e-10.
"""
from __future__ import annotations

import contextlib
import math
from typing import Callable, Dict, List, Optional, Sequence

import numpy as np


def size(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


def strides(shape: Sequence[int]) -> List[int]:
    s = [0] * len(shape)
    acc = 1
    for i in range(len(shape) - 1, -1, -1):
        s[i] = acc
        acc *= int(shape[i])
    return s


def _nd(x: np.ndarray, shape: Sequence[int]) -> np.ndarray:
    return x.reshape(tuple(int(d) for d in shape)) if len(shape) else x.reshape(())


def _reduce_dims(shape, axis):
    return size(shape[:axis]), int(shape[axis]), size(shape[axis + 1:])


def k_sum(x: np.ndarray, in_shape, axis) -> np.ndarray:
    outer, n, inner = _reduce_dims(in_shape, axis)
    v = x.reshape(outer, n, inner)
    acc = np.zeros((outer, inner), dtype=np.float64)
    for k in range(n):
        acc = acc + v[:, k, :]
    return acc.reshape(-1)


def k_max(x: np.ndarray, in_shape, axis) -> np.ndarray:
    outer, n, inner = _reduce_dims(in_shape, axis)
    v = x.reshape(outer, n, inner)
    acc = np.full((outer, inner), -np.inf, dtype=np.float64)
    for k in range(n):
        col = v[:, k, :]
        acc = np.where(col > acc, col, acc)
    return acc.reshape(-1)


# Products with at least this many multiply-adds go to the BLAS (float64, its own
# summation order) inside a `blas_matmul()` block; everything else, and every product
# outside such a block, accumulates p = 0..K-1 as the reference does.
_BLAS_FROM: Optional[int] = None


@contextlib.contextmanager
def blas_matmul(min_macs: int = 1 << 22):
    """Within the block, large products are summed in the BLAS's order instead of p
    ascending. Two orders of a float64 sum of K products differ by at most
    2*gamma64(K) * sum|a||b| (gamma64(K) = K*2^-53 / (1 - K*2^-53)), about 1e-9 of the
    float32 budget's gamma32(K) * sum|a||b| term; tests/test_oracle_golden.py pins
    the difference to that bound and the golden cases to 1e-12 under it. For the
    full-size training steps, whose products an ordered sum takes minutes to form."""
    global _BLAS_FROM
    prev, _BLAS_FROM = _BLAS_FROM, int(min_macs)
    try:
        yield
    finally:
        _BLAS_FROM = prev


def k_matmul(a: np.ndarray, b: np.ndarray, a_shape, b_shape, rows: Optional[np.ndarray] = None) -> np.ndarray:
    """Batched matmul, p ascending from 0 per output; `rows` restricts to a subset of output rows."""
    m, k, n = int(a_shape[-2]), int(a_shape[-1]), int(b_shape[-1])
    batch = size(a_shape[:-2])
    A = a.reshape(batch, m, k)
    B = b.reshape(batch, k, n)
    if rows is not None:
        A = A[:, rows, :]
    if _BLAS_FROM is not None and batch * A.shape[1] * k * n >= _BLAS_FROM:
        return np.matmul(A, B).reshape(-1)
    acc = np.zeros((batch, A.shape[1], n), dtype=np.float64)
    for p in range(k):
        acc = acc + A[:, :, p:p + 1] * B[:, p:p + 1, :]
    return acc.reshape(-1)


def k_broadcast(x: np.ndarray, from_shape, to_shape) -> np.ndarray:
    lead = len(to_shape) - len(from_shape)
    src = _nd(x, [1] * lead + list(from_shape))
    return np.broadcast_to(src, tuple(to_shape)).reshape(-1).copy()


def k_transpose(x: np.ndarray, from_shape, perm) -> np.ndarray:
    return np.ascontiguousarray(np.transpose(_nd(x, from_shape), tuple(perm))).reshape(-1)


def _const(node) -> np.ndarray:
    v = node["attrs"]["value"]
    n = size(node["shape"])
    if isinstance(v, (int, float)):
        return np.full(n, float(v), dtype=np.float64)
    return np.array([float(t) for t in v], dtype=np.float64)


def _relu(x):
    return np.where(x > 0, x, 0.0)


def _step(x):
    return np.where(x > 0, 1.0, 0.0)


UNARY: Dict[str, Callable[[np.ndarray], np.ndarray]] = {
    "neg": lambda x: -x,
    "exp": np.exp,
    "log": np.log,
    "relu": _relu,
    "tanh": np.tanh,
    "sqrt": np.sqrt,
    "step": _step,
    "stopGradient": lambda x: x.copy(),
}
BINARY = {
    "add": lambda a, b: a + b,
    "sub": lambda a, b: a - b,
    "mul": lambda a, b: a * b,
    "div": lambda a, b: a / b,
}


def kernel(node, args: List[np.ndarray], graph) -> np.ndarray:
    """The value of one non-input node from its input values (interp.js KERNELS)."""
    op = node["op"]
    nodes = graph["nodes"]
    if op == "const":
        return _const(node)
    if op in BINARY:
        return BINARY[op](args[0], args[1])
    if op in UNARY:
        return UNARY[op](args[0])
    if op == "matmul":
        return k_matmul(args[0], args[1], nodes[node["inputs"][0]]["shape"], nodes[node["inputs"][1]]["shape"])
    if op == "sum":
        return k_sum(args[0], nodes[node["inputs"][0]]["shape"], node["attrs"]["axis"])
    if op == "max":
        return k_max(args[0], nodes[node["inputs"][0]]["shape"], node["attrs"]["axis"])
    if op == "broadcast":
        return k_broadcast(args[0], nodes[node["inputs"][0]]["shape"], node["shape"])
    if op == "reshape":
        return args[0].copy()
    if op == "transpose":
        return k_transpose(args[0], nodes[node["inputs"][0]]["shape"], node["attrs"]["perm"])
    if op == "fused":
        body = node["attrs"]["body"]
        vals = evaluate(body, {f"a{k}": a for k, a in enumerate(args)})
        return vals[node["attrs"]["output"]]
    raise ValueError(f"no kernel for '{op}'")


def evaluate(graph, inputs: Dict[str, Sequence[float]], kernels: Optional[Callable] = None,
             on_node: Optional[Callable] = None) -> List[np.ndarray]:
    """Every node's float64 value, flat row-major (interp.js:136-157)."""
    k = kernels or kernel
    values: List[np.ndarray] = []
    with np.errstate(all="ignore"):
        for node in graph["nodes"]:
            if node["op"] == "input":
                name = node["attrs"]["name"]
                if name not in inputs:
                    raise KeyError(f"no value for input '{name}'")
                v = np.asarray(inputs[name], dtype=np.float64).reshape(-1).copy()
                if v.size != size(node["shape"]):
                    raise ValueError(f"input '{name}': expected {size(node['shape'])} numbers, got {v.size}")
            else:
                args = [values[i] for i in node["inputs"]]
                v = k(node, args, graph)
                if on_node:
                    on_node(node, args, v)
            values.append(v)
    return values


def run(graph, inputs, outputs):
    vals = evaluate(graph, inputs)
    return [vals[i] for i in outputs]
