"""Float64 training trajectories of a step graph, and the metrics the reference compares
them with PyTorch by — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, and only as the checker; no product code path calls
it. It restates, from abho7/tensor-compiler-webgpu:

  * trainCpu3b (src/m3b/cpu.js:19-35): the training step graph (forward, autodiff's
    backward, the optimizer as IR ops) evaluated in float64 by interp.evaluate, each
    step's new parameters and optimizer state fed to the next step as its inputs;
  * encodeBatch (src/m3b/data.js:62-72): one-hot tokens x and next-token targets y, both
    [B*T, V];
  * v2Score and projectionScore (src/m3b/verify-cpu.js:14-44) with TAU1 = 1e-10 and
    TAU2 = 1e-8 (verify-cpu.js:10-11);
  * projectionVector (src/m3b/config.js:14-24): FNV-1a of the parameter's name, plus
    7919*k, seeds mulberry32 (src/testing/rng.js), whose draws give the k-th vector,
    uniform in [-1, 1];
  * sha256F64 (src/m3b/spec.js:13-18).

Pins (tests/test_golden_runs.py): the projection vectors of every parameter hash to
golden/spec-m3b.json's projections.sha256, so the generator is the reference's bit for
bit; each golden run's parameters hash to its initSha; the forward pass at each run's
initialisation matches golden/torch-m3b.f64's logits and torch-m3b.json's loss at 1e-10;
the 20-step trajectories of all four golden runs match torch-m3b.json's per-step losses
and parameter projections at 1e-8, and golden-seed1's final parameters element by
element at 1e-8; a trajectory that does not feed the optimizer state back fails the
projections at its second step.
"""
from __future__ import annotations

import hashlib
from typing import Dict, List, Sequence

import numpy as np

from oracle import interp

TAU1 = 1e-10
TAU2 = 1e-8


def mulberry32(seed: int, n: int) -> np.ndarray:
    """The first `n` draws of mulberry32 from `seed`, as float64 in [0, 1) (rng.js next()).

    The generator's state advances by a constant per draw, so draw i's state is
    seed + i * 0x6D2B79F5 (mod 2^32) and the draws can be formed side by side; every
    step of the output mix is 32-bit wrap-around arithmetic, as the reference's
    Math.imul and ToInt32 conversions make it."""
    i = np.arange(1, n + 1, dtype=np.uint64)
    t = ((np.uint64(seed & 0xFFFFFFFF) + i * np.uint64(0x6D2B79F5)) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    t = (t ^ (t >> np.uint32(15))) * (t | np.uint32(1))
    t = t ^ (t + (t ^ (t >> np.uint32(7))) * (t | np.uint32(61)))
    t = t ^ (t >> np.uint32(14))
    return t.astype(np.float64) / 4294967296.0


def fnv1a(name: str) -> int:
    """FNV-1a over a name's characters, 32 bits (config.js:15-19)."""
    h = 0x811C9DC5
    for ch in name:
        h ^= ord(ch)
        h = (h * 0x01000193) & 0xFFFFFFFF
    return h


def projection_vector(name: str, n: int, k: int) -> np.ndarray:
    """The k-th projection vector of a parameter of `n` elements (config.js:22-24)."""
    return -1.0 + 2.0 * mulberry32((fnv1a(name) + 7919 * k) & 0xFFFFFFFF, n)


def sha256_f64(arrays: Sequence[Sequence[float]]) -> str:
    """SHA-256 of the arrays' float64 little-endian bytes, in order (spec.js:13-18)."""
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.asarray(a, dtype="<f8").tobytes())
    return h.hexdigest()


def encode_batch(seqs: Sequence[Sequence[int]], V: int, T: int):
    """One-hot x and y [B*T, V] for sequences of T + 1 tokens; y holds token t + 1 (data.js:62-72)."""
    B = len(seqs)
    x = np.zeros(B * T * V)
    y = np.zeros(B * T * V)
    for b, s in enumerate(seqs):
        rows = (b * T + np.arange(T)) * V
        x[rows + np.asarray(s[:T])] = 1.0
        y[rows + np.asarray(s[1:T + 1])] = 1.0
    return x, y


def train(step: Dict, params: Dict[str, Sequence[float]], state: Dict[str, Sequence[float]],
          batches: Sequence, feed_state: bool = True) -> Dict[str, List]:
    """`len(batches)` steps of the step graph in float64 (cpu.js:19-35).

    `step` holds the step graph (`graph`), the parameter and state names (`names`,
    `stateNames`), the node id of the loss and of every new value (`loss`, `outputs`) and
    the cotangent input's name (`cotangent`, fed 1). `batches[t]` is step t's (x, y).
    Returns the losses and the parameters and state after each step. With `feed_state`
    false the initial state is fed to every step (a planted mistake for the pins)."""
    params = {k: np.asarray(v, dtype=np.float64) for k, v in params.items()}
    state0 = {k: np.asarray(v, dtype=np.float64) for k, v in state.items()}
    state = dict(state0)
    losses, kept_params, kept_state = [], [], []
    for x, y in batches:
        feed = dict(params)
        feed.update(state)
        feed["x"], feed["y"] = x, y
        feed[step["cotangent"]] = np.ones(1)
        v = interp.evaluate(step["graph"], feed)
        losses.append(float(v[step["loss"]][0]))
        params = {n: v[step["outputs"][n]] for n in step["names"]}
        state = {n: v[step["outputs"][n]] for n in step["stateNames"]} if feed_state else dict(state0)
        kept_params.append(params)
        kept_state.append(state)
    return {"losses": losses, "params": kept_params, "states": kept_state}


def v2_score(ours, ref, tau: float) -> float:
    """Metric v2: the largest |ours - ref| / (tau * max(1, max|ref|) + tau * |ref|) (verify-cpu.js:14-24)."""
    ours = np.asarray(ours, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    atol = tau * max(1.0, scale)
    d = np.abs(ours - ref)
    with np.errstate(invalid="ignore"):
        r = np.where(np.isnan(d), np.inf, d / (atol + tau * np.abs(ref)))
    return float(np.max(r)) if r.size else 0.0


def projection_score(ours, r, ref_proj: float, tau: float) -> float:
    """|<r, ours> - ref_proj| over sum_i |r_i| (atol + tau |ours_i|) (verify-cpu.js:33-44):
    the projected form of the elementwise check, with the scale taken from this side."""
    ours = np.asarray(ours, dtype=np.float64)
    scale = float(np.max(np.abs(ours))) if ours.size else 0.0
    atol = tau * max(1.0, scale)
    p = float(np.dot(r, ours))
    allow = float(np.dot(np.abs(r), atol + tau * np.abs(ours)))
    d = abs(p - ref_proj)
    return float("inf") if np.isnan(d) else d / allow
