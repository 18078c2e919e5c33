"""GPU parity of config 5's training step at its benchmark batch (B 64): every launch of
the checked lowering and of the trainer's perf lowering (split-K weight gradients over
8192 rows, batched dispatches, transposes read in place, the [8192, ...] elementwise and
rowwise kernels, row statistics folded into their reductions) judged node-locally against the float64 oracle within the float32
budget (src/gpu/harness-m4.js:182-223), on the GPU's own operands from one run of the
checked lowering.

A launch whose output carries the batch is judged on sampled sequences: sequence b's
block of its output against the oracle on sequence b's blocks of its operands, with the
block shapes of the same builder's one-sequence graph and the full graph's constants
(the loss scale 1/(B*T) among them); tests/test_step_slices.py shows on the CPU that
these blocks equal the blocks of the whole launch's expectation bit for bit. A launch
whose output does not (weight and bias gradients over all 8192 rows, their SGD updates,
the loss) is judged whole on whole operands. The oracle sums the large products in the
BLAS's order (interp.blas_matmul, pinned within 2*gamma64(K)*sum|a||b| of the ordered
sum)."""
import sys

import numpy as np
import pytest

from oracle import bounds, interp
from step_slices import batch_axis, expectations

pytestmark = pytest.mark.gpu

SEQUENCES = [0, 21, 42, 63]


@pytest.mark.parametrize("attention", [False, True])
def test_c5_full_batch_step_node_local(tmp_path, tool, attention):
    """With `attention`, the step with each attention and its gradient fused
    (fusion/attention.js): the forward attention kernels and the gradients' dQ, dK and dV
    kernels (checked lowering) and joint kernels (perf lowering) judged on the sequences'
    blocks like every other launch."""
    import tcmi_bridge
    print(f"gpu step: gpu-step-slices transformer B 64, sequences {SEQUENCES}, attention {attention}", flush=True)
    tool("gpu-step-slices", {"model": "transformer", "B": 64, "sequences": SEQUENCES, "attention": attention},
         out=str(tmp_path), timeout=900)
    b = tcmi_bridge.Bundle(tmp_path)
    c = b.cases[0]
    full, twin = c["graph"], c["twin"]
    assert c["canaryChecked"] and c["canaryPerf"]
    assert c["splitK"] > 0 and c["batches"] > 0, (c["splitK"], c["batches"])
    assert abs(c["loss"] - np.log(96)) < 0.1
    for i, (n, t) in enumerate(zip(full["nodes"], twin["nodes"])):
        p = batch_axis(n["shape"], t["shape"])
        assert c["axis"][i] == p
        if p >= 0:
            assert n["shape"][p] == 64 * t["shape"][p]
    vals = {int(k): v for k, v in c["values"].items()}
    perf = {int(k): v for k, v in c["perf"].items()}

    def operand(i, s):
        return b.arr(vals[i]["whole"] if s is None else vals[i]["blocks"][s])

    counts = {}
    for variant, outs, launched in (("checked", vals, c["launched"]), ("perf", perf, c["perfLaunched"])):
        ref_v, ref_e, gpu = [], [], []
        blocks = wholes = 0
        with interp.blas_matmul():
            folds = c["rowFolds"] if variant == "perf" else None
            took = c["absorbed"] if variant == "perf" else None
            formed = c["formed"] if variant == "perf" else None
            for nid, s, v, e in expectations(full, twin, launched, operand, SEQUENCES, folds, took, formed):
                ref_v.append(v)
                ref_e.append(e)
                gpu.append(b.arr(outs[nid]["whole"] if s is None else outs[nid]["blocks"][s]))
                blocks += s is not None
                wholes += s is None
                if (blocks + wholes) % 200 == 0:
                    print(f"C5 B64 {variant}: {blocks + wholes} expectations", file=sys.stderr, flush=True)
        j = bounds.judge_outputs(ref_v, ref_e, gpu)
        counts[variant] = (blocks, wholes)
        print(f"C5 B64 {variant}: {len(launched)} launches ({blocks} sequence blocks, {wholes} whole), worst "
              f"{j['worst']:.3g} over {j['elements']} elements, unjudgeable {j['unjudgeable']}", file=sys.stderr)
        assert j["pass"], (variant, j["first"], j["unjudged"])
    print(f"C5 B64: split-K launches {c['splitK']}, batched dispatches {c['batches']}, row reductions folded into "
          f"{len(c['rowFolds'])} chains, producers absorbed by {len(c['absorbed'])} launches, values formed by "
          f"{len(c['formed'])} launches", file=sys.stderr)
    assert len(c["rowFolds"]) > 0 and len(c["absorbed"]) > 0 and len(c["formed"]) > 0
    assert counts["checked"][0] >= 4 * (250 if attention else 300) and counts["checked"][1] >= 40, counts
    assert counts["perf"][0] > 0 and counts["perf"][1] > 0, counts
