"""GPU parity of the fused attention kernel (the fusion extension: matmul(Q, Kt), the
softmax group and matmul(P, V) as one kernel, fuse(..., {attention: true})).

Each graph runs with attention fused in the plain lowering (head-split and key
transposes materialised by gathers) and in the perf lowering (Q, Kt and V read in place
through strided views), and with the contract's own fusion (three launches). Every
fused node is judged against the float64 oracle within the float32 budget (judgeFused,
harness-m4.js:46-60), canaries must be intact, and the perf lowering's output must equal
the plain one's bit for bit. Sizes cover the transformer's two head shapes, ragged
query/key counts and head sizes (tile padding), head sizes that force per-element loads,
more than one 64-row query block, keys and values given already transposed, a key
count past the kernel's limit that must stay three launches, and two independent
attentions of one shape, which the perf lowering runs as one batched launch."""
import sys

import numpy as np
import pytest

from oracle import bounds

pytestmark = pytest.mark.gpu


def _cases(tool, golden_cases):
    reqs = []
    att = next(c for c in golden_cases if c["name"] == "attention")
    reqs.append(({"name": "golden-attention", "graph": att["graph"], "inputs": att["inputs"], "keep": att["outputs"]}, True))
    for config, V, B in (("reference", 16, 2), ("c5", 96, 2)):
        fw = tool("transformer-forward", {"config": config, "V": V, "B": B})
        reqs.append(({"name": f"transformer-{config}", "graph": fw["graph"], "inputs": fw["inputs"], "keep": fw["keep"]}, True))
    # The synthetic cases (tool.js ATTENTION_CASES): ragged sizes, per-element loads, several
    # query blocks, pre-transposed keys and values, one past the kernel's key limit, and two
    # independent attentions of one shape (a batched launch).
    for b in tool("attention-graphs"):
        fuses = b.pop("fuses")
        reqs.append((b, fuses))
    return reqs


def test_fused_attention_within_budget(tmp_path, tool, golden_cases):
    import tcmi_bridge
    cases = _cases(tool, golden_cases)
    reqs = [dict(r, perf=True, attention=True) for r, _ in cases] + [dict(r, name=r["name"] + "/contract") for r, _ in cases]
    print(f"gpu step: gpu-graphs, {len(reqs)} attention graphs", flush=True)
    tool("gpu-graphs", {"graphs": reqs}, out=str(tmp_path), timeout=300)
    b = tcmi_bridge.Bundle(tmp_path)
    by = {c["name"]: c for c in b.cases}
    for req, fuses in cases:
        c = by[req["name"]]
        contract = by[req["name"] + "/contract"]
        inputs = {k: np.asarray(v) for k, v in req["inputs"].items()}
        ref = bounds.reference_with_bounds(req["graph"], inputs)
        n_att = c["kinds"].count("fused-attention")
        assert (n_att > 0) == fuses, (req["name"], c["kinds"])
        assert "fused-attention" not in contract["kinds"]
        for entry in (c, contract):
            nodes = entry["fused"]["nodes"]
            gpu = [b.arr(entry["gpuFused"][str(i)]) for i in range(len(nodes))]
            j = bounds.judge_fused(entry["fused"], entry["origin"], gpu, ref)
            assert j["pass"], (entry["name"], j["first"])
            assert all(entry["canaryFused"]), entry["name"]
        assert c["canaryPerf"], req["name"]
        for k, h in c["gpuPerf"].items():
            perf, plain = b.arr(h), b.arr(c["gpuFused"][k])
            assert np.array_equal(perf.view(np.uint32), plain.view(np.uint32)), (req["name"], k)
        if req["name"].startswith("transformer"):
            # The head split and the key transpose: Q, Kt and V all read in place in the perf lowering.
            assert c["perfViews"] and all(v == ["k", "q", "v"] for v in c["perfViews"]), (req["name"], c["perfViews"])
        if req["name"] == "pre-transposed":
            # Kt is an input as it is; only V's transpose is read in place.
            assert c["perfViews"] == [["v"]], c["perfViews"]
        if req["name"] == "twin":
            # The two independent attentions run as one batched launch of the attention kernel.
            assert [(x["count"], x["kind"]) for x in c["perfBatches"]] == [(2, "fused-attention")], c["perfBatches"]
        # The fused output against the contract's three launches: both within the budget of
        # the same reference; report how far apart they are.
        out_id = req["keep"][0]
        a = b.arr(c["gpuFused"][str(c["origin"].index(out_id))])
        z = b.arr(contract["gpuFused"][str(contract["origin"].index(out_id))])
        print(f"{req['name']}: attention kernels {n_att}, max |fused - contract| {np.max(np.abs(a - z)):.3g}", file=sys.stderr)
