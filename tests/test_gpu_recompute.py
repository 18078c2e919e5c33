"""GPU parity of the fusion pass's recompute option (src/fusion/fuse.js:64-67,149-152:
a producer is pulled into a group across a broadcast, or duplicated into every consumer
group, and evaluated at the source index), the codegen path of the reference's
deliberate "fusion loses" measurements:

- the broadcast-recompute workloads (R 16, 256, 4096: a 16-op chain on a [256] row
  recomputed for every row) and the lost-reuse workloads (a 1-op and a 16-op chain
  shared by four consumers), src/fusion/workloads.js:96-104: fused and recompute
  variants, every surviving node in the plain lowering judged against its original
  node's reference (judgeFused, harness-m4.js:46-60), and every variant's outputs in
  the perf lowering the bench times (judgeOutputs, workloads.js:351-374), canaries intact;
- corpus programs 1..100 (200 graphs) fused with recomputation, plain and perf
  lowerings, every surviving node judged the same way and the perf lowering's kept
  outputs equal to the plain lowering's bit for bit.
The recompute variants of the five workloads have fewer fused nodes (launches of the
checked lowering) than their fused variants: the option changed the partition (the
reference's own check of that is 2 fused nodes without it and 1 with it,
test/m4-fusion.test.js:55-63)."""
import sys

import numpy as np
import pytest

from oracle import bounds

pytestmark = pytest.mark.gpu

LOSES = ["broadcast-recompute-R16", "broadcast-recompute-R256", "broadcast-recompute-R4096", "lost-reuse-1op",
         "lost-reuse-16op"]


def test_fusion_loses_workloads_with_recompute(tmp_path, tool):
    import tcmi_bridge
    print(f"gpu step: gpu-workloads {LOSES} with every node", flush=True)
    tool("gpu-workloads", {"ids": LOSES, "allNodes": True}, out=str(tmp_path), timeout=600)
    b = tcmi_bridge.Bundle(tmp_path)
    assert [c["id"] for c in b.cases] == LOSES
    for c in b.cases:
        inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
        ref = bounds.reference_with_bounds(c["graph"], inputs)
        outs = c["outputs"]
        assert set(c["variants"]) == {"unfused", "fused", "recompute"}
        for v, r in c["variants"].items():
            j = bounds.judge_outputs([ref["values"][i] for i in outs], [ref["bounds"][i] for i in outs],
                                     [b.arr(x) for x in r["outputs"]])
            assert j["pass"] and r["canary"], (c["id"], v, "perf lowering", j["first"], r["canary"])
            if v == "unfused":
                continue
            gpu = [b.arr(x) for x in r["nodes"]]
            jf = bounds.judge_fused(r["fused"], r["origin"], gpu, ref)
            print(f"{c['id']} {v}: {r['launches']} launches, surviving nodes worst {jf['worst']:.3g}, outputs worst "
                  f"{j['worst']:.3g}", file=sys.stderr)
            assert jf["pass"] and r["canaryPlain"], (c["id"], v, jf["first"])
        # The partition: one launch per fused node in the checked lowering (the perf
        # lowering may form a shared value in its readers either way).
        assert c["variants"]["recompute"]["plainLaunches"] < c["variants"]["fused"]["plainLaunches"], c["id"]
        assert c["variants"]["recompute"]["launches"] <= c["variants"]["fused"]["launches"], c["id"]


def test_corpus_with_recompute(tmp_path, tool):
    import tcmi_bridge
    print("gpu step: gpu-fuzz programs 1..100 with recompute", flush=True)
    tool("gpu-fuzz", {"from": 1, "to": 100, "recompute": True}, out=str(tmp_path), timeout=600)
    b = tcmi_bridge.Bundle(tmp_path)
    assert b.manifest["recompute"] is True
    failures, graphs, worst = [], 0, 0.0
    for c in b.cases:
        graphs += 1
        inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
        ref = bounds.reference_with_bounds(c["graph"], inputs)
        if bounds.unjudgeable_count(ref["values"], ref["bounds"]) > 0:
            failures.append((c["program"], "unjudgeable"))
            continue
        nf = len(c["fused"]["nodes"])
        gf = [b.arr(c["gpuFused"][str(i)]) for i in range(nf)]
        jf = bounds.judge_fused(c["fused"], c["origin"], gf, ref)
        worst = max(worst, jf["worst"])
        if not (jf["pass"] and c["canary"]):
            failures.append((c["program"], c["label"], jf["first"], c["canary"]))
        for k, v in c["gpuPerf"].items():
            if not np.array_equal(b.arr(v).view(np.uint32), gf[int(k)].view(np.uint32)):
                failures.append((c["program"], c["label"], "perf lowering differs", int(k)))
    print(f"recompute corpus: {graphs} graphs, worst {worst:.3g}", file=sys.stderr)
    assert graphs == 200
    assert not failures, failures[:5]
