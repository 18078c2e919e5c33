"""The reference's differential GPU fuzzer (src/gpu/harness-m4.js:126-172) over its own
corpus (programs 1..2000: each program and its gradient graph, 4000 graphs, with the
inputs and cotangents the reference draws), on the MI355X: every graph fused (plain
lowering), fused in the perf lowering, and unfused, canary-padded. Every node of the
fused graph and of the unfused graph is judged against the float64 oracle within the
float32 budget (S = 2); a program is skipped, as in the reference, only if a node of
its reference is unjudgeable (the reference recorded 0 skipped programs and every run
passing, golden/gpu-m4.json fuzz). The perf lowering's kept outputs equal the plain
fused ones bit for bit; the number of graphs whose fused and unfused values agree bit
for bit at every surviving node is reported."""
import sys

import numpy as np
import pytest

from oracle import bounds

pytestmark = pytest.mark.gpu


def _judge_part(b):
    skipped_programs, failures, same, graphs = set(), [], 0, 0
    worst_f = worst_u = 0.0
    for c in b.cases:
        graphs += 1
        inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
        ref = bounds.reference_with_bounds(c["graph"], inputs)
        if bounds.unjudgeable_count(ref["values"], ref["bounds"]) > 0:
            skipped_programs.add(c["program"])
            continue
        nf = len(c["fused"]["nodes"])
        gf = [b.arr(c["gpuFused"][str(i)]) for i in range(nf)]
        gu = [b.arr(c["gpuUnfused"][str(i)]) for i in range(len(c["graph"]["nodes"]))]
        jf = bounds.judge_fused(c["fused"], c["origin"], gf, ref)
        ju = bounds.judge(c["graph"], gu, ref["values"], ref["bounds"])
        worst_f, worst_u = max(worst_f, jf["worst"]), max(worst_u, ju["worst"])
        if not (jf["pass"] and ju["pass"] and c["canary"]):
            failures.append((c["program"], c["label"], jf["first"], ju["first"], c["canary"]))
        for k, v in c["gpuPerf"].items():
            if not np.array_equal(b.arr(v).view(np.uint32), gf[int(k)].view(np.uint32)):
                failures.append((c["program"], c["label"], "perf lowering differs", int(k)))
        if all(np.array_equal(gf[i].view(np.uint32), gu[c["origin"][i]].view(np.uint32)) for i in range(nf)):
            same += 1
    return skipped_programs, failures, same, graphs, worst_f, worst_u


def test_fuzz_corpus_on_the_gpu(tmp_path, tool, m4_counts):
    import tcmi_bridge
    skipped, failures, same, graphs = set(), [], 0, 0
    worst_f = worst_u = 0.0
    for lo, hi in ((1, 1000), (1001, 2000)):
        d = tmp_path / f"fuzz-{lo}"
        print(f"gpu step: gpu-fuzz programs {lo}..{hi}", flush=True)
        tool("gpu-fuzz", {"from": lo, "to": hi}, out=str(d), timeout=900)
        s, f, sm, g, wf, wu = _judge_part(tcmi_bridge.Bundle(d))
        skipped |= s
        failures += f
        same += sm
        graphs += g
        worst_f, worst_u = max(worst_f, wf), max(worst_u, wu)
    print(f"fuzz: {graphs} graphs, {len(skipped)} programs skipped, worst fused {worst_f:.3g} unfused {worst_u:.3g}, "
          f"fused = unfused bit for bit in {same} graphs", file=sys.stderr)
    assert graphs == 4000
    assert len(skipped) == m4_counts["fuzz"]["skipped"] == 0
    assert not failures, failures[:5]
