"""GPU parity of the three fused kernel classes on the reference's 100 direct
adversarial cases: each case fused into its one kernel, run on the MI355X through
the Node host and the C ABI with canary-padded buffers, and every surviving node
judged against the float64 oracle within the float32 budget (S = 2, the
reference's bound; judgeFused, harness-m4.js:46-60). Canaries must be intact."""
import sys

import numpy as np
import pytest

from oracle import bounds

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def direct_bundle(tmp_path_factory, tool):
    import tcmi_bridge
    d = tmp_path_factory.mktemp("direct")
    print("gpu step: gpu-direct (100 fused direct cases)", flush=True)
    tool("gpu-direct", out=str(d), timeout=600)
    return tcmi_bridge.Bundle(d)


def test_direct_cases_within_float32_budget(direct_bundle):
    b = direct_bundle
    assert len(b.cases) == 100
    worst = {}
    failures = []
    for c in b.cases:
        inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
        ref = bounds.reference_with_bounds(c["graph"], inputs)
        assert bounds.unjudgeable_count(ref["values"], ref["bounds"]) == 0, c["name"]
        gpu = [b.arr(c["gpu"][str(i)]) for i in range(len(c["fused"]["nodes"]))]
        j = bounds.judge_fused(c["fused"], c["origin"], gpu, ref)
        worst[c["pattern"]] = max(worst.get(c["pattern"], 0.0), j["worst"])
        if not j["pass"]:
            failures.append((c["name"], j["worst"], j["first"]))
        if not all(c["canaryIntact"]):
            failures.append((c["name"], "canary", c["canaryIntact"]))
    print("worst ratio by pattern:", worst, file=sys.stderr)
    assert not failures, failures[:5]


def test_direct_cases_launch_the_intended_kernel(direct_bundle):
    for c in direct_bundle.cases:
        kinds = [l["kind"] for l in c["launches"]]
        assert kinds == [f"fused-{c['kind']}"], (c["name"], kinds)
