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


# The reference's four kernel sabotages (harness-m4.js:33-39) and the kernels each targets.
SABOTAGES = {
    "epilogue-before-bias": lambda c: c["kind"] == "epilogue",
    "layernorm-tree-short": lambda c: c["pattern"] == "layernorm",
    "softmax-no-max": lambda c: c["pattern"] in ("softmax", "log-softmax"),
    "fused-bounds-off-by-one": lambda c: c["kind"] == "elementwise",
}


@pytest.mark.parametrize("sabotage", list(SABOTAGES))
def test_kernel_sabotage_is_caught(sabotage, tmp_path, tool):
    """Each of the reference's kernel sabotages, planted in this backend's kernels, is caught
    by the direct cases' checks (the float32 budget or the canaries), and only in the kernels
    it targets. The off-by-one kernel reads and writes one element past its buffers, inside
    the canary pad every check-mode buffer carries (the runner refuses it without one)."""
    import tcmi_bridge
    print(f"gpu step: gpu-direct with sabotage {sabotage}", flush=True)
    tool("gpu-direct", {"sabotage": sabotage}, out=str(tmp_path), timeout=600)
    b = tcmi_bridge.Bundle(tmp_path)
    assert b.manifest["sabotage"] == sabotage
    targeted = SABOTAGES[sabotage]
    caught, missed, collateral = [], [], []
    for c in b.cases:
        inputs = {k: b.arr(v) for k, v in c["inputs"].items()}
        ref = bounds.reference_with_bounds(c["graph"], inputs)
        gpu = [b.arr(c["gpu"][str(i)]) for i in range(len(c["fused"]["nodes"]))]
        j = bounds.judge_fused(c["fused"], c["origin"], gpu, ref)
        failed = (not j["pass"]) or not all(c["canaryIntact"])
        if targeted(c):
            (caught if failed else missed).append(c["name"])
        elif failed:
            collateral.append(c["name"])
    print(f"{sabotage}: caught in {len(caught)} of {len(caught) + len(missed)} targeted cases", file=sys.stderr)
    assert caught, f"sabotage {sabotage} was not caught"
    assert not collateral, collateral[:5]
