"""The bench's allocation counters and their self-test, on the GPU (the reference's
amendment 32: every object-creating call and every write counted, none allowed inside a
timed region, and a deliberate leak that must be caught, src/fusion/bench.js:41-47,
122-132,175-192): a fused program timed as the bench times it creates nothing; the same
timing with an allocation and a free inside every repetition throws with the counts; an
upload inside a timed region throws unless the region allows uploads (a training step's
batch)."""
import pytest

pytestmark = pytest.mark.gpu


def test_timed_regions_create_nothing_and_a_planted_leak_trips(tool):
    print("gpu step: gpu-bench-selftest", flush=True)
    r = tool("gpu-bench-selftest", timeout=120)
    assert r["clean"]["checked"] >= 1
    assert r["leak"]["threw"] is True, r["leak"]
    assert r["leak"]["created"]["malloc"] >= 2 and r["leak"]["created"]["free"] >= 2, r["leak"]
    assert r["upload"]["threw"] is True and r["upload"]["created"] == {"h2d": 1}, r["upload"]
    assert r["uploadAllowed"]["threw"] is False, r["uploadAllowed"]
