"""The stream schedule of the perf path (js/src/mi355x/schedule.js), checked on the CPU.

Every schedule (configs 1 and 5, the reference transformer, 400 corpus graphs, at 2, 3
and 4 streams) is replayed with vector clocks (js/src/testing/schedule_check.js), the
way in-order streams and event waits order work: each launch must run after the launch
that wrote each operand it reads and after the previous workspace user. Dropping any
one wait must be caught. The GPU side (trainers on several streams, bit for bit the
single-stream results) is in test_gpu_train.py."""


def test_schedules_order_every_dependency(tool):
    res = tool("schedule-check", {"models": [{"model": "transformer", "B": 64}, {"model": "mlp"},
                                             {"model": "transformer-ref"},
                                             {"model": "transformer", "B": 64, "attention": True}],
                                  "corpus": {"from": 1, "to": 200}})
    assert len(res) == 3 * (4 + 400)
    bad = [r for r in res if not r["check"]["ok"]]
    assert not bad, bad[:3]
    c5 = [r for r in res if r["name"] == "transformer-64"]
    # Config 5's step: 212 launches (the dead ones not launched, the row reductions and the
    # producers of their operands folded into their chains, producers formed by their
    # readers, row and full-size values formed by theirs, column sums included, the
    # attention heads read back into rows through mapped views, the MLP's relu applied by
    # the matmuls reading it) on a dependency chain of under 200; every stream gets work.
    # Its bias gradients sum too many rows to take their updates in (two passes).
    assert all(r["launches"] == 212 and r["criticalPath"] < 200 and r["used"] == r["streams"] for r in c5), c5
    # With attention and its gradient fused (fusion/attention.js): 196 launches.
    c5a = [r for r in res if r["name"] == "transformer-64-attention"]
    assert all(r["launches"] == 196 and r["used"] == r["streams"] for r in c5a), c5a


def test_a_dropped_wait_is_caught(tool):
    res = tool("schedule-check", {"models": [{"model": "transformer", "B": 64}, {"model": "mlp"}],
                                  "corpus": {"from": 1, "to": 60}, "plant": True})
    planted = [r for r in res if "planted" in r]
    assert len(planted) > 100
    assert all(not r["planted"]["ok"] for r in planted), [r["name"] for r in planted if r["planted"]["ok"]][:5]
