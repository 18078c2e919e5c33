"""The liveness arena of the perf path (js/src/mi355x/arena.js), checked on the CPU.

Every plan is run abstractly over the arena's bytes (js/src/testing/arena_check.js):
each launch must find its operands still holding their own values, must not write over
an operand it reads, and every pinned buffer (inputs, constants, kept outputs) must
survive to the end. The plan's size is compared with the peak of live bytes over the
launch list, which no placement can go under. The GPU side (the trainer with an arena,
bit for bit the checked path) is in test_gpu_train.py."""

MODELS = [{"model": "transformer", "B": 64}, {"model": "transformer", "B": 1}, {"model": "mlp"},
          {"model": "transformer-ref"}, {"model": "transformer", "B": 64, "attention": True},
          {"model": "transformer-ref", "attention": True}]


def test_arena_plans_keep_every_value_until_its_last_use(tool):
    res = tool("arena-check", {"models": MODELS, "corpus": {"from": 1, "to": 300}})
    assert len(res) == len(MODELS) + 600
    bad = [r for r in res if not r["check"]["ok"]]
    assert not bad, bad[:3]
    for r in res:
        # First fit by decreasing size lands within a few percent of the lower bound here.
        assert r["peak"] <= r["bytes"] <= max(256, r["peak"]) * 1.03 + 4096, r
        assert r["bytes"] <= r["unshared"]
    c5 = next(r for r in res if r["name"] == "transformer-64")
    # Config 5's step: 1.29 GB of node buffers in 0.80 GB (the values its launches form in
    # place have no buffer at all, so what is left to share is mostly live at once).
    assert c5["bytes"] < 0.65 * c5["unshared"] and c5["bytes"] < 0.85e9, c5


def test_a_planted_overlap_is_caught(tool):
    """One buffer moved onto another that is live at the same time: the simulation refuses
    every such plan (the check is not the planner's own interval arithmetic)."""
    res = tool("arena-check", {"models": MODELS[:1] + MODELS[2:3], "corpus": {"from": 1, "to": 50}, "plant": True})
    planted = [r for r in res if "planted" in r]
    assert len(planted) > 50
    assert all(not r["planted"]["check"]["ok"] for r in planted), [r["name"] for r in planted if r["planted"]["check"]["ok"]]


def test_batched_launches_share_one_position(tool):
    """The members of a batched launch run concurrently, so the arena places them at one
    position. A plan that takes them one after another lets a later member's output reuse
    the bytes of an earlier member's last operand: the simulation, which reads and writes
    a batch as one step, refuses that plan for config 5's step and some corpus programs."""
    res = tool("arena-check", {"models": MODELS[:1], "corpus": {"from": 1, "to": 50}, "plant": True})
    blind = [r for r in res if "batchBlind" in r]
    assert any(r["name"] == "transformer-64" for r in blind)
    assert all(r["check"]["ok"] for r in blind)
    caught = [r["name"] for r in blind if not r["batchBlind"]["ok"]]
    assert "transformer-64" in caught and len(caught) >= 3, caught
