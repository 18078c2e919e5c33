"""Batched launches of the perf lowering (js/src/mi355x/lower.js batchPlan), checked on the
CPU by js/src/testing/batch_check.js from the launch records alone: the batched list holds
the plain list's launches, every launch reads only buffers written before it, a batch's
members are launches of one kernel text (or of matmul, elementwise or rowwise texts of one
grid, each member then run by its own case of the batched kernel) with no data path
between them, the batched grid has one z-slice per member, and launches that share the
workspace keep their order. A ragged batch's members (small kernels whose grids differ)
each run their own branch over their own range of the dispatch's workgroups. Planted
mistakes (a batch whose second member reads the first's output; a launch moved in front of
its operand's writer; a member over another grid; members' bodies exchanged) must be
refused. The GPU side, batched runs bit for bit the plain ones, is in test_gpu_train.py
(configs 1 and 5's steps) and test_gpu_fuzz.py (corpus programs)."""

MODELS = [{"model": "transformer", "B": 64}, {"model": "transformer", "B": 1}, {"model": "mlp"},
          {"model": "transformer-ref"}, {"model": "transformer", "B": 64, "attention": True},
          {"model": "transformer-ref", "attention": True}]


def test_batched_launch_lists_are_valid_orders(tool):
    res = tool("batch-check", {"models": MODELS, "corpus": {"from": 1, "to": 400}})
    assert len(res) == len(MODELS) + 800
    bad = [r for r in res if not r["check"]["ok"]]
    assert not bad, bad[:3]
    c5 = next(r for r in res if r["name"] == "transformer-64")
    # Config 5's step: the q/k/v projections and their head transposes per layer, the
    # score-gradient matmul pairs and the per-tensor parameter updates batch.
    assert c5["check"]["batches"] >= 12 and c5["check"]["saved"] >= 40, c5
    assert sum(1 for r in res if r["check"]["batches"]) > 120


def test_planted_batch_mistakes_are_caught(tool):
    """Four planted mistakes: a batch whose second member reads the first's output; a
    launch moved in front of its operand's writer; a member whose kernel has the same
    text over another grid (a column sum's text leaves its outer extent to the grid:
    batching two such launches by name alone once ran one member over the other's grid,
    which the GPU fuzz test caught as a canary overwrite and as perf-lowering
    differences in 3 of 4000 corpus graphs); two members of a batch whose members run
    different bodies (matmuls, or elementwise chains of one grid) exchanged, so that each
    member's case of the batched kernel holds the other's body."""
    res = tool("batch-check", {"models": MODELS[:1], "corpus": {"from": 1, "to": 900}, "plant": True})
    dep = [r for r in res if "dependent" in r]
    early = [r for r in res if "early" in r]
    grid = [r for r in res if "grid" in r]
    # A dependent pair needs two launches of one kernel outside any batch: ragged batches
    # leave fewer of those (8 in this corpus).
    assert len(dep) >= 5 and len(early) >= 100 and len(grid) >= 20
    assert all(not r["dependent"]["ok"] for r in dep)
    assert all(not r["early"]["ok"] for r in early)
    assert all(not r["grid"]["ok"] and "member" in r["grid"]["why"] for r in grid), [r["grid"] for r in grid if r["grid"]["ok"]]
    body = [r for r in res if "body" in r]
    assert len(body) >= 100 and any(r["name"] == "transformer-64" for r in body)
    assert all(not r["body"]["ok"] and "member" in r["body"]["why"] for r in body), [r["name"] for r in body if r["body"]["ok"]]


def test_same_text_over_another_grid_is_not_batched(tool):
    """Corpus programs 935, 1101 and 1391 (gradient) hold column sums of one kernel text
    over different outer extents (grids): no batch mixes them."""
    res = tool("batch-check", {"corpus": {"from": 935, "to": 935}})
    res += tool("batch-check", {"corpus": {"from": 1101, "to": 1101}})
    res += tool("batch-check", {"corpus": {"from": 1391, "to": 1391}})
    assert all(r["check"]["ok"] for r in res), res


def test_headers_never_read_the_z_index():
    """A batched kernel is the member kernel's text with its z index rewritten to
    blockIdx.z % Z: that is complete only if no device header reads blockIdx.z or
    gridDim.z itself (the matmul takes its z index as an argument). The one exception
    is tcmi::xcd_grouped, which places a workgroup over the whole launch's grid on
    purpose; a batched kernel that calls it chooses its member from that place's z
    index (test_xcd_grouped_batches_choose_members_by_place)."""
    import pathlib
    import re
    kernels = pathlib.Path(__file__).resolve().parents[1] / "tensor-compiler-webgpu_amd" / "csrc" / "kernels"
    grouped = 0
    for h in sorted(kernels.glob("*.h")):
        code = "\n".join(line.split("//")[0] for line in h.read_text().splitlines())
        code, n = re.subn(r"__device__ __forceinline__ Wg xcd_grouped\(\) \{.*?\n\}", "", code, flags=re.S)
        grouped += n
        assert not re.search(r"\b(blockIdx|gridDim)\.z\b", code), h.name
    assert grouped == 1


def test_xcd_grouped_batches_choose_members_by_place(tool):
    """Config 5's weight gradients are split-K products batched 16 and 4 at a time:
    each member kernel takes its place from tcmi::xcd_grouped, and its batched form
    takes that place once, over the whole batched grid, chooses the member by the
    place's z index and hands the member the rest of it, never blockIdx.z."""
    r = tool("grouped-batches", {"model": "transformer", "B": 64})
    assert r["batches"] >= 3, r
    for k in r["kernels"]:
        src = k["source"]
        assert src.count("const tcmi::Wg wg = tcmi::xcd_grouped();") == 1, k["name"]
        assert f"B.m[wg.z / {k['z']}u]" in src and f"(wg.z % {k['z']}u), wg.x, wg.y)" in src, k["name"]
        assert "blockIdx" not in src, k["name"]


def test_a_producer_of_constants_is_not_absorbed(tool):
    """Corpus program 1285 (forward) holds a fused chain of constants alone ([1, 1], no
    operands) read by one elementwise node: absorbing it would leave its reader's slot
    with no operand, so it stays a launch, and the lowering (producers absorbed, as the
    trainer lowers) goes through."""
    res = tool("batch-check", {"corpus": {"from": 1285, "to": 1285}})
    assert len(res) == 2 and all(r["check"]["ok"] for r in res), res


def test_ragged_batches_cover_each_member_grid_once(tool):
    """Ragged batches (launches of small kernels whose grids differ, in one dispatch:
    codegen.js raggedKernel): read back from each batched kernel's text, the branch a
    workgroup L takes and the place it gives the member's body, simulated for every L of
    the dispatch, cover every member's own grid exactly once, in member order, and the
    dispatch has no workgroup beyond the last member's. Config 1's step then runs in as
    many dispatches as its longest chain of dependent launches (5: its bias updates run
    inside their column sums' launches)."""
    import re
    res = tool("ragged-batches", {"models": [{"model": "mlp"}, {"model": "transformer", "B": 64, "attention": True}],
                                  "corpus": {"from": 1, "to": 60}})
    assert any(r["name"] == "mlp-" for r in res) and sum(1 for r in res if r["name"].startswith("corpus")) >= 20
    head = re.compile(r"if \(tcmi_wg_ < (\d+)u\) \{.*?\n\s*const uint32_t tcmi_l_ = tcmi_wg_ - (\d+)u;\n\s*const TcmiPtrs& A = B\.m\[(\d+)\];\n"
                      r"\s*const uint3 gridDim = make_uint3\((\d+)u, (\d+)u, (\d+)u\);\n"
                      r"\s*const uint3 blockIdx = make_uint3\(tcmi_l_ % (\d+)u, \(tcmi_l_ / (\d+)u\) % (\d+)u, tcmi_l_ / (\d+)u\);")
    for r in res:
        branches = [tuple(int(x) for x in m.groups()) for m in head.finditer(r["source"])]
        assert len(branches) == len(r["members"]), r["name"]
        assert r["grid"][1:] == [1, 1] and all(m["block"] == r["block"] for m in r["members"])
        seen = [set() for _ in r["members"]]
        for L in range(r["grid"][0]):
            # The if / else-if chain: the first branch whose bound exceeds L.
            k = next(i for i, b in enumerate(branches) if L < b[0])
            bound, start, member, gx, gy, gz, mx, dx, my, dz = branches[k]
            assert member == k and (gx, gy, gz) == tuple(r["members"][k]["grid"]) and (mx, dx, my, dz) == (gx, gx, gy, gx * gy)
            l = L - start
            assert 0 <= l
            place = (l % mx, (l // dx) % my, l // dz)
            assert place not in seen[k]
            seen[k].add(place)
        for k, m in enumerate(r["members"]):
            gx, gy, gz = m["grid"]
            assert seen[k] == {(x, y, z) for x in range(gx) for y in range(gy) for z in range(gz)}, (r["name"], k)
    c1 = tool("batch-check", {"models": [{"model": "mlp"}]})[0]
    assert c1["check"]["ok"] and c1["launches"] - c1["check"]["saved"] == 5, c1
