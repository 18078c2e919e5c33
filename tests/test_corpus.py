"""The reference's fuzzing corpus, restated (js/src/testing/random_graph.js), pinned to
what the reference's own files record about it:

- golden/cases.json holds 40 graphs made by the reference's generator (v2-random-1..25
  and three targeted programs for each of matmul, transpose, reshape, broadcast, sum):
  the restated generator makes exactly those node lists and outputs;
- golden/measurements.json m4.semantics.corpus records what the fusion pass makes of
  corpus programs 1..2000 (forward and gradient graphs: 4000 graphs, how many hold a
  fused node, how many fused nodes of each pattern), m4.passSabotage what the pass
  sabotage changes on programs 1..500, and golden/gpu-m4.json fuzz the structure of the
  reference's GPU fuzzer over the same corpus (runs, runs with a fused node, kinds and
  patterns per run). The restated generator, builder, autodiff and fusion pass
  reproduce every one of those counts; a planted change (one program's seed shifted)
  moves them."""


def test_generator_reproduces_the_golden_v2_programs(golden_cases, tool):
    cases = {c["name"]: c for c in golden_cases}
    reqs = [{"seed": i} for i in range(1, 26)]
    reqs += [{"seed": i, "focus": op} for op in ("matmul", "transpose", "reshape", "broadcast", "sum") for i in (1, 2, 3)]
    out = tool("random-programs", {"programs": reqs})
    assert len(out) == 40
    for r in out:
        name = f"v2-random-{r['seed']}" if not r["focus"] else f"v2-{r['focus']}-{r['seed']}"
        c = cases[name]
        assert r["graph"]["nodes"] == c["graph"]["nodes"], name
        assert r["outputs"] == c["outputs"], name


def test_fusion_over_the_corpus_matches_the_recorded_counts(m4_counts, tool):
    got = tool("corpus-fusion", {"from": 1, "to": 2000, "sabotageTo": 500}, timeout=300)
    want = m4_counts["corpus"]
    for k in ("graphs", "withFused", "fusedNodes", "byPattern"):
        assert got["semantics"][k] == want[k], (k, got["semantics"][k], want[k])
    fz = m4_counts["fuzz"]
    for k in ("runs", "fusedRuns", "byKind", "byPattern"):
        assert got["fuzz"][k] == fz[k], (k, got["fuzz"][k], fz[k])
    sab = m4_counts["passSabotage"]
    for k in ("graphs", "changed", "threw"):
        assert got["passSabotage"][k] == sab[k], (k, got["passSabotage"][k], sab[k])


def test_corpus_counts_see_a_planted_change(m4_counts, tool):
    """Programs 2..2001 in place of 1..2000: the same number of graphs, other counts."""
    got = tool("corpus-fusion", {"from": 2, "to": 2001}, timeout=300)
    assert got["semantics"]["graphs"] == m4_counts["corpus"]["graphs"]
    assert got["semantics"]["byPattern"] != m4_counts["corpus"]["byPattern"]
