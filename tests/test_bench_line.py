"""bench.py's one-line record, composed on the CPU from a measurement document that
bench.js wrote on the MI355X (tests/golden/bench_document.json, a `--quick` run trimmed by
tests/golden/trim_bench_document.py): every field of the driver's contract is there with
its type, `value` is config 2's step rate, the roofline figure is the named kernel's
algorithmic bytes over its measured duration against the 8 TB/s peak, its HBM traffic comes
from the committed profile that names the same kernel, and the side figures of the other
configs are carried along."""
import json

import pytest

from conftest import ROOT


@pytest.fixture(scope="module")
def line():
    import bench
    doc = json.loads((ROOT / "tests" / "golden" / "bench_document.json").read_text())
    return doc, bench.compose(doc)


def test_contract_fields(line):
    doc, r = line
    for k, t in (("metric", str), ("value", float), ("unit", str), ("n_gpus", int), ("steps", int), ("warmup", int),
                 ("ms_per_step", float), ("higher_is_better", bool), ("scaling", str), ("dtype", str), ("data", str),
                 ("config", dict), ("roofline", dict)):
        assert isinstance(r[k], t), (k, r[k])
    assert r["n_gpus"] == 1 and r["higher_is_better"] is True and r["vs_baseline"] is None
    assert r["unit"] == "GB/s" and r["dtype"] == "f32" and r["data"] == "synthetic"
    assert "workload" in r["config"] and not ({"model", "global_batch", "seq_len"} & set(r["config"]))
    c2 = doc["configs"]["c2"]
    assert r["value"] == c2["gbs"] and r["ms_per_step"] == c2["msPerStep"]
    assert r["value"] == pytest.approx(c2["stepBytes"] / (c2["msPerStep"] * 1e6))


def test_roofline_of_the_named_kernel(line):
    import bench
    doc, r = line
    rf = r["roofline"]
    dom = doc["configs"]["c2"]["dominant"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert rf["kernel"] == dom["code"]
    assert rf["achieved"] == pytest.approx(rf["bytes_per_launch"] / (rf["kernel_avg_us"] * 1e3))
    assert rf["frac"] == pytest.approx(rf["achieved"] / rf["peak"])
    traffic, src = bench.profiled_traffic(rf["kernel"])
    assert rf["traffic"] == traffic and rf["traffic_source"] == src and traffic is not None
    # The kernel moves its algorithmic bytes: traffic within a percent of them.
    assert abs(rf["traffic"] / rf["bytes_per_launch"] - 1) < 0.01


def test_side_figures_are_carried(line):
    _, r = line
    ex = r["extra"]
    for k in ("rowwise_c3", "matmul_c4", "mlp_step_c1", "transformer_step_c5", "attention_extension", "workload_sweep",
              "c2_programs", "c2_step_sequential", "device", "ceiling_1GiB"):
        assert k in ex, k
    t = ex["transformer_step_c5"]
    assert t["steps_per_sec"] > 0 and t["resident_steps_per_sec"] >= t["steps_per_sec"] * 0.9
    assert t["dispatches"] < t["unbatched"]["dispatches"]
    assert 0 < ex["rowwise_c3"]["frac_hbm"] < 1
    assert all(0 < v["frac_mfma"] < 1 for v in ex["matmul_c4"].values())
