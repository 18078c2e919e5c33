"""bench.py's one-line record, composed on the CPU from a measurement document that
bench.js wrote on the MI355X (tests/golden/bench_document.json, a `--quick` run trimmed by
tests/golden/trim_bench_document.py): every field of the driver's contract is there with
its type, `value` is config 2's step rate, the roofline figure is the named kernel's
algorithmic bytes over its cold (HBM-read) duration against the 8 TB/s peak and does not
exceed the measured read ceiling, its HBM traffic comes from the committed profile that
names the same kernel, every config's figures and fusion-group verdicts are carried in a
compact `extra`, and the whole line stays small enough for the driver's output tail."""
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


def test_roofline_is_the_cold_figure_of_the_named_kernel(line):
    import bench
    doc, r = line
    rf = r["roofline"]
    dom = doc["configs"]["c2"]["dominant"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert rf["kernel"] == dom["code"]
    assert rf["kernel_avg_us"] == dom["cold"]["avgUs"]
    assert rf["achieved"] == pytest.approx(rf["bytes_per_launch"] / (rf["kernel_avg_us"] * 1e3))
    assert rf["frac"] == pytest.approx(rf["achieved"] / rf["peak"])
    # Cold: below the pure-read ceiling measured in the same run, and below the warm figure.
    assert rf["achieved"] <= rf["read_ceiling"] and rf["achieved"] < rf["warm_achieved"]
    assert rf["above_read_ceiling"] is False and rf["timing"].startswith("cold: operands read from HBM")
    # The rotation spans several times the 256 MB last-level cache.
    assert dom["cold"]["spanBytes"] >= 4 * 256 * 2 ** 20
    traffic, src = bench.profiled_traffic(rf["kernel"])
    assert rf["traffic"] == traffic and rf["traffic_source"] == src and traffic is not None
    assert abs(rf["traffic"] / rf["bytes_per_launch"] - 1) < 0.01


def test_every_config_is_carried_compactly(line):
    _, r = line
    ex = r["extra"]
    for k in ("c1", "c2", "c3", "c4", "c5", "attention", "sweep", "ceiling_1GiB_GBs", "timed_regions_checked"):
        assert k in ex, k
    assert ex["timed_regions_checked"] > 0
    for k in ("c1", "c2", "c3", "c5"):
        g = ex[k]["groups"]
        assert g["n"] == g["win"] + g["loss"] + g["noise"] > 0 and g["worst"]["verdict"] in ("win", "loss", "noise"), k
    assert ex["c4_groups"]["n"] > 0
    assert ex["c5"]["resident_steps_s"] >= ex["c5"]["steps_s"] * 0.9
    assert 0 < ex["c3"]["frac"] < 1
    assert all(0 < v["frac_fwd"] < 1 for v in ex["c4"].values())
    assert ex["sweep"]["timed"] == ex["sweep"]["gate_pass"] <= ex["sweep"]["workloads"]
    assert len(json.dumps(r, separators=(",", ":"))) < 6000


def test_a_cold_figure_above_the_read_ceiling_is_marked():
    """compose() marks a roofline figure above the pure-read ceiling of the same run as
    cache-assisted instead of reporting it as an HBM figure (planted: the document's cold
    figure raised to 1.1 times the ceiling)."""
    import bench
    doc = json.loads((ROOT / "tests" / "golden" / "bench_document.json").read_text())
    ceiling = doc["configs"]["ceiling"]["read"]["gbs"]
    doc["configs"]["c2"]["dominant"]["gbs"] = 1.1 * ceiling
    rf = bench.compose(doc)["roofline"]
    assert rf["above_read_ceiling"] is True and "cache-assisted" in rf["timing"]
