"""Trims a bench.js measurement document (`python bench.py --quick --no-cpu --out FILE`
on the MI355X) to the fields bench.py's compose() reads, for the fixture
bench_document.json that tests/test_bench_line.py composes a record from.

    python tests/golden/trim_bench_document.py FILE tests/golden/bench_document.json
"""
import json
import sys


def trim(doc: dict) -> dict:
    cfg = doc["configs"]
    for key in ("c2", "c3", "c4"):
        for r in cfg.get(key, {}).get("results", []):
            r.pop("launches", None)
            r.pop("launchF", None)
            r.pop("launchU", None)
            r.pop("groups", None)
    for key in ("c1", "c5"):
        if key in cfg:
            cfg[key]["byKind"] = {k: {"us": v["us"]} for k, v in cfg[key].get("byKind", {}).items()}
            cfg[key].pop("groupList", None)
    if "attention" in cfg:
        for r in cfg["attention"]["results"]:
            r["groups"] = [{k: g[k] for k in ("kernelUs", "replacedUs", "tflops")} for g in r.get("groups", [])]
    if "sweep" in cfg:
        sw = cfg["sweep"]
        sw["workloads"] = [{k: w[k] for k in ("id", "family", "fused", "recompute", "timed") if k in w} for w in sw["workloads"]]
    if "gate" in doc:
        doc["gate"] = {k: {"pass": v["pass"]} for k, v in doc["gate"].items()}
    return doc


if __name__ == "__main__":
    doc = trim(json.load(open(sys.argv[1])))
    with open(sys.argv[2], "w") as f:
        json.dump(doc, f, separators=(",", ":"))
