"""Benchmark of the MI355X fused-kernel backend; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c2,c3,c4] [--quick]

The headline (`value`) is config 2 of the benchmark, the one its metric is
quoted on first: fused elementwise chains — 8 seeded programs of 8–16 ops over
fp32 [8192, 1024] with a [1024] row-vector broadcast, each run forward and as
its autodiff gradient graph — in algorithmic HBM GB/s (every unique operand of
a launch read once at its own size, plus its output: the reference's byte
count, src/fusion/workloads.js:171-172). A step is one run of every fused
program; K steps are timed between a sync and hipEvents on both sides, with the
inputs already in HBM.

Rowwise (config 3) GB/s and matmul (config 4) TFLOP/s are reported beside it,
with fused-vs-unfused speedups per program. `roofline` is the dominant kernel
of the headline workload; `cpu_baseline` is the float64 oracle
(oracle/interp.py, the restated reference interpreter) timed single-threaded
on this host on a bounded sample of the same workload.

The GPU work runs in a node child process (the Node host over the N-API addon
and the C ABI); this process never touches the GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import subprocess
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
PKG = ROOT / "tensor-compiler-webgpu_amd"
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(PKG))

METRIC = "fused-kernel HBM GB/s + matmul TFLOP/s (% roofline); transformer train steps/sec"
HBM_PEAK = 8000.0
MFMA_FP32_PEAK = 157.3


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def cpu_baseline(rows: int, seeds, min_seconds: float = 10.0) -> dict:
    """The oracle's float64 interpreter, one thread, on C2 programs at `rows` of 8192 rows:
    passes over every program (forward and gradient) until at least `min_seconds` of CPU
    work have been timed (a bounded sample, so the bench still ends within minutes)."""
    import numpy as np
    import tcmi_bridge
    from oracle import interp
    C = 1024
    graphs = tcmi_bridge.node_tool("chain-graphs", {"seeds": list(seeds), "R": rows, "C": C})
    rng = np.random.default_rng(12345)
    feeds = []
    for g in graphs:
        feeds.append({"x0": rng.standard_normal(rows * C).astype(np.float32),
                      "x1": rng.standard_normal(rows * C).astype(np.float32),
                      "r": rng.standard_normal(C).astype(np.float32),
                      "d0": rng.standard_normal(rows * C).astype(np.float32)})
    total_bytes = 0
    passes = 0
    t0 = time.perf_counter()
    while passes == 0 or time.perf_counter() - t0 < min_seconds:
        for g, feed in zip(graphs, feeds):
            interp.evaluate(g["forward"]["graph"], {k: v for k, v in feed.items() if k != "d0"})
            interp.evaluate(g["gradient"]["graph"], feed)
            total_bytes += g["forward"]["fusedBytes"] + g["gradient"]["fusedBytes"]
        passes += 1
    secs = time.perf_counter() - t0
    return {"value": total_bytes / secs / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"C2 programs {list(seeds)} forward+gradient at [{rows},{C}] ({rows}/8192 of the rows), "
                      f"{passes} pass(es), float64 numpy interpreter, {secs:.1f} s on {cpu_model()} "
                      f"({os.cpu_count()} cores visible, 1 used)",
            "seconds": secs}


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from a committed rocprofv3 --pmc summary
    (profiles/*.md, the json block profile_summary.py writes: {"traffic_bytes_per_launch":
    {kernel: bytes}}), or None when no profile covers that kernel."""
    for md in sorted((ROOT / "profiles").glob("*.md")):
        text = md.read_text()
        if "```json" not in text:
            continue
        block = text.split("```json", 1)[1].split("```", 1)[0]
        try:
            rec = json.loads(block)
        except ValueError:
            continue
        traffic = rec.get("traffic_bytes_per_launch")
        if isinstance(traffic, dict) and kernel in traffic:
            return traffic[kernel], md.name
    return None, None


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--configs", default="ceiling,c2,c3,c4,c1,c5,attention,sweep")
    ap.add_argument("--programs", type=int, default=8)
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--out", default=None, help="also write the full measurement JSON here")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    cmd = ["node", str(PKG / "js" / "cli" / "bench.js"), "--configs", a.configs, "--steps", str(a.steps),
           "--warmup", str(a.warmup), "--programs", str(a.programs)]
    if a.quick:
        cmd.append("--quick")
    p = subprocess.run(cmd, stdout=subprocess.PIPE)
    if p.returncode != 0:
        print(f"bench.py: node bench exited {p.returncode}", file=sys.stderr)
        sys.exit(p.returncode)
    full = json.loads(p.stdout)
    if a.out:
        pathlib.Path(a.out).write_text(json.dumps(full, indent=1))
    line = compose(full)
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline(8192 if not a.quick else 256, range(min(a.programs, 8)), 0.0 if a.quick else 10.0)
    print(json.dumps(line))


def compose(full: dict) -> dict:
    """The driver's one-line record from bench.js's measurement document (everything but
    the CPU baseline, which this process times itself)."""
    cfg = full["configs"]
    c2 = cfg.get("c2")
    extra = {}
    if "c3" in cfg:
        c3 = cfg["c3"]
        extra["rowwise_c3"] = {"GBs": c3["gbs"], "frac_hbm": c3["gbs"] / HBM_PEAK,
                               "dominant": {k: c3["dominant"][k] for k in ("code", "pattern", "avgUs", "gbs")},
                               "programs": {r["name"]: {"fused_us": r["fused"]["median"], "unfused_us": r["unfused"]["median"],
                                                        "speedup": r["verdict"]["speedup"], "verdict": r["verdict"]["verdict"],
                                                        "GBs": r["gbs"]["fused"]} for r in c3["results"]}}
    if "c4" in cfg:
        c4 = cfg["c4"]
        extra["matmul_c4"] = {r["name"]: {"fused_us": r["fused"]["median"], "TFLOPs": (r["tflops"] or {}).get("fused"),
                                          "frac_mfma": ((r["tflops"] or {}).get("fused") or 0) / MFMA_FP32_PEAK,
                                          "speedup_vs_unfused": r["verdict"]["speedup"]} for r in c4["results"]}
    for key, label in (("c1", "mlp_step_c1"), ("c5", "transformer_step_c5")):
        if key in cfg:
            t = cfg[key]
            extra[label] = {"steps_per_sec": t["stepsPerSec"], "ms_per_step": t["msPerStep"], "hip_graph_replay": t["graphReplay"],
                            "resident_steps_per_sec": t["residentStepsPerSec"], "resident_ms_per_step": t["residentMsPerStep"],
                            "launches": t["launches"], "fused_us": t["fused"]["median"], "unfused_us": t["unfused"]["median"],
                            "speedup_vs_unfused": t["verdict"]["speedup"], "matmul_TFLOPs_resident": t["matmulTflopsResident"],
                            "loss": t["lossLast"], "time_by_kind_us": {k: round(v["us"], 1) for k, v in t["byKind"].items()},
                            "arena": {"bytes": t["arena"]["bytes"], "unshared_bytes": t["arena"]["unshared"],
                                      "steps_per_sec": t["arena"]["stepsPerSec"],
                                      "resident_steps_per_sec": t["arena"]["residentStepsPerSec"]},
                            "dispatches": t["dispatches"], "batched_launches": t["batches"],
                            "unbatched": {"dispatches": t["unbatched"]["dispatches"],
                                          "steps_per_sec": t["unbatched"]["stepsPerSec"],
                                          "resident_steps_per_sec": t["unbatched"]["residentStepsPerSec"]}}
    if "attention" in cfg:
        extra["attention_extension"] = {
            r["name"]: {"contract_us": r["contract"]["median"], "attention_us": r["attention"]["median"],
                        "speedup": r["verdict"]["speedup"], "verdict": r["verdict"]["verdict"], "launches": r["launches"],
                        "max_abs_diff_logits": r["maxAbsDiffLogits"],
                        "kernel_us": sum(g["kernelUs"] for g in r["groups"]) / len(r["groups"]),
                        "replaced_launches_us": sum(g["replacedUs"] for g in r["groups"]) / len(r["groups"]),
                        "kernel_TFLOPs": sum(g["tflops"] for g in r["groups"]) / len(r["groups"])}
            for r in cfg["attention"]["results"]}
    if "sweep" in cfg:
        sw = cfg["sweep"]
        extra["workload_sweep"] = {
            "workloads": len(sw["workloads"]), "families": sw["families"],
            "fusion_loses_by_design": {r["id"]: {"fused_vs_unfused": round(r["fused"]["speedup"], 3), "verdict": r["fused"]["verdict"],
                                                 **({"recompute_vs_fused": round(r["recompute"]["speedup"], 3),
                                                     "recompute_verdict": r["recompute"]["verdict"]} if "recompute" in r else {})}
                                       for r in sw["workloads"] if r["family"] in ("broadcast-recompute", "lost-reuse")}}
    if c2 is None:
        raise SystemExit("bench.py: the headline needs config c2")
    dom = c2["dominant"]
    extra["c2_programs"] = {r["name"]: {"fused_us": r["fused"]["median"], "unfused_us": r["unfused"]["median"],
                                        "speedup": r["verdict"]["speedup"], "verdict": r["verdict"]["verdict"],
                                        "GBs": r["gbs"]["fused"], "bitwise_same_outputs": r["bitwiseSameOutputs"]}
                            for r in c2["results"]}
    seq = c2["schedule"].get("sequential")
    if seq:
        extra["c2_step_sequential"] = {"GBs": seq["gbs"], "ms_per_step": seq["msPerStep"],
                                       "note": "every program after the previous on one stream"}
    extra["device"] = {k: full["device"].get(k) for k in ("name", "arch", "computeUnits", "clockKHz", "totalMemory")}
    if "ceiling" in cfg:
        extra["ceiling_1GiB"] = {"copy_GBs": cfg["ceiling"]["copy"]["gbs"], "read_GBs": cfg["ceiling"]["read"]["gbs"]}
    traffic, traffic_src = profiled_traffic(dom["code"])
    line = {
        "metric": METRIC, "value": c2["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": c2["steps"], "warmup": c2["warmup"],
        "ms_per_step": c2["msPerStep"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "C2: fused elementwise chains, seeded programs of 8-16 ops (forward + autodiff gradient) "
                               "over fp32 [8192,1024] with a [1024] row broadcast",
                   "programs": c2["programs"], "shape": c2["shape"], "step_bytes": c2["stepBytes"],
                   "schedule": f"the {2 * c2['programs']} independent programs issued over {c2['schedule']['streams']} "
                               "streams, balanced by bytes"},
        "roofline": {"bound": "hbm", "achieved": dom["gbs"], "peak": HBM_PEAK, "unit": "GB/s", "frac": dom["gbs"] / HBM_PEAK,
                     "traffic": traffic, "traffic_source": traffic_src, "kernel": dom["code"], "kernel_avg_us": dom["avgUs"],
                     "bytes_per_launch": dom["bytesPerLaunch"], "launches_per_step": dom["count"]},
        "extra": extra,
    }
    return line


if __name__ == "__main__":
    main()
