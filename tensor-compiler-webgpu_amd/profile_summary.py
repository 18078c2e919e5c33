"""Per-kernel roofline table from rocprofv3 runs of the Node bench.

    python tensor-compiler-webgpu_amd/profile_summary.py --bench STEP_ONLY.json \
        --stats TRACE_kernel_stats.csv --fetch FETCH_counter_collection.csv \
        --write WRITE_counter_collection.csv [--mfma MFMA_counter_collection.csv] \
        [--events FULL_BENCH.json --events-stats FULL_kernel_stats.csv] [--configs c2,c3,c4]

Inputs are what `node js/cli/bench.js --step-only` prints (every launch of every
program with its kernel names, algorithmic bytes and flops) and the CSV files that
`rocprofv3 --kernel-trace --stats -f csv` and `rocprofv3 --pmc FETCH_SIZE` /
`--pmc WRITE_SIZE` (and optionally `--pmc MfmaUtil MfmaFlopsF32 LDSBankConflict`)
write for the same command. The counter passes are calibrated on the bench's 1 GiB
copy kernel (k_copy16, run in the same process by `--configs ceiling,...`): the
factor that turns its FETCH_SIZE and WRITE_SIZE (KiB per dispatch) into 1 GiB is
applied to every kernel.

Prints a markdown table (kernel, launch kind, programs, calls, average duration,
algorithmic bytes or flops, achieved rate and fraction of peak, HBM traffic per
launch) and a json block {kernel: traffic bytes per launch} that bench.py reads
for its roofline record.
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import pathlib

HBM_PEAK_GBS = 8000.0
MFMA_FP32_PEAK_TFLOPS = 157.3
GIB_KIB = 1024 * 1024


def counters(path: pathlib.Path) -> dict:
    """{kernel name: {counter: mean value per dispatch}} from a counter_collection.csv."""
    acc = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(path)):
        acc[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in acc.items()}


def launch_info(bench: dict, configs) -> dict:
    """{kernel name: kind, pattern, programs, bytes and flops per launch} over the step-only results."""
    info = {}
    for cfg in configs:
        for r in bench["configs"][cfg]["results"]:
            for l in r.get("launches", []):
                for i, k in enumerate(l["kernels"]):
                    # A launch's algorithmic work belongs to its first kernel; the others
                    # (split-K chunk sums, column sums' second pass) carry none of their own.
                    e = info.setdefault(k, {"kind": l["kind"] if i == 0 else f"{l['kind']} (second pass)",
                                            "pattern": l["pattern"], "programs": set(),
                                            "bytes": l["bytes"] if i == 0 else 0, "flops": l["flops"] if i == 0 else 0})
                    e["programs"].add(r["name"])
    return info


def summarize(a) -> str:
    bench = json.loads(pathlib.Path(a.bench).read_text())
    configs = a.configs.split(",")
    info = launch_info(bench, configs)
    stats = {r["Name"]: r for r in csv.DictReader(open(a.stats))}
    fetch = counters(pathlib.Path(a.fetch))
    write = counters(pathlib.Path(a.write))
    mfma = counters(pathlib.Path(a.mfma)) if a.mfma else {}
    copy = next(k for k in fetch if "k_copy16" in k)
    ff = GIB_KIB / fetch[copy]["FETCH_SIZE"]
    wf = GIB_KIB / write[next(k for k in write if "k_copy16" in k)]["WRITE_SIZE"]
    rows = []
    traffic = {}
    for k, e in info.items():
        s = stats.get(k)
        if s is None or k not in fetch or k not in write:
            continue
        avg_us = float(s["AverageNs"]) / 1e3
        t = (fetch[k]["FETCH_SIZE"] * ff + write[k]["WRITE_SIZE"] * wf) * 1024
        traffic[k] = round(t)
        rows.append((k, e, int(s["Calls"]), avg_us, t))
    # Kernels by total time in the run, largest first.
    rows.sort(key=lambda r: -r[2] * r[3])
    out = [f"Calibration: k_copy16 FETCH_SIZE = {fetch[copy]['FETCH_SIZE']:.0f} KiB and WRITE_SIZE = "
           f"{GIB_KIB / wf:.0f} KiB per dispatch for 1 GiB each way: FETCH_SIZE x {ff:.4f}, WRITE_SIZE x {wf:.4f}.", ""]
    head = "| kernel | kind | programs | calls | avg us | algorithmic | achieved | of peak | HBM traffic / launch | traffic / algorithmic bytes |"
    if mfma:
        head += " MfmaUtil | MfmaFlopsF32 / flops | LDS conflict |"
    out += [head, "|" + "---|" * (head.count("|") - 1)]
    for k, e, calls, avg, t in rows:
        progs = ", ".join(sorted(e["programs"]))
        if len(progs) > 70:
            progs = f"{len(e['programs'])} programs"
        kind = e["kind"] + (f" {e['pattern']}" if e["pattern"] else "")
        if e["flops"]:
            alg = f"{e['flops'] / 1e9:.2f} GFLOP"
            rate = e["flops"] / (avg * 1e6)
            ach, frac = f"{rate:.1f} TFLOP/s", f"{100 * rate / MFMA_FP32_PEAK_TFLOPS:.1f} %"
        elif e["bytes"]:
            alg = f"{e['bytes'] / 1e6:.1f} MB"
            rate = e["bytes"] / (avg * 1e3)
            ach, frac = f"{rate:.0f} GB/s", f"{100 * rate / HBM_PEAK_GBS:.1f} %"
        else:
            alg = ach = frac = "–"
        ratio = f"{t / e['bytes']:.3f}" if e["bytes"] else "–"
        line = f"| {k} | {kind} | {progs} | {calls} | {avg:.2f} | {alg} | {ach} | {frac} | {t / 1e6:.1f} MB | {ratio} |"
        if mfma:
            m = mfma.get(k, {})
            util = m.get("MfmaUtil")
            fl = m.get("MfmaFlopsF32")
            line += (f" {util:.1f} % |" if util is not None else " – |") + \
                    (f" {fl / e['flops']:.4f} |" if fl is not None and e["flops"] else " – |") + \
                    (f" {m['LDSBankConflict']:.1f} % |" if "LDSBankConflict" in m else " – |")
        out.append(line)
    if a.events:
        full = json.loads(pathlib.Path(a.events).read_text())
        full_stats = {r["Name"]: r for r in csv.DictReader(open(a.events_stats))} if a.events_stats else stats
        for cfg in configs:
            dom = full["configs"].get(cfg, {}).get("dominant")
            if dom and dom["code"] in full_stats:
                s = full_stats[dom["code"]]
                out += ["", f"Roofline kernel of {cfg}: {dom['code']}, {dom['bytesPerLaunch']:.0f} algorithmic bytes per launch; "
                            f"bench hipEvents average {dom['avgUs']:.2f} us, rocprofv3 average {float(s['AverageNs']) / 1e3:.2f} us "
                            f"over {s['Calls']} calls."]
    out += ["", "```json", json.dumps({"factors": {"FETCH_SIZE": ff, "WRITE_SIZE": wf}, "traffic_bytes_per_launch": traffic},
                                      sort_keys=True), "```"]
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--bench", required=True)
    ap.add_argument("--stats", required=True)
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--mfma")
    ap.add_argument("--events", help="the full bench's json (its hipEvents average of each roofline kernel)")
    ap.add_argument("--events-stats", help="kernel_stats.csv of a trace of that full bench command")
    ap.add_argument("--configs", default="c2")
    print(summarize(ap.parse_args()))


if __name__ == "__main__":
    main()
