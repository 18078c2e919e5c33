"""Write the fixtures under tests/golden/ from the data files the reference's own
tests hold (abho7/tensor-compiler-webgpu golden/*.json and golden/torch-m3b.f64).

Run once, in a container where the reference is mounted:

    python tests/golden/extract.py /root/reference

Only data is copied (graphs as node lists, inputs, expected float64 outputs,
recorded counts); no reference source text. The outputs are committed, so no
test reads the reference at run time.

  cases.json          golden/cases.json (112 graphs + inputs + cotangents) with
                      golden/torch.json's float64 outputs and gradients merged in
  m4_counts.json      golden/measurements.json m4.fusion / m4.semantics.model /
                      m4.semantics.corpus counts / m4.passSabotage counts, and
                      golden/gpu-m4.json direct-case names with their kind and
                      pattern and the fuzzer's structural counts
  transformer_init.json + transformer_init.f64
                      golden/spec-m3b.json golden-seed1 (V, batch, seed, initSha,
                      the four token sequences of its first batch) and
                      golden/torch-m3b.f64's init logits, loss and gradients
  transformer_golden.json + transformer_golden.f64
                      the four golden training runs of golden/spec-m3b.json
                      (seed, V, batch, steps, initSha, the 20-step batch
                      schedule, the optimizer, the projection count and its
                      sha256, and the 512 synthetic training sequences the
                      schedules index) with golden/torch-m3b.json's per-step
                      training losses and parameter projections, its initial
                      loss per run, and from golden/torch-m3b.f64 each run's
                      initial logits and golden-seed1's final parameters
"""
import json
import pathlib
import struct
import sys

HERE = pathlib.Path(__file__).resolve().parent


def main(ref_root: str) -> None:
    ref = pathlib.Path(ref_root) / "golden"
    cases = json.loads((ref / "cases.json").read_text())["cases"]
    torch = json.loads((ref / "torch.json").read_text())
    answers = {c["name"]: c for c in torch["cases"]}
    out = []
    for c in cases:
        a = answers[c["name"]]
        entry = {k: c[k] for k in ("name", "kind", "graph", "outputs", "inputs", "cotangents")}
        if "native" in c:
            entry["native"] = c["native"]
            entry["torchNative"] = a.get("native")
        if "set" in c:
            entry["set"] = c["set"]
        entry["torchOutputs"] = a["outputs"]
        entry["torchGrads"] = a["grads"]
        out.append(entry)
    (HERE / "cases.json").write_text(json.dumps({"source": "golden/cases.json + golden/torch.json",
                                                 "torch": torch["torch"], "dtype": torch["dtype"], "cases": out}))

    m = json.loads((ref / "measurements.json").read_text())["m4"]
    gpu = json.loads((ref / "gpu-m4.json").read_text())
    direct = [{"name": d["name"], "kind": d["kind"], "pattern": d["pattern"], "matmul": d.get("matmul")}
              for d in gpu["direct"]]
    corpus = m["semantics"]["corpus"]
    fuzz = gpu["fuzz"]
    sab = m["passSabotage"]
    counts = {"source": "golden/measurements.json m4, golden/gpu-m4.json direct and fuzz",
              "fusion": m["fusion"], "semanticsModel": m["semantics"]["model"],
              "corpusByPattern": corpus["byPattern"],
              "corpus": {k: corpus[k] for k in ("programs", "graphs", "withFused", "fusedNodes", "byPattern")},
              "fuzz": {k: fuzz[k] for k in ("programs", "skipped", "runs", "fusedRuns", "byKind", "byPattern")},
              "passSabotage": {k: sab[k] for k in ("programs", "graphs", "changed", "threw")},
              "gpuDirect": m["gpu"]["direct"], "direct": direct}
    (HERE / "m4_counts.json").write_text(json.dumps(counts, indent=1))

    spec = json.loads((ref / "spec-m3b.json").read_text())
    g = spec["golden"][0]
    tm = json.loads((ref / "torch-m3b.json").read_text())
    init = next(i for i in tm["init"] if i["name"] == g["name"])
    index = tm["blob"]["index"]
    blob = (ref / tm["blob"]["file"]).read_bytes()
    prefix = f"init/{g['name']}/"
    keys = [k for k in index if k.startswith(prefix)]
    tensors = {}
    data = bytearray()
    for k in keys:
        off, n = index[k]
        vals = struct.unpack_from(f"<{n}d", blob, off * 8)
        tensors[k[len(prefix):]] = [len(data) // 8, n]
        data += struct.pack(f"<{n}d", *vals)
    first = [spec["synthetic"]["train"][i] for i in g["schedule"][0]]
    meta = {"source": "golden/spec-m3b.json golden[0] + golden/torch-m3b.json/.f64 init",
            "name": g["name"], "seed": g["seed"], "V": g["V"], "batch": g["batch"], "initSha": g["initSha"],
            "config": spec["config"], "paramOrder": spec["paramOrder"], "firstBatch": first,
            "loss": init["loss"], "tensors": tensors}
    (HERE / "transformer_init.json").write_text(json.dumps(meta))
    (HERE / "transformer_init.f64").write_bytes(bytes(data))

    golden_runs(spec, tm, blob, index)


def golden_runs(spec, tm, blob, index) -> None:
    """The four golden training runs: what the teacher-forced, forward and trajectory
    checks need, as data (golden/spec-m3b.json, golden/torch-m3b.json and .f64)."""
    tensors, data = {}, bytearray()

    def take(key, name):
        off, n = index[key]
        tensors[name] = [len(data) // 8, n]
        data.extend(blob[off * 8: (off + n) * 8])

    runs = []
    inits = {i["name"]: i["loss"] for i in tm["init"]}
    training = {t["name"]: t for t in tm["training"]}
    for g in spec["golden"]:
        t = training[g["name"]]
        take(f"init/{g['name']}/logits", f"init/{g['name']}/logits")
        runs.append({k: g[k] for k in ("name", "seed", "V", "batch", "steps", "initSha", "schedule")}
                    | {"initLoss": inits[g["name"]], "losses": t["losses"], "projections": t["projections"]})
    first = spec["golden"][0]["name"]
    for p in spec["paramOrder"]:
        take(f"train/{first}/final/{p['name']}", f"final/{first}/{p['name']}")
    syn = spec["synthetic"]
    meta = {"source": "golden/spec-m3b.json golden[0..3] + synthetic.train, golden/torch-m3b.json init/training, "
                      "golden/torch-m3b.f64 init logits and golden-seed1's final parameters",
            "config": spec["config"], "optimizer": spec["optimizer"], "paramOrder": spec["paramOrder"],
            "projections": spec["projections"],
            "synthetic": {k: syn[k] for k in ("seed", "vocab", "period")} | {"train": syn["train"]},
            "golden": runs, "tensors": tensors}
    (HERE / "transformer_golden.json").write_text(json.dumps(meta))
    (HERE / "transformer_golden.f64").write_bytes(bytes(data))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
