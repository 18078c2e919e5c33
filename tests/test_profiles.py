"""The committed rocprofv3 summaries and the tool that writes them (CPU only).

Each profile names the rocprofv3 commands it came from and carries the json block
of HBM traffic per kernel that bench.py's roofline record reads; profile_summary.py
turns a trace and two counter runs into that table, calibrated on the copy kernel."""
import csv
import json
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def _json_block(text):
    return json.loads(text.split("```json", 1)[1].split("```", 1)[0])


def test_profiles_name_their_commands_and_carry_traffic():
    mds = sorted((ROOT / "profiles").glob("*.md"))
    assert len(mds) >= 3
    for md in mds:
        text = md.read_text()
        assert "rocprofv3 --kernel-trace --stats" in text, md.name
        assert "--pmc FETCH_SIZE" in text and "--pmc WRITE_SIZE" in text, md.name
        block = _json_block(text)
        traffic = block["traffic_bytes_per_launch"]
        assert traffic and all(isinstance(v, int) and v > 0 for v in traffic.values()), md.name
        assert abs(block["factors"]["FETCH_SIZE"] - 2.0) < 1e-3 and abs(block["factors"]["WRITE_SIZE"] - 1.0) < 1e-3


def test_bench_reads_the_traffic_of_a_profiled_kernel():
    import bench
    md = ROOT / "profiles" / "c2_fused_elementwise_trace_traffic.md"
    traffic = _json_block(md.read_text())["traffic_bytes_per_launch"]
    kernel, value = next(iter(traffic.items()))
    assert bench.profiled_traffic(kernel) == (value, md.name)
    assert bench.profiled_traffic("tcmi_ew_00000000") == (None, None)


def test_profile_summary_scales_counters_by_the_copy_kernel(tmp_path):
    """A synthetic run: the copy kernel reads FETCH_SIZE 512 KiB-units for 1 GiB (factor 2),
    a kernel of 1 MB algorithmic bytes with FETCH 256 KiB and WRITE 512 KiB -> 1 MiB + 0.5 MiB."""
    bench_json = {"configs": {"c2": {"results": [{"name": "p0", "launches": [
        {"node": 3, "kind": "fused-elementwise", "pattern": "elementwise", "kernels": ["k_a"], "bytes": 1_572_864, "flops": 0},
        {"node": 4, "kind": "colreduce", "pattern": None, "kernels": ["k_b", "k_b2"], "bytes": 1000, "flops": 0}]}]}}}
    (tmp_path / "b.json").write_text(json.dumps(bench_json))
    with open(tmp_path / "stats.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"])
        w.writerow(["k_a", 10, 10000, 1000.0, 50, 900, 1100, 1])
        w.writerow(["k_b", 10, 5000, 500.0, 25, 400, 600, 1])
        w.writerow(["k_b2", 10, 5000, 500.0, 25, 400, 600, 1])

    def counter_file(name, counter, values):
        with open(tmp_path / name, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["Kernel_Name", "Counter_Name", "Counter_Value"])
            for k, v in values.items():
                w.writerow([k, counter, v])
                w.writerow([k, counter, v])
    counter_file("fetch.csv", "FETCH_SIZE", {"(anonymous namespace)::k_copy16(x)": 524288, "k_a": 512, "k_b": 10, "k_b2": 1})
    counter_file("write.csv", "WRITE_SIZE", {"(anonymous namespace)::k_copy16(x)": 1048576, "k_a": 512, "k_b": 1, "k_b2": 1})
    out = subprocess.run([sys.executable, str(ROOT / "tensor-compiler-webgpu_amd" / "profile_summary.py"),
                          "--bench", str(tmp_path / "b.json"), "--stats", str(tmp_path / "stats.csv"),
                          "--fetch", str(tmp_path / "fetch.csv"), "--write", str(tmp_path / "write.csv")],
                         check=True, capture_output=True, text=True).stdout
    block = _json_block(out)
    assert block["factors"] == {"FETCH_SIZE": 2.0, "WRITE_SIZE": 1.0}
    assert block["traffic_bytes_per_launch"]["k_a"] == (512 * 2 + 512) * 1024
    row = next(l for l in out.splitlines() if l.startswith("| k_a "))
    assert "1573 GB/s" in row and "| 1.000 |" in row      # 1.572864 MB in 1 us; traffic == algorithmic
    second = next(l for l in out.splitlines() if l.startswith("| k_b2 "))
    assert "(second pass)" in second and "| – |" in second   # no algorithmic bytes of its own
