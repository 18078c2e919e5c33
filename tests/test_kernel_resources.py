"""The generated kernels' register use, checked on the CPU: every kernel the standard runs
launch (config 5's step in both lowerings, configs 2-4, the forward pass with attention
fused) is compiled for gfx950 with the runner's options, and none may use scratch memory
(a private array the compiler could not keep in registers, or a register spill): scratch
traffic goes through memory and is slow. It found one: an array of HIP float4 structs
holding staged V values across the attention kernel's score products."""
import pathlib
import re
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
KERNELS = ROOT / "tensor-compiler-webgpu_amd" / "csrc" / "kernels"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not pathlib.Path(HIPCC).exists(), reason="hipcc is not installed")
def test_generated_kernels_use_no_scratch(tool, tmp_path):
    r = tool("kernel-unit", {}, timeout=300)
    assert len(r["kernels"]) > 150
    src = tmp_path / "unit.hip"
    src.write_text(r["unit"])
    opts = ["-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-Xclang", "-target-feature", "-Xclang",
            "-packed-fp32-ops"]
    p = subprocess.run([HIPCC, "--offload-arch=gfx950", *opts, f"-I{KERNELS}", "--cuda-device-only", "-c", str(src),
                        "-o", str(tmp_path / "unit.o"), "-Rpass-analysis=kernel-resource-usage"],
                       capture_output=True, text=True, timeout=600)
    assert p.returncode == 0, p.stderr[-2000:]
    usage, cur = {}, None
    for line in p.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
            usage[cur] = {}
            continue
        m = re.search(r"(VGPRs|ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill): (\d+)", line)
        if m and cur:
            usage[cur][m.group(1)] = int(m.group(2))
    assert set(usage) == set(r["kernels"])
    bad = {k: v for k, v in usage.items()
           if v.get("ScratchSize [bytes/lane]", 0) or v.get("VGPRs Spill", 0) or v.get("SGPRs Spill", 0)}
    assert not bad, bad
