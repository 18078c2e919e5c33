"""Build the MI355X backend in place (no GPU needed; hipcc cross-compiles gfx950).

    python tensor-compiler-webgpu_amd/build.py [--no-precompile]

Produces, under tensor-compiler-webgpu_amd/lib/:
  libtcmi.so   the C ABI of include/tcmi.h (HIP runtime, hiprtc, fixed kernels),
               built with hipcc --offload-arch=gfx950
  tcmi.node    the Node-API addon over it (g++ against Node's headers)
and fills tensor-compiler-webgpu_amd/_build/kcache/ with the code objects of
the kernels the standard runs ask for (compiled offline by hiprtc for gfx950,
keyed by their exact text), so a GPU box starts without compiling.
"""
from __future__ import annotations

import hashlib
import json
import os
import pathlib
import shutil
import subprocess
import sys
import time

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "lib"
CSRC = PKG / "csrc"
JS = PKG / "js"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
NODE_INCLUDE = os.environ.get("NODE_INCLUDE", "/usr/include/node")
# hipcc options for every device build: packed fp32 instructions off.
HIP_DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd, **kw):
    print("+", " ".join(str(c) for c in cmd), flush=True)
    subprocess.run([str(c) for c in cmd], check=True, **kw)


def build_stamp() -> str:
    """A hash of every source the build reads (part of the kernel-cache key)."""
    h = hashlib.sha256()
    for p in sorted(list(CSRC.rglob("*.cpp")) + list(CSRC.rglob("*.h")) + [ROOT / "include" / "tcmi.h"]):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:16]


def build_runtime(stamp: str) -> pathlib.Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libtcmi.so"
    tmp = LIB / "libtcmi.so.tmp"
    _run([f"{ROCM}/bin/hipcc", "--offload-arch=gfx950", "-O3", "-fPIC", "-shared", "-std=c++17", *HIP_DEVICE_FLAGS,
          f'-DTCMI_BUILD_STAMP="{stamp}"', CSRC / "runtime.cpp", "-o", tmp,
          f"-L{ROCM}/lib", "-lhiprtc", f"-Wl,-rpath,{ROCM}/lib"])
    tmp.replace(out)
    return out


def build_addon() -> pathlib.Path:
    out = LIB / "tcmi.node"
    tmp = LIB / "tcmi.node.tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-DNODE_GYP_MODULE_NAME=tcmi", f"-I{NODE_INCLUDE}",
          CSRC / "napi_addon.cpp", "-o", tmp, f"-L{LIB}", "-ltcmi", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM}/lib"])
    tmp.replace(out)
    return out


def check_node_loads() -> None:
    _run(["node", "-e", "const a=require(process.argv[1]); if (typeof a.launch !== 'function') process.exit(3);",
          LIB / "tcmi.node"])


# (group, shard, shards): the fuzz corpus's ~7500 kernels are compiled in 6 parts.
PRECOMPILE_JOBS = ([("direct", 0, 1), ("models", 0, 1), ("golden", 0, 1), ("configs", 0, 1), ("sweep", 0, 1),
                    ("attention", 0, 1), ("recompute", 0, 1), ("scratch", 0, 1)]
                   + [("fuzz", k, 6) for k in range(6)])
KCACHE = PKG / "_build" / "kcache"


def precompile(jobs=None, workers=None) -> None:
    """Compile the code objects of the standard runs into a fresh cache, several
    groups at a time (each job is one hiprtc translation unit in its own node
    process)."""
    jobs = jobs or PRECOMPILE_JOBS
    if KCACHE.exists():
        shutil.rmtree(KCACHE)   # only what this build's kernels need travels to a GPU box
    KCACHE.mkdir(parents=True)
    workers = workers or max(1, min(len(jobs), os.cpu_count() or 1, 8))
    pending = list(jobs)
    running = []
    failed = []
    while pending or running:
        while pending and len(running) < workers:
            group, shard, shards = pending.pop(0)
            req = PKG / "_build" / f"precompile-{group}-{shard}.json"
            req.write_text(json.dumps({"group": group, "arch": "gfx950", "shard": shard, "shards": shards}))
            cmd = ["node", str(JS / "cli" / "tool.js"), "precompile", str(req)]
            print("+", " ".join(cmd), flush=True)
            running.append((group, shard, subprocess.Popen(cmd, stdout=subprocess.PIPE)))
        time.sleep(0.2)
        for job in list(running):
            group, shard, proc = job
            if proc.poll() is None:
                continue
            running.remove(job)
            out = proc.stdout.read().decode()
            print(f"  {group}[{shard}]: {out.strip()}", flush=True)
            if proc.returncode != 0:
                failed.append(f"{group}[{shard}]")
    if failed:
        raise SystemExit(f"precompile failed: {', '.join(failed)}")


def main(argv) -> None:
    if not shutil.which(f"{ROCM}/bin/hipcc") and not os.path.exists(f"{ROCM}/bin/hipcc"):
        raise SystemExit(f"hipcc not found under {ROCM}")
    stamp = build_stamp()
    build_runtime(stamp)
    build_addon()
    check_node_loads()
    if "--no-precompile" not in argv:
        precompile()


if __name__ == "__main__":
    main(sys.argv[1:])
