"""Python side of the host CLI (js/cli/tool.js): run a command in a node child
process and read what it returns — one JSON document on stdout, or a result
bundle (manifest.json + data.f32) written under an output directory.

Used by the Python harnesses (tests, bench.py, __graft_entry__). The GPU work
of a GPU command happens in the node child, through the N-API addon over
lib/libtcmi.so.
"""
from __future__ import annotations

import json
import os
import pathlib
import subprocess
import sys
import tempfile
import threading
from typing import Any, Dict, Optional

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent
TOOL = PKG / "js" / "cli" / "tool.js"
NODE = os.environ.get("TCMI_NODE", "node")


class ToolError(RuntimeError):
    pass


def node_tool(cmd: str, request: Optional[Dict[str, Any]] = None, out: Optional[str] = None,
              timeout: float = 600, echo_stderr: Optional[bool] = None) -> Any:
    """Run `node tool.js cmd [request.json] [--out out]` and return its parsed stdout.

    The child's stderr (its progress lines) is forwarded line by line as it comes
    when `echo_stderr` is true (the default for the GPU commands, `gpu-*`), and
    its tail is kept for the error raised if the child fails."""
    if echo_stderr is None:
        echo_stderr = cmd.startswith("gpu-")
    args = [NODE, str(TOOL), cmd]
    tmp = None
    try:
        if request is not None:
            tmp = tempfile.NamedTemporaryFile("w", suffix=".json", delete=False)
            json.dump(request, tmp)
            tmp.close()
            args.append(tmp.name)
        if out is not None:
            args += ["--out", str(out)]
        tail: list = []

        def pump(stream):
            for raw in iter(stream.readline, b""):
                line = raw.decode(errors="replace")
                tail.append(line)
                del tail[:-200]
                if echo_stderr:
                    sys.stderr.write(line)
                    sys.stderr.flush()

        chunks: list = []
        p = subprocess.Popen(args, stdout=subprocess.PIPE, stderr=subprocess.PIPE)
        readers = [threading.Thread(target=pump, args=(p.stderr,), daemon=True),
                   threading.Thread(target=lambda: chunks.append(p.stdout.read()), daemon=True)]
        for t in readers:
            t.start()
        try:
            p.wait(timeout=timeout)
        except subprocess.TimeoutExpired:
            p.kill()
            p.wait()
            raise
        for t in readers:
            t.join(timeout=10)
        stdout = b"".join(chunks)
        if p.returncode != 0:
            raise ToolError(f"node tool.js {cmd} exited {p.returncode}:\n{''.join(tail)[-4000:]}")
        return json.loads(stdout.decode()) if stdout else None
    finally:
        if tmp is not None:
            os.unlink(tmp.name)


class Bundle:
    """A result bundle written by a GPU command."""

    def __init__(self, directory):
        self.dir = pathlib.Path(directory)
        self.manifest = json.loads((self.dir / "manifest.json").read_text())
        # Mapped, not read: a full-size training step's bundle holds gigabytes.
        path = self.dir / "data.f32"
        self.data = (np.memmap(path, dtype=np.float32, mode="r") if path.stat().st_size
                     else np.zeros(0, dtype=np.float32))

    def arr(self, at) -> np.ndarray:
        return self.data[at["offset"]: at["offset"] + at["n"]]

    @property
    def cases(self):
        return self.manifest["cases"]
