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
from typing import Any, Dict, Optional

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent
TOOL = PKG / "js" / "cli" / "tool.js"
NODE = os.environ.get("TCMI_NODE", "node")


class ToolError(RuntimeError):
    pass


def node_tool(cmd: str, request: Optional[Dict[str, Any]] = None, out: Optional[str] = None,
              timeout: float = 600, echo_stderr: bool = False) -> Any:
    """Run `node tool.js cmd [request.json] [--out out]` and return its parsed stdout."""
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
        p = subprocess.run(args, stdout=subprocess.PIPE, stderr=None if echo_stderr else subprocess.PIPE,
                           timeout=timeout)
        if p.returncode != 0:
            err = "" if echo_stderr else p.stderr.decode(errors="replace")[-4000:]
            raise ToolError(f"node tool.js {cmd} exited {p.returncode}:\n{err}")
        return json.loads(p.stdout.decode()) if p.stdout else None
    finally:
        if tmp is not None:
            os.unlink(tmp.name)


class Bundle:
    """A result bundle written by a GPU command."""

    def __init__(self, directory):
        self.dir = pathlib.Path(directory)
        self.manifest = json.loads((self.dir / "manifest.json").read_text())
        self.data = np.fromfile(self.dir / "data.f32", dtype=np.float32)

    def arr(self, at) -> np.ndarray:
        return self.data[at["offset"]: at["offset"] + at["n"]]

    @property
    def cases(self):
        return self.manifest["cases"]
