import json
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG = ROOT / "tensor-compiler-webgpu_amd"
GOLDEN = ROOT / "tests" / "golden"
for p in (ROOT, PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


@pytest.fixture(scope="session")
def golden_cases():
    return json.loads((GOLDEN / "cases.json").read_text())["cases"]


@pytest.fixture(scope="session")
def m4_counts():
    return json.loads((GOLDEN / "m4_counts.json").read_text())


@pytest.fixture(scope="session")
def tool():
    import tcmi_bridge
    return tcmi_bridge.node_tool
