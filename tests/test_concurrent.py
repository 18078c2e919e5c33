"""The concurrent group of independent programs (js/src/mi355x/runner.js Concurrent: the
config-2 headline step issues its 16 programs over two streams), checked on the CPU with
stand-in programs: programs go to streams longest first, each to the least-loaded stream,
every program's launches stay together and in order on one stream, the argument blocks
are concatenated with their offsets shifted, and programs that share a written buffer are
refused. On the GPU, the group gives the kept outputs of config 2's 16 programs the same
bits as running them one after another (whose values `test_gpu_c2.py` judges)."""
import pytest


def test_concurrent_group_balances_and_keeps_programs_whole(tool):
    r = tool("concurrent-check", {"bytes": [[5], [3, 3], [4], [1], [2, 2]], "streams": 2})
    # Longest first to the least-loaded stream: 6 -> s0, 5 -> s1, 4 -> s1, 4 -> s0, 1 -> s1.
    assert r["load"] == [10, 10]
    kernels = [2, 3, 2, 2, 3]   # each stand-in program has one kernel more than launches
    expect = []
    for p, s in zip(range(5), [1, 0, 1, 1, 0]):
        expect += [s] * kernels[p]
    assert r["streamOf"] == expect
    assert r["fns"] == sum(([p + 1] * k for p, k in enumerate(kernels)), [])
    assert r["offsets"] == [16 * i for i in range(sum(kernels) + 1)]
    # Each program's argument bytes follow the previous program's, unchanged.
    args, at = r["args"], 0
    for p, k in enumerate(kernels):
        assert args[at:at + 16 * k] == [(p * 16 + q) % 256 for q in range(16 * k)]
        at += 16 * k
    assert r["refused"] and "both write buffer" in r["refused"]


def test_concurrent_group_with_one_stream_keeps_the_order(tool):
    r = tool("concurrent-check", {"bytes": [[1], [2], [3]], "streams": 1})
    assert set(r["streamOf"]) == {0} and r["load"] == [6]


@pytest.mark.gpu
def test_concurrent_group_gives_the_sequential_bits(tool):
    """Config 2's 16 programs at [2048, 1024], run one after another, then (outputs
    overwritten first) as a concurrent group over 2, 3 and 4 streams: every kept output
    is the same bits."""
    r = tool("gpu-concurrent", {"programs": 8, "R": 2048, "C": 1024, "streams": [2, 3, 4]}, timeout=300)
    assert r["programs"] == 16
    for s, e in r["streams"].items():
        assert e["total"] > 0 and e["same"] == e["total"], (s, e)
