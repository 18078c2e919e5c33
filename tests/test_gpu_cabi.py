"""The one-call training step of the C ABI (tcmi_graph_step), in-process through the
ctypes binding on the GPU: a captured graph of one copy kernel stands in for a step;
the step's uploads (a small one staged through pinned memory, a large one copied
directly), the replay and the readback must all happen, in order, in one call, and a
call with an unknown graph or an out-of-range copy must fail before anything is
enqueued."""
import ctypes

import numpy as np
import pytest


@pytest.mark.gpu
def test_graph_step_uploads_replays_and_reads_back():
    import tcmi_ctypes
    t = tcmi_ctypes.load()
    t.init()
    u64 = tcmi_ctypes.u64
    small, large = 1 << 10, 1 << 20            # bytes: staged, and copied directly
    bufs = {}
    for name, n in (("a", small), ("b", small), ("c", large)):
        h = u64()
        t.malloc(n, ctypes.byref(h))
        bufs[name] = h.value
    try:
        t.fill32(bufs["b"], 0, 0, small // 4)
        # The stand-in step: copy a -> b (one kernel), captured once.
        t.capture_begin()
        t.ceiling_copy(bufs["b"], bufs["a"], small, 4)
        g = u64()
        t.capture_end(ctypes.byref(g))
        x = np.arange(small // 4, dtype=np.float32) * 0.5 + 1.0
        y = np.arange(large // 4, dtype=np.float32) * -0.25
        dst = (u64 * 2)(bufs["a"], bufs["c"])
        src = (ctypes.c_void_p * 2)(x.ctypes.data, y.ctypes.data)
        nbytes = (u64 * 2)(small, large)
        out = np.zeros(4, dtype=np.float32)
        rc = t.lib.tcmi_graph_step(2, dst, src, nbytes, g.value, bufs["b"] + 16, out.ctypes.data, 16)
        assert rc == 0, t.lib.tcmi_last_error()
        # The readback ran after the replay, which ran after the upload of a.
        assert np.array_equal(out, x[4:8])
        back = np.zeros(large // 4, dtype=np.float32)
        t.d2h(back.ctypes.data, bufs["c"], 0, large)
        assert np.array_equal(back, y)
        # Refused before anything is enqueued: an unknown graph, a copy past its allocation.
        x2 = x + 100.0
        src2 = (ctypes.c_void_p * 2)(x2.ctypes.data, y.ctypes.data)
        assert t.lib.tcmi_graph_step(2, dst, src2, nbytes, g.value + 1000, bufs["b"], out.ctypes.data, 4) == 10001
        over = (u64 * 2)(small, large + 16)
        assert t.lib.tcmi_graph_step(2, dst, src2, over, g.value, bufs["b"], out.ctypes.data, 4) == 10001
        a_now = np.zeros(small // 4, dtype=np.float32)
        t.d2h(a_now.ctypes.data, bufs["a"], 0, small)
        assert np.array_equal(a_now, x)
        t.graph_destroy(g.value)
    finally:
        for h in bufs.values():
            t.free(h)


@pytest.mark.gpu
def test_launch_dag_over_several_streams_is_refused_inside_a_capture():
    """Capture over several streams is switched off in the C ABI itself: an empty
    two-stream launch group is accepted eagerly and refused, with nothing enqueued,
    while the library stream is capturing; the capture then ends normally."""
    import tcmi_ctypes
    t = tcmi_ctypes.load()
    t.init()
    lib = t.lib
    assert lib.tcmi_launch_dag(0, None, None, None, None, 2, None, None, None, None) == 0, lib.tcmi_last_error()
    t.sync()
    h = tcmi_ctypes.u64()
    t.malloc(1 << 12, ctypes.byref(h))
    try:
        t.capture_begin()
        refused = lib.tcmi_launch_dag(0, None, None, None, None, 2, None, None, None, None)
        message = lib.tcmi_last_error()
        one_stream = lib.tcmi_launch_dag(0, None, None, None, None, 1, None, None, None, None)
        t.fill32(h.value, 0, 7, 1 << 10)
        g = tcmi_ctypes.u64()
        t.capture_end(ctypes.byref(g))
        assert refused == 10001 and b"stream capture" in message
        assert one_stream == 0
        t.graph_launch(g.value)
        t.sync()
        back = np.zeros(1 << 10, dtype=np.uint32)
        t.d2h(back.ctypes.data, h.value, 0, 1 << 12)
        assert np.all(back == 7)
        t.graph_destroy(g.value)
    finally:
        t.free(h.value)


@pytest.mark.gpu
def test_staggered_allocations_keep_their_size_alignment_and_contents():
    """Allocations of 1 MiB or more start at staggered offsets past their hipMalloc
    base: every handle is still 256-byte aligned, copies are checked against the size
    asked for (a copy of exactly that size works, one element more is refused), the
    last bytes hold what was written, and every allocation frees."""
    import tcmi_ctypes
    t = tcmi_ctypes.load()
    t.init()
    u64 = tcmi_ctypes.u64
    sizes = [(1 << 20) + 4 * k for k in range(18)] + [4096, 1 << 22]
    handles = []
    try:
        for n in sizes:
            h = u64()
            t.malloc(n, ctypes.byref(h))
            handles.append((h.value, n))
            assert h.value % 256 == 0, (n, h.value)
            got = u64()
            t.size(h.value, ctypes.byref(got))
            assert got.value == n
        assert len({h for h, _ in handles}) == len(handles)
        for i, (h, n) in enumerate(handles):
            data = (np.arange(n // 4, dtype=np.uint32) * 2654435761 + i).astype(np.uint32)
            t.h2d(h, 0, data.ctypes.data, n)
            assert t.lib.tcmi_h2d(h, 4, data.ctypes.data, n) == 10001      # one element past the end
            back = np.zeros(n // 4, dtype=np.uint32)
            t.d2h(back.ctypes.data, h, 0, n)
            assert np.array_equal(back, data), n
    finally:
        for h, _ in handles:
            t.free(h)
