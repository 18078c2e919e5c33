"""The launch that allocates nothing (tcmi_launch_scratch), on the GPU, in-process through
the C ABI's ctypes binding: split-K matmuls (a workspace of partial sums per K chunk,
summed by a second kernel) launched with the library's own device scratch as the
workspace give the bits the ordinary launch gives with a tcmi_malloc'd workspace, on two
calls in a row, the second smaller (the scratch keeps the first call's partials); no
allocation is counted meanwhile; a launch asking for more scratch than the library holds,
or naming a workspace slot outside its argument block, is refused before anything is
enqueued."""
import ctypes

import numpy as np
import pytest

from conftest import PKG

pytestmark = pytest.mark.gpu

MAX_IN, MAX_P = 8, 48
ARG_BYTES = MAX_IN * 8 + 8 + 8 + MAX_P * 4
WS_SLOT = MAX_IN * 8 + 8          # byte offset of the workspace pointer in TcmiArgs
MALLOC = 0                        # TCMI_COUNT_MALLOC


def pack(ins, out, ws, params):
    """A TcmiArgs block: operand pointers, output, workspace, u32 parameters."""
    b = np.zeros(ARG_BYTES, dtype=np.uint8)
    p64 = b[: (MAX_IN + 2) * 8].view(np.uint64)
    for k, v in enumerate(ins):
        p64[k] = v
    p64[MAX_IN] = out
    p64[MAX_IN + 1] = ws
    b[(MAX_IN + 2) * 8:].view(np.uint32)[: len(params)] = params
    return b


def test_scratch_launch_gives_the_workspace_launch_bits(tool):
    import tcmi_ctypes
    u32, u64 = tcmi_ctypes.u32, tcmi_ctypes.u64
    d = tool("scratch-kernels")
    t = tcmi_ctypes.load()
    t.init()
    t.set_include_dir(str(PKG / "csrc" / "kernels").encode())
    t.set_cache_dir(str(PKG / "_build" / "kcache").encode())
    mod = u64()
    t.module_compile(d["unit"].encode(), None, ctypes.byref(mod))
    counters = (u64 * 7)()
    rng = np.random.default_rng(7)
    owned = []

    def alloc(nbytes):
        h = u64()
        t.malloc(nbytes, ctypes.byref(h))
        owned.append(h.value)
        return h.value

    try:
        for (M, K, N), launch in zip(d["shapes"], d["launches"]):
            print(f"gpu step: scratch launch {M}x{K}x{N}, workspace {launch['workspace']} bytes", flush=True)
            assert 0 < launch["workspace"] <= 64 << 20 and len(launch["kernels"]) == 2   # split-K: partials, then their sum
            x = (rng.standard_normal(M * K) / np.sqrt(K)).astype(np.float32)
            w = rng.standard_normal(K * N).astype(np.float32)
            hx, hw = alloc(x.nbytes), alloc(w.nbytes)
            t.h2d(hx, 0, x.ctypes.data, x.nbytes)
            t.h2d(hw, 0, w.ctypes.data, w.nbytes)
            y_ws, y_scr, ws = alloc(M * N * 4), alloc(M * N * 4), alloc(launch["workspace"])
            fns = []
            for k in launch["kernels"]:
                f = u64()
                t.module_function(mod.value, k["name"].encode(), ctypes.byref(f))
                fns.append(f.value)
            # The ordinary launch, its workspace from tcmi_malloc.
            for f, k in zip(fns, launch["kernels"]):
                a = pack([hx, hw], y_ws, ws, launch["params"])
                t.launch(f, (u32 * 3)(*k["grid"]), (u32 * 3)(*k["block"]), k["lds"], a.ctypes.data, ARG_BYTES)
            # The same kernels with the library's scratch as the workspace: no allocation.
            t.counters(counters, 7)
            before = counters[MALLOC]
            a = pack([hx, hw], y_scr, 0, launch["params"])
            tcmi_ctypes.launch_list_with_scratch(t, [(fns, launch, a.ctypes.data, ARG_BYTES)])
            t.sync()
            t.counters(counters, 7)
            assert counters[MALLOC] == before
            got_ws = np.empty(M * N, dtype=np.float32)
            got_scr = np.empty(M * N, dtype=np.float32)
            t.d2h(got_ws.ctypes.data, y_ws, 0, M * N * 4)
            t.d2h(got_scr.ctypes.data, y_scr, 0, M * N * 4)
            assert np.array_equal(got_ws.view(np.uint32), got_scr.view(np.uint32)), (M, K, N)
            # And the product is the product: within gamma(K) * sum |x||w| of float64's.
            X, W = x.astype(np.float64).reshape(M, K), w.astype(np.float64).reshape(K, N)
            u = 2.0 ** -24
            budget = 2 * (K * u / (1 - K * u)) * (np.abs(X) @ np.abs(W))
            assert np.all(np.abs(got_scr.reshape(M, N) - X @ W) <= budget), (M, K, N)
        # Refused before anything is enqueued: more scratch than the library holds, a slot
        # that is misaligned or outside the block.
        k = d["launches"][0]["kernels"][0]
        f = u64()
        t.module_function(mod.value, k["name"].encode(), ctypes.byref(f))
        a = pack([0, 0], 0, 0, d["launches"][0]["params"])
        grid, block = (u32 * 3)(*k["grid"]), (u32 * 3)(*k["block"])
        lib = t.lib
        assert lib.tcmi_launch_scratch(f.value, grid, block, k["lds"], a.ctypes.data, ARG_BYTES, WS_SLOT, (64 << 20) + 1) == 10001
        assert b"scratch" in lib.tcmi_last_error()
        assert lib.tcmi_launch_scratch(f.value, grid, block, k["lds"], a.ctypes.data, ARG_BYTES, WS_SLOT + 4, 16) == 10001
        assert lib.tcmi_launch_scratch(f.value, grid, block, k["lds"], a.ctypes.data, ARG_BYTES, ARG_BYTES, 16) == 10001
        t.sync()
    finally:
        for h in owned:
            t.free(h)
