"""ctypes binding of the tcmi C ABI (include/tcmi.h) for Python callers.

This is the reference-side binding a Python harness would add: every entry
point of the header with its prototype, and a status check that raises with
tcmi_last_error(). There is no fallback — if lib/libtcmi.so is missing, load()
raises.
"""
from __future__ import annotations

import ctypes
import pathlib

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libtcmi.so"

u64 = ctypes.c_uint64
u32 = ctypes.c_uint32
i32 = ctypes.c_int32
P = ctypes.POINTER


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("compute_units", i32),
                ("clock_khz", i32), ("memory_clock_khz", i32), ("memory_bus_width", i32), ("total_memory", u64),
                ("l2_bytes", i32), ("lds_bytes_per_block", i32), ("warp_size", i32), ("max_threads_per_block", i32)]


# name -> (argtypes, restype); restype int means a status code.
PROTOTYPES = {
    "tcmi_init": ([], ctypes.c_int),
    "tcmi_device_info_get": ([P(DeviceInfo)], ctypes.c_int),
    "tcmi_lost": ([], ctypes.c_int),
    "tcmi_last_error": ([], ctypes.c_char_p),
    "tcmi_version": ([], ctypes.c_char_p),
    "tcmi_compile_options": ([], ctypes.c_char_p),
    "tcmi_malloc": ([u64, P(u64)], ctypes.c_int),
    "tcmi_free": ([u64], ctypes.c_int),
    "tcmi_size": ([u64, P(u64)], ctypes.c_int),
    "tcmi_h2d": ([u64, u64, ctypes.c_void_p, u64], ctypes.c_int),
    "tcmi_d2h": ([ctypes.c_void_p, u64, u64, u64], ctypes.c_int),
    "tcmi_d2d": ([u64, u64, u64, u64, u64], ctypes.c_int),
    "tcmi_fill32": ([u64, u64, u32, u64], ctypes.c_int),
    "tcmi_count_not32": ([u64, u64, u32, u64, P(u64)], ctypes.c_int),
    "tcmi_set_cache_dir": ([ctypes.c_char_p], ctypes.c_int),
    "tcmi_set_include_dir": ([ctypes.c_char_p], ctypes.c_int),
    "tcmi_module_compile": ([ctypes.c_char_p, ctypes.c_char_p, P(u64)], ctypes.c_int),
    "tcmi_precompile": ([ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p], ctypes.c_int),
    "tcmi_module_function": ([u64, ctypes.c_char_p, P(u64)], ctypes.c_int),
    "tcmi_module_unload": ([u64], ctypes.c_int),
    "tcmi_function_attrs": ([u64, P(i32), P(i32), P(i32), P(i32)], ctypes.c_int),
    "tcmi_launch": ([u64, P(u32), P(u32), u32, ctypes.c_void_p, u64], ctypes.c_int),
    "tcmi_sync": ([], ctypes.c_int),
    "tcmi_launch_scratch": ([u64, P(u32), P(u32), u32, ctypes.c_void_p, u64, u64, u64], ctypes.c_int),
    "tcmi_dag_reserve": ([u32], ctypes.c_int),
    "tcmi_launch_dag": ([u32, P(u64), P(u32), P(ctypes.c_uint8), P(u32), u32, P(ctypes.c_uint8), P(i32), P(u32), P(u32)],
                        ctypes.c_int),
    "tcmi_event_create": ([P(u64)], ctypes.c_int),
    "tcmi_event_record": ([u64], ctypes.c_int),
    "tcmi_event_elapsed": ([u64, u64, P(ctypes.c_float)], ctypes.c_int),
    "tcmi_event_destroy": ([u64], ctypes.c_int),
    "tcmi_capture_begin": ([], ctypes.c_int),
    "tcmi_capture_end": ([P(u64)], ctypes.c_int),
    "tcmi_graph_launch": ([u64], ctypes.c_int),
    "tcmi_graph_step": ([u32, P(u64), P(ctypes.c_void_p), P(u64), u64, u64, ctypes.c_void_p, u64], ctypes.c_int),
    "tcmi_graph_destroy": ([u64], ctypes.c_int),
    "tcmi_counters": ([P(u64), u32], ctypes.c_int),
    "tcmi_ceiling_copy": ([u64, u64, u64, u32], ctypes.c_int),
    "tcmi_ceiling_read": ([u64, u64, u64, u32], ctypes.c_int),
}


class TcmiError(RuntimeError):
    pass


class Tcmi:
    """The loaded library; attribute access returns checked callables (status != 0 raises)."""

    def __init__(self, path: pathlib.Path = LIB_PATH):
        if not path.exists():
            raise TcmiError(f"the MI355X backend is not built: {path} is missing")
        self.lib = ctypes.CDLL(str(path))
        for name, (args, res) in PROTOTYPES.items():
            f = getattr(self.lib, name)
            f.argtypes = args
            f.restype = res

    def __getattr__(self, name):
        f = getattr(self.lib, "tcmi_" + name)
        if f.restype is not ctypes.c_int or name in ("lost",):
            return f

        def checked(*args):
            rc = f(*args)
            if rc != 0:
                raise TcmiError(f"tcmi_{name} failed ({rc}): {self.lib.tcmi_last_error().decode()}")
            return rc
        return checked

    def device_info(self) -> dict:
        d = DeviceInfo()
        self.device_info_get(ctypes.byref(d))
        return {k: (getattr(d, k).decode() if isinstance(getattr(d, k), bytes) else getattr(d, k)) for k, _ in d._fields_}


def load(path: pathlib.Path = LIB_PATH) -> Tcmi:
    return Tcmi(path)


TCMI_SCRATCH_BYTES = 64 << 20             # include/tcmi.h
WORKSPACE_SLOT = 8 * 8 + 8                # byte offset of the workspace pointer in a TcmiArgs block


def launch_list_with_scratch(t: Tcmi, items) -> None:
    """Issue lowered launches with the library's device scratch as their workspace
    (tcmi_launch_scratch). `items` is [(functions, launch, args, args_bytes)]: a launch
    record from the lowering (its `kernels`, each with grid, block and lds, and its
    `workspace` in bytes), the module function of each of its kernels, and its packed
    argument block. The scratch size given to the library is each record's own workspace,
    never a caller's figure (an under-stated size would let the kernels write past the
    array); a list any launch of which needs more than TCMI_SCRATCH_BYTES is refused before
    any kernel is enqueued."""
    items = list(items)
    for _, launch, _, _ in items:
        need = int(launch["workspace"])
        if need > TCMI_SCRATCH_BYTES:
            raise TcmiError(f"launch of {launch['kernels'][0]['name']} needs {need} bytes of workspace, "
                            f"the library's scratch holds {TCMI_SCRATCH_BYTES}: nothing launched")
    for functions, launch, args, args_bytes in items:
        for f, k in zip(functions, launch["kernels"]):
            t.launch_scratch(f, (u32 * 3)(*k["grid"]), (u32 * 3)(*k["block"]), k["lds"], args, args_bytes,
                             WORKSPACE_SLOT, int(launch["workspace"]))
