"""The boundary: the C ABI library loads and exports every entry point
include/tcmi.h declares, the ctypes binding declares each with a prototype, the
Node addon loads and exposes its functions, and host-side argument checks fail
cleanly before any device call. No test here touches a GPU."""
import ctypes
import re
import subprocess

import pytest

from conftest import PKG, ROOT


def declared():
    text = (ROOT / "include" / "tcmi.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(tcmi_[a-z0-9_]+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    import tcmi_ctypes
    names = declared()
    assert len(names) >= 30
    lib = ctypes.CDLL(str(tcmi_ctypes.LIB_PATH))
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", str(tcmi_ctypes.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (tcmi_[a-z0-9_]+)", out))
    assert set(names) <= exported
    assert set(tcmi_ctypes.PROTOTYPES) == set(names)


def test_calls_before_init_fail_cleanly():
    import tcmi_ctypes
    t = tcmi_ctypes.load()
    h = tcmi_ctypes.u64()
    # No tcmi_init in this process: allocation must refuse without touching a device.
    rc = t.lib.tcmi_malloc(16, ctypes.byref(h))
    assert rc == 10004
    assert b"tcmi_init" in t.lib.tcmi_last_error()
    assert b"packed-fp32-ops" in t.lib.tcmi_compile_options()
    # So must a whole training step, the launch-list and the stream-graph entry points.
    out = (ctypes.c_float * 1)()
    assert t.lib.tcmi_graph_step(0, None, None, None, 1, 0, out, 4) == 10004
    assert t.lib.tcmi_launch_dag(0, None, None, None, None, 1, None, None, None, None) == 10004
    assert t.lib.tcmi_dag_reserve(1) == 10004
    # The counters read without a device, and nothing has been counted in this process.
    c = (tcmi_ctypes.u64 * 7)()
    assert t.lib.tcmi_counters(c, 7) == 0 and list(c) == [0] * 7
    assert t.lib.tcmi_counters(None, 1) == 10001


def test_node_addon_loads_and_exports():
    js = ("const a=require(process.argv[1]);"
          "const want=['init','info','malloc','free','h2d','d2h','d2d','fill32','countNot32','compile','precompile',"
          "'function','launch','launchMany','sync','eventCreate','eventRecord','eventElapsed','captureBegin','captureEnd',"
          "'graphLaunch','graphStep','launchDag','dagReserve','ceilingCopy','ceilingRead','counters'];"
          "const miss=want.filter((k)=>typeof a[k]!=='function'); if(miss.length){console.log(miss.join());process.exit(2);}"
          "try{a.malloc(16);process.exit(3);}catch(e){if(!/tcmi_init/.test(e.message))process.exit(4);}"
          # graphStep reads its destinations as handles held in doubles: other arrays are refused
          # before anything reaches the C ABI.
          "try{a.graphStep(new Uint8Array(8),[new Float32Array(1)],1,0,new Float32Array(1));process.exit(5);}"
          "catch(e){if(!/Float64Array/.test(e.message))process.exit(6);}"
          # launchMany and launchDag take function handles only as a Float64Array of whole
          # numbers, dims/offsets only as Uint32Arrays: NaN, negative or fractional handles
          # and reinterpretable arrays of the right byte length are refused the same way.
          "const U=(n)=>new Uint32Array(n);"
          "const many=[[new Float32Array(2),U(7),new Uint8Array(0),U(2)],[new Float64Array([NaN]),U(7),new Uint8Array(0),U(2)],"
          "[new Float64Array([-1]),U(7),new Uint8Array(0),U(2)],[new Float64Array([1.5]),U(7),new Uint8Array(0),U(2)],"
          "[new Float64Array(1),new Float32Array(7),new Uint8Array(0),U(2)],[new Float64Array(1),U(7),new Uint8Array(0),new Int32Array(2)]];"
          "for(const [i,m] of many.entries()){try{a.launchMany(...m);console.log('many',i);process.exit(7);}"
          "catch(e){if(!/launchMany/.test(e.message)||/tcmi_init/.test(e.message)){console.log('many',i,e.message);process.exit(8);}}}"
          "const dag=(f,d)=>[f,d,new Uint8Array(0),U(2),1,new Uint8Array(1),new Int32Array(1),U(2),U(0)];"
          "for(const [i,m] of [dag(new Float64Array([NaN]),U(7)),dag(new Float64Array([2**60]),U(7)),dag(new Float64Array(1),new Int32Array(7)),"
          "dag(new BigUint64Array(1),U(7))].entries()){try{a.launchDag(...m);console.log('dag',i);process.exit(9);}"
          "catch(e){if(!/launchDag/.test(e.message)||/tcmi_init/.test(e.message)){console.log('dag',i,e.message);process.exit(10);}}}")
    p = subprocess.run(["node", "-e", js, str(PKG / "lib" / "tcmi.node")], capture_output=True, text=True)
    assert p.returncode == 0, p.stdout + p.stderr


def test_backend_entry_point_exports_what_the_reference_binds():
    """js/src/mi355x/index.js, the module a reference harness requires in place of
    src/gpu/runtime.js, lower-fused.js, trainer-fused.js and bench.js: every name the
    integration binds is there, and what it gives is the backend's own (its lowering of
    the reference transformer's fused training step holds the same launches as the
    trainer's, and a launch list the batch checker accepts)."""
    js = ("const be=require(process.argv[1]);"
          "const want=['lowerMI355X','kernelSources','HipRunner','Program','precompile','fusedStep','fusedForward','HipTrainer',"
          "'HipBench','summarize','verdict','fuseAttention','planArena'];"
          "const miss=want.filter((k)=>typeof be[k]!=='function'); if(miss.length){console.log(miss.join());process.exit(2);}"
          "const {modelStep}=require(process.argv[2]);const m=modelStep({model:'transformer-ref'});"
          "const fs=be.fusedStep(m.step);"
          "const keep=[fs.loss,fs.logits].concat(Object.values(fs.outputs));"
          "const lo=be.lowerMI355X(fs.graph,{perf:true,keep,absorb:true});"
          "if(lo.launches.map((l)=>l.node).join()!==fs.lowered.launches.map((l)=>l.node).join())process.exit(3);"
          "const {checkBatches}=require(process.argv[3]);"
          "const c=checkBatches(be.lowerMI355X(fs.graph,{perf:true,keep,absorb:true,batch:false}),lo);"
          "if(!c.ok){console.log(c.why);process.exit(4);}"
          "if(be.kernelSources(lo).size<10)process.exit(5);")
    src = PKG / "js" / "src"
    p = subprocess.run(["node", "-e", js, str(src / "mi355x" / "index.js"), str(src / "builders" / "models.js"),
                        str(src / "testing" / "batch_check.js")], capture_output=True, text=True)
    assert p.returncode == 0, (p.returncode, p.stdout + p.stderr)


def test_kernel_headers_compile_for_gfx950_offline(tool):
    """The skeletons compile with hiprtc for gfx950 (no GPU): every direct case's kernels as one module."""
    out = tool("precompile", {"group": "direct", "arch": "gfx950"})
    assert out["kernels"] > 30


def test_scratch_launches_take_their_size_from_the_lowering(tool):
    """launch_list_with_scratch (the Python binding of tcmi_launch_scratch) gives the library
    each launch record's own workspace as the scratch size, and refuses a launch list any
    launch of which needs more than the library's 64 MiB before any kernel is enqueued
    (a stand-in library records the calls; nothing reaches a GPU)."""
    import tcmi_ctypes
    calls = []

    class Stub:
        def launch_scratch(self, *args):
            calls.append(args)

    d = tool("scratch-kernels")
    launches = d["launches"]
    assert all(0 < launch["workspace"] <= tcmi_ctypes.TCMI_SCRATCH_BYTES for launch in launches)
    items = [([11, 12], launch, 0, 272) for launch in launches]
    tcmi_ctypes.launch_list_with_scratch(Stub(), items)
    assert [c[-1] for c in calls] == [launch["workspace"] for launch in launches for _ in launch["kernels"]]
    assert all(c[-2] == tcmi_ctypes.WORKSPACE_SLOT for c in calls)
    calls.clear()
    big = dict(launches[1], workspace=tcmi_ctypes.TCMI_SCRATCH_BYTES + 4)
    with pytest.raises(tcmi_ctypes.TcmiError, match="nothing launched"):
        tcmi_ctypes.launch_list_with_scratch(Stub(), items[:1] + [([11, 12], big, 0, 272)])
    assert calls == []
