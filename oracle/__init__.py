"""The oracle: a CPU restatement of the reference's float64 semantics and float32
error budget (abho7/tensor-compiler-webgpu src/interp.js, src/gpu/bounds.js,
the judges of src/gpu/harness-m4.js and src/fusion/workloads.js).

TEST INFRASTRUCTURE ONLY. It is imported by tests/, by __graft_entry__.smoke()
(as the checker of one small GPU run) and by bench.py's cpu_baseline leg (timed
as the CPU baseline). No product code path imports, calls or links it; the
MI355X backend fails loudly when its HIP library is missing instead of falling
back to anything here.

Parity status of each function is recorded in the module docstrings:
  interp.evaluate / kernel       pinned: golden/torch.json (1e-12), torch-m3b.f64 (1e-10), closed forms
  bounds.reference_with_bounds   pinned: test/gpu-bounds.test.js closed forms
  bounds.judge*/local_*          pinned: planted errors must fail, exact values must pass
"""
