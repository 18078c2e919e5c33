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
  bounds.streaming_reference     pinned: equal to reference_with_bounds, value and bound, on 40 golden cases
  bounds.judge                   pinned: planted errors (an input moved where its bound is 0, 1.99x / 2.01x
                                 the budget, NaN) in tests/test_oracle_golden.py
  bounds.judge_outputs           pinned: planted errors in tests/test_judges.py (1.99x / 2.01x the budget and
                                 NaN in every output, the last element of the last output, a missing or short
                                 output, unjudgeable fractions of 0.99 % and 1.01 %)
  bounds.local_reference_fused,  pinned: tests/test_judges.py on a host-fused graph (a matmul epilogue, a plain
  bounds.judge_local             column sum, an elementwise chain): the same planted errors in each kind of
                                 node, a missing or short node, unjudgeable fractions of 0.99 % and 1.01 %
  bounds.judge_fused             pinned: the reference's kernel sabotages must fail on the GPU
                                 (tests/test_gpu_direct.py)
"""
