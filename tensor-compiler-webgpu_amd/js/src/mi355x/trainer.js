'use strict';
// A fused training step on the MI355X: the drop-in for the reference's
// fusedStep / FusedTrainer (src/fusion/trainer-fused.js:18-109 in
// abho7/tensor-compiler-webgpu).
//
// fusedStep(step) fuses a step graph keeping the loss, the logits and every
// new parameter and state value, renumbers the step's ids into the fused graph
// and lowers it. HipTrainer makes every buffer, constant and packed launch
// once; train(x, y) writes the batch, enqueues every launch, copies each new
// parameter/state value back into its input buffer on the device, and reads
// back only the loss (one sync per step). read(names) returns current values;
// destroy() frees everything.

const { fuse } = require('../fusion/fuse');
const { lowerMI355X } = require('./lower');

/**
 * Fuse and lower a step from the builders ({ graph, loss, logits, inputs, outputs, cotangent, ... }).
 * `lowered` is the perf lowering the trainer runs (reshapes share buffers,
 * transposes read in place by their matmuls; `perf: false` turns it off);
 * `checked` is the plain lowering, one launch per node, for node-by-node checks.
 */
function fusedStep(step, options) {
  const o = options || {};
  const keep = [step.loss, step.logits].concat(Object.values(step.outputs));
  const f = fuse(step.graph, { keep, sabotage: o.passSabotage });
  const at = (id) => f.index.get(id);
  const remap = (m) => { const r = {}; for (const k of Object.keys(m)) r[k] = at(m[k]); return r; };
  const checked = lowerMI355X(f.graph, { sabotage: o.sabotage, tuning: o.tuning });
  const lowered = o.perf === false ? checked
    : lowerMI355X(f.graph, { sabotage: o.sabotage, tuning: o.tuning, perf: true, keep: keep.map(at) });
  return Object.assign({}, step, {
    graph: f.graph, fusion: f, original: step.graph,
    loss: at(step.loss), logits: at(step.logits),
    inputs: remap(step.inputs), outputs: remap(step.outputs),
    lowered, checked,
  });
}

class HipTrainer {
  /** `step` from fusedStep (or an unfused step with `lowered`); `params`/`state` map names to values. */
  constructor(runner, step, params, state) {
    this.runner = runner;
    this.a = runner.a;
    this.step = step;
    this.program = runner.prepare(step.graph, step.lowered);
    const p = this.program;
    const cot = step.graph.inputId(step.cotangent);
    if (cot === undefined) throw new Error(`the step has no cotangent input '${step.cotangent}'`);
    p.write(cot, new Float32Array([1]));
    const all = Object.assign({}, params, state || {});
    for (const name of Object.keys(all)) {
      if (step.inputs[name] === undefined) throw new Error(`the step has no input '${name}'`);
      p.write(step.inputs[name], all[name]);
    }
    this.names = Object.keys(all);
    this.feedback = this.names.map((name) => {
      const from = step.outputs[name], to = step.inputs[name];
      if (from === undefined) throw new Error(`the step has no output for '${name}'`);
      return [p.bufs[from], p.bufs[to], p.n[to] * 4];
    });
    this.lossBuf = new Float32Array(1);
  }

  /** Enqueue one step (no sync): batch, every launch, the feedback copies. */
  enqueue(x, y) {
    const { step, program: p } = this;
    p.write(step.inputs.x, x);
    p.write(step.inputs.y, y);
    p.run();
    for (const [from, to, bytes] of this.feedback) this.a.d2d(to, 0, from, 0, bytes);
  }

  /** One training step; returns the loss computed from the parameters before the update. */
  train(x, y) {
    this.enqueue(x, y);
    this.a.d2h(this.program.bufs[this.step.loss], 0, this.lossBuf);
    return this.lossBuf[0];
  }

  read(names) {
    const out = {};
    for (const n of names) out[n] = this.program.read(this.step.inputs[n]);
    return out;
  }

  destroy() { this.program.destroy(); }
}

module.exports = { fusedStep, HipTrainer };
