'use strict';
// A fused training step on the MI355X: the drop-in for the reference's
// fusedStep / FusedTrainer (src/fusion/trainer-fused.js:18-109 in
// abho7/tensor-compiler-webgpu).
//
// fusedStep(step) fuses a step graph keeping the loss, the logits and every
// new parameter and state value, renumbers the step's ids into the fused graph
// and lowers it (the perf lowering, and the plain one for node-by-node checks).
//
// HipTrainer makes every buffer, constant and packed launch once. Where the
// reference copies each new parameter back onto its input buffer after every
// step (trainer-fused.js:72), this trainer keeps two programs over the same
// buffers with each parameter's input and output buffers exchanged: step t
// runs program t mod 2, which reads the parameters the previous step wrote, so
// a step is its launches alone — no copies — and, with `graph`, the replay of
// one captured HIP graph. train(x, y) writes the batch, enqueues the step and
// reads back only the loss (one sync per step); read(names) returns current
// values; destroy() frees everything. With `arena`, every buffer but the
// parameters, state, batch, loss and logits is placed by live range in one
// allocation (arena.js), shared by both programs.

const { fuse } = require('../fusion/fuse');
const { fuseAttentionTraining } = require('../fusion/attention');
const { lowerMI355X } = require('./lower');

/**
 * Products transposed by their one reader, formed transposed instead (in place, on the
 * fused graph, ids unchanged): transpose(matmul(A, B)) over the last two axes, where A is
 * itself transpose(A0) over them and only that transpose reads the product, becomes
 * matmul(transpose(B), A0) — the product's node now holds transpose(B) and the
 * transpose's node the product. Every output element sums the same terms in the same
 * order of k (only which operand is which changes), and the result comes out in the
 * layout its readers take. Autodiff's gradient of the transposed keys of an attention,
 * transpose(matmul(transpose(q), dS)), is one: the key gradient then has the query
 * gradient's layout, so the same kernels (and batches) read both. `origin` (the fusion's
 * map of each node to the original node holding its value) marks the new transpose -1:
 * no original node holds transpose(B), and `index` (original id -> fused id) drops the
 * product's entry, since no node holds the product itself any more. Returns the count.
 */
function formTransposedProducts(graph, keep, origin, index) {
  const readers = graph.nodes.map(() => 0);
  for (const n of graph.nodes) for (const i of n.inputs) readers[i]++;
  const swapsLast = (n) => n.op === 'transpose' && n.attrs.perm.every((p, d) => {
    const r = n.attrs.perm.length;
    return d < r - 2 ? p === d : p === (d === r - 2 ? r - 1 : r - 2);
  });
  let count = 0;
  for (const t of graph.nodes) {
    if (!swapsLast(t) || t.shape.length < 2) continue;
    const x = graph.nodes[t.inputs[0]];
    if (x.op !== 'matmul' || keep.has(x.id) || readers[x.id] !== 1) continue;
    const a = graph.nodes[x.inputs[0]], b = graph.nodes[x.inputs[1]];
    if (!swapsLast(a) || a.shape.length !== b.shape.length || a.shape.slice(0, -2).join() !== b.shape.slice(0, -2).join()) continue;
    const bt = b.shape.slice(0, -2).concat([b.shape[b.shape.length - 1], b.shape[b.shape.length - 2]]);
    graph.nodes[x.id] = { id: x.id, op: 'transpose', inputs: [b.id], attrs: { perm: t.attrs.perm.slice() }, shape: bt };
    graph.nodes[t.id] = { id: t.id, op: 'matmul', inputs: [x.id, a.inputs[0]], attrs: {}, shape: t.shape.slice() };
    readers[b.id]++;
    if (index && origin && origin[x.id] >= 0 && index.get(origin[x.id]) === x.id) index.delete(origin[x.id]);
    if (origin) origin[x.id] = -1;
    count++;
  }
  return count;
}

/**
 * Fuse and lower a step from the builders ({ graph, loss, logits, inputs, outputs, cotangent, ... }).
 * `lowered` is the perf lowering the trainer runs (reshapes share buffers,
 * transposes read in place by their matmuls; `perf: false` turns it off);
 * `checked` is the plain lowering, one launch per node, for node-by-node checks. Both
 * lower the fused graph with its transposed products formed transposed (above). With
 * `contract`, the perf lowering adds nothing to the fusion contract's partition beyond
 * views and batching: no row folds, no absorbed producers, no relus applied on load.
 */
function fusedStep(step, options) {
  const o = options || {};
  const keep = [step.loss, step.logits].concat(Object.values(step.outputs));
  let f = fuse(step.graph, { keep, sabotage: o.passSabotage });
  formTransposedProducts(f.graph, new Set(keep.map((id) => f.index.get(id))), f.origin, f.index);
  // With `attention`, each attention and its gradient take the attention extension's
  // nodes (fusion/attention.js fuseAttentionTraining); off, the contract's partition.
  if (o.attention) f = fuseAttentionTraining(f, { keep });
  const at = (id) => f.index.get(id);
  const remap = (m) => { const r = {}; for (const k of Object.keys(m)) r[k] = at(m[k]); return r; };
  const checked = lowerMI355X(f.graph, { sabotage: o.sabotage, tuning: o.tuning });
  const lowered = o.perf === false ? checked
    : o.contract ? lowerMI355X(f.graph, { sabotage: o.sabotage, tuning: o.tuning, perf: true, keep: keep.map(at), batch: o.batch,
      rowFolds: false, absorb: false, loadOps: false })
      : lowerMI355X(f.graph, { sabotage: o.sabotage, tuning: o.tuning, perf: true, keep: keep.map(at), batch: o.batch, absorb: true,
        loadOps: o.loadOps, formRows: o.formRows });
  return Object.assign({}, step, {
    graph: f.graph, fusion: f, original: step.graph,
    loss: at(step.loss), logits: at(step.logits),
    inputs: remap(step.inputs), outputs: remap(step.outputs),
    lowered, checked,
  });
}

/**
 * Fuse and lower a forward pass ({ graph, logits, loss } from a builder) keeping the logits
 * and the loss, as the reference's fused forward check does (src/gpu/harness-m4.js:281-289:
 * fuse(f.graph, { keep: [f.logits, f.loss] }) then lowerFused). `checked` is the plain
 * lowering (one launch per node), `lowered` the perf lowering with those two kept.
 */
function fusedForward(fwd, options) {
  const o = options || {};
  const keep = [fwd.logits, fwd.loss];
  const f = fuse(fwd.graph, { keep, sabotage: o.passSabotage });
  const at = (id) => f.index.get(id);
  const checked = lowerMI355X(f.graph, { sabotage: o.sabotage, tuning: o.tuning });
  const lowered = o.perf === false ? checked
    : lowerMI355X(f.graph, { sabotage: o.sabotage, tuning: o.tuning, perf: true, keep: keep.map(at), absorb: true });
  return { graph: f.graph, fusion: f, original: fwd.graph, logits: at(fwd.logits), loss: at(fwd.loss), lowered, checked };
}

class HipTrainer {
  /**
   * `step` from fusedStep (or an unfused step with `lowered`); `params`/`state`
   * map names to values; options.graph: replay each step as a captured HIP graph;
   * options.arena: place the step's other buffers by live range in one allocation;
   * options.streams: issue the step's independent launches on up to 4 streams.
   */
  constructor(runner, step, params, state, options) {
    const o = options || {};
    this.runner = runner;
    this.a = runner.a;
    this.step = step;
    this.graph = !!o.graph;
    if (this.graph && o.streams > 1) throw new Error('graph replay and several streams are not combined (multi-stream capture is switched off)');
    const keep = [step.loss, step.logits].concat(Object.values(step.outputs));
    const first = runner.prepare(step.graph, step.lowered, Object.assign(o.arena ? { arena: { keep } } : {}, { streams: o.streams }));
    const cot = step.graph.inputId(step.cotangent);
    if (cot === undefined) throw new Error(`the step has no cotangent input '${step.cotangent}'`);
    first.write(cot, new Float32Array([1]));
    const all = Object.assign({}, params, state || {});
    this.names = Object.keys(all);
    // The second program: every parameter's input and output buffers exchanged,
    // and the nodes sharing a buffer (aliases) re-pointed at the exchanged one.
    const bufs = first.bufs.slice();
    for (const name of this.names) {
      const from = step.outputs[name], to = step.inputs[name];
      if (to === undefined) throw new Error(`the step has no input '${name}'`);
      if (from === undefined) throw new Error(`the step has no output for '${name}'`);
      if (from === to) throw new Error(`'${name}' is its own output`);
      first.write(to, all[name]);
      bufs[to] = first.bufs[from];
      bufs[from] = first.bufs[to];
    }
    for (const [node, source] of step.lowered.aliases || []) bufs[node] = bufs[source];
    const second = runner.prepare(step.graph, step.lowered, { buffers: bufs, arena: first.arena, streams: o.streams });
    this.programs = [first, second];
    this.turn = 0;   // the program the next step runs; its parameter inputs hold the current values
    this.lossBuf = new Float32Array(1);
  }

  /** The program the next step runs. */
  get program() { return this.programs[this.turn]; }

  /** Enqueue one step on the resident batch (no sync): every launch, then the buffers' roles swap. */
  advance() {
    const p = this.programs[this.turn];
    if (this.graph) p.replay(); else p.run();
    this.lossAt = p.bufs[this.step.loss];
    this.turn ^= 1;
  }

  /** Enqueue one step (no sync): the batch, then every launch. */
  enqueue(x, y) {
    const p = this.programs[this.turn];
    p.write(this.step.inputs.x, x);
    p.write(this.step.inputs.y, y);
    this.advance();
  }

  /**
   * One training step; returns the loss computed from the parameters before the update.
   * With graph replay the whole step (batch upload, replay, loss readback) is one
   * native call (tcmi_graph_step).
   */
  train(x, y) {
    if (!this.graph) {
      this.enqueue(x, y);
      this.a.d2h(this.lossAt, 0, this.lossBuf);
      return this.lossBuf[0];
    }
    const p = this.programs[this.turn];
    if (!p.graphHandle) p.capture();
    const ix = this.step.inputs.x, iy = this.step.inputs.y;
    const xs = x instanceof Float32Array ? x : Float32Array.from(x);
    const ys = y instanceof Float32Array ? y : Float32Array.from(y);
    if (xs.length !== p.n[ix] || ys.length !== p.n[iy]) throw new Error(`batch of ${xs.length} and ${ys.length} values, the step takes ${p.n[ix]} and ${p.n[iy]}`);
    this.a.graphStep(Float64Array.from([p.bufs[ix], p.bufs[iy]]), [xs, ys], p.graphHandle, p.bufs[this.step.loss], this.lossBuf);
    this.lossAt = p.bufs[this.step.loss];
    this.turn ^= 1;
    return this.lossBuf[0];
  }

  read(names) {
    const out = {};
    for (const n of names) out[n] = this.program.read(this.step.inputs[n]);
    return out;
  }

  destroy() {
    this.programs[1].destroy();
    this.programs[0].destroy();
  }
}

module.exports = { fusedStep, fusedForward, HipTrainer, formTransposedProducts };
