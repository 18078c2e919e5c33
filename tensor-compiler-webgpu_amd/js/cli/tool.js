#!/usr/bin/env node
'use strict';
// Command-line entry to the host side, for harnesses in other processes
// (the Python tests and bench). Usage:
//
//   node tool.js <command> [request.json] [--out DIR]
//
// CPU commands print one JSON document on stdout:
//   builder-cases    the hand-built graphs of the reference's exported cases
//   grad             request {cases: [{name, graph, outputs}]} -> gradient graphs
//   fuse             request {graphs: [{name, graph, keep, recompute?, sabotage?}]} -> fused graphs
//   lower            request {graph, fuse?: {keep}} -> launch records (sources omitted)
//   model-fusion     fusion summaries of the reference's transformer forward pass and Adam step
//   direct-catalogue the direct adversarial cases: names, kinds, patterns, and what fuse() makes of each
//   transformer-init the reference transformer (golden config) forward + gradient graph and its inputs
// GPU commands write a bundle (manifest.json + data.f32) under --out:
//   gpu-direct       every direct case, fused, canary-padded, on the GPU
//   gpu-graphs       request {graphs: [{name, graph, inputs, keep, unfused?}]} fused (and unfused) on the GPU

const fs = require('fs');
const fs_ = fs;
const path = require('path');
const { Graph } = require('../src/ir/graph');
const { grad } = require('../src/autodiff');
const { fuse, fusionSummary } = require('../src/fusion/fuse');
const { lowerMI355X } = require('../src/mi355x/lower');
const { builderCases } = require('../src/testing/cases');
const { fusedDirectCases } = require('../src/builders/direct_cases');
const tf = require('../src/builders/transformer');
const { Bundle } = require('../src/testing/bundle');

function readRequest(argv) {
  const file = argv.find((a, i) => i > 0 && !a.startsWith('--') && argv[i - 1] !== '--out');
  if (!file) return {};
  return JSON.parse(fs.readFileSync(file, 'utf8'));
}

function outDir(argv) {
  const i = argv.indexOf('--out');
  if (i < 0 || !argv[i + 1]) throw new Error('--out DIR is required');
  return argv[i + 1];
}

const fusedOut = (f) => ({
  graph: f.graph.toJSON(), origin: f.origin,
  groups: f.groups.map((g) => ({ sink: g.sink, members: Array.from(g.members), kind: g.kind, root: g.root, pattern: g.pattern })),
});

function modelFusion() {
  const cfg = tf.REFERENCE_CONFIG;
  const V = 16, B = 4;
  const fwd = tf.buildForward(V, B, cfg);
  const step = tf.buildStep(V, B, cfg, tf.ADAM_3B);
  const out = [];
  const cases = [
    { label: 'forward', graph: fwd.graph, keep: [fwd.logits, fwd.loss] },
    { label: 'step', graph: step.graph, keep: [step.loss, step.logits].concat(Object.values(step.outputs)) },
  ];
  for (const c of cases) {
    const f = fuse(c.graph, { keep: c.keep });
    const epilogues = f.groups.filter((g) => g.kind === 'epilogue');
    const withActivation = epilogues.filter((g) => Array.from(g.members).some((id) => ['tanh', 'relu'].includes(c.graph.nodes[id].op))).length;
    let threw = null;
    try { fuse(c.graph, { keep: c.keep, sabotage: 'fusion-absorbs-shared' }); } catch (e) { threw = String(e.message); }
    out.push(Object.assign({ graph: c.label }, fusionSummary(c.graph, f), { epilogues: epilogues.length, epiloguesWithActivation: withActivation,
      passSabotageError: threw, unfusedLaunches: lowerMI355X(c.graph).launches.length, fusedLaunches: lowerMI355X(f.graph).launches.length }));
  }
  return out;
}

function directCatalogue() {
  return fusedDirectCases().map((c) => {
    const f = fuse(c.graph);
    const launched = f.graph.nodes.filter((n) => n.op !== 'input' && n.op !== 'const');
    return { name: c.name, kind: c.kind, pattern: c.pattern, matmul: c.matmul || null,
      launched: launched.map((n) => ({ op: n.op, kind: n.attrs.kind || null, pattern: n.attrs.pattern || null })),
      graph: c.graph.toJSON(), inputs: c.inputs };
  });
}

function transformerInit(req) {
  const cfg = Object.assign({}, tf.REFERENCE_CONFIG);
  const V = req.V || 16, B = req.batch || 4, seed = req.seed || 1;
  const fwd = tf.buildForward(V, B, cfg);
  const names = tf.paramSpec(V, cfg).map((s) => s[0]);
  const G = grad(fwd.graph, [fwd.loss], names.map((n) => fwd.ids[n]));
  const params = tf.initParams(V, seed, cfg);
  const { x, y } = tf.encodeBatch(req.firstBatch, V, cfg.T);
  return { graph: G.graph.toJSON(), logits: fwd.logits, loss: fwd.loss, names, grads: G.grads, cotangent: G.cotangents[0],
    params, x: Array.from(x), y: Array.from(y) };
}

/** Compile, offline, the kernels a named group of GPU runs will ask for (same module text as on the box). */
function precompileGroup(group, arch) {
  const { precompile } = require('../src/mi355x/runner');
  if (group === 'direct') return precompile(fusedDirectCases().map((c) => lowerMI355X(fuse(c.graph).graph)), arch);
  if (group === 'models') {
    // The trainer compiles a step's kernels as one module: the same text here.
    const { modelStep } = require('../src/builders/models');
    const { fusedStep } = require('../src/mi355x/trainer');
    const reqs = [{ model: 'mlp' }, { model: 'transformer', B: 1 }, { model: 'transformer', B: 64 }, { model: 'transformer-ref' }];
    let n = 0;
    for (const r of reqs) n += precompile([fusedStep(modelStep(r).step).lowered], arch);
    return n;
  }
  throw new Error(`unknown precompile group '${group}'`);
}

async function gpuDirect(dir) {
  const { HipRunner } = require('../src/mi355x/runner');
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  const cases = fusedDirectCases();
  const plans = cases.map((c) => { const f = fuse(c.graph); return { f, lowered: lowerMI355X(f.graph) }; });
  process.stderr.write(`gpu-direct: compiling ${plans.length} launch lists\n`);
  runner.functions(plans.map((p) => p.lowered));
  for (const [k, c] of cases.entries()) {
    process.stderr.write(`gpu-direct: ${c.name}\n`);
    const { f, lowered } = plans[k];
    const inputs = {};
    for (const n of c.graph.inputs()) inputs[n.attrs.name] = Float32Array.from(c.inputs[n.attrs.name]);
    const r = await runner.run(f.graph, lowered, inputs, { canary: true });
    const gpu = {};
    f.graph.nodes.forEach((n) => { gpu[n.id] = bundle.put(r.values[n.id]); });
    const ins = {};
    for (const k of Object.keys(inputs)) ins[k] = bundle.put(inputs[k]);
    bundle.add({ name: c.name, kind: c.kind, pattern: c.pattern, graph: c.graph.toJSON(), fused: f.graph.toJSON(), origin: f.origin,
      inputs: ins, gpu, canaryIntact: r.canaryIntact, launches: lowered.launches.map((l) => ({ node: l.node, kind: l.kind, code: l.code })) });
  }
  bundle.close({ device: runner.info() });
}

async function gpuGraphs(req, dir) {
  const { HipRunner } = require('../src/mi355x/runner');
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  for (const c of req.graphs) {
    process.stderr.write(`gpu-graphs: ${c.name}\n`);
    const g = Graph.fromJSON(c.graph);
    const inputs = {};
    for (const n of g.inputs()) inputs[n.attrs.name] = Float32Array.from(c.inputs[n.attrs.name]);
    const f = fuse(g, { keep: c.keep || [] });
    const lf = lowerMI355X(f.graph);
    const rf = await runner.run(f.graph, lf, inputs, { canary: true });
    const entry = { name: c.name, fused: f.graph.toJSON(), origin: f.origin, gpuFused: {}, canaryFused: rf.canaryIntact };
    f.graph.nodes.forEach((n) => { entry.gpuFused[n.id] = bundle.put(rf.values[n.id]); });
    if (c.unfused) {
      const lu = lowerMI355X(g);
      const ru = await runner.run(g, lu, inputs, { canary: true });
      entry.gpuUnfused = {};
      g.nodes.forEach((n) => { entry.gpuUnfused[n.id] = bundle.put(ru.values[n.id]); });
      entry.canaryUnfused = ru.canaryIntact;
    }
    bundle.add(entry);
  }
  bundle.close({ device: runner.info() });
}

/**
 * Config-2 programs on the GPU: for each seed, forward and gradient graphs at [R, C],
 * fused (and with `unfused`, unfused), canary-padded; the bundle holds the inputs,
 * the kept outputs of each variant (by original node id) and the canary verdicts.
 */
async function gpuChains(req, dir) {
  const { HipRunner } = require('../src/mi355x/runner');
  const { chainWorkload, chainInputs } = require('../src/builders/chains');
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  for (const seed of req.seeds) {
    const w = chainWorkload(seed, req.R, req.C);
    const inputs = chainInputs(seed, req.R, req.C);
    const ins = {};
    for (const k of Object.keys(inputs)) ins[k] = bundle.put(inputs[k]);
    for (const kind of ['forward', 'gradient']) {
      process.stderr.write(`gpu-chains: seed ${seed} ${kind}\n`);
      const v = w[kind];
      const f = fuse(v.graph, { keep: v.keep });
      const lf = lowerMI355X(f.graph);
      const rf = await runner.run(f.graph, lf, inputs, { canary: true });
      const entry = { name: `c2-p${seed}-${kind}`, seed, kind, graph: v.graph.toJSON(), keep: v.keep, inputs: ins,
        fusedLaunches: lf.launches.length, canaryFused: rf.canaryIntact.every(Boolean), fused: {} };
      for (const id of v.keep) entry.fused[id] = bundle.put(rf.values[f.index.get(id)]);
      if (req.unfused) {
        const lu = lowerMI355X(v.graph);
        const ru = await runner.run(v.graph, lu, inputs, { canary: true });
        entry.unfused = {};
        for (const id of v.keep) entry.unfused[id] = bundle.put(ru.values[id]);
        entry.canaryUnfused = ru.canaryIntact.every(Boolean);
      }
      bundle.add(entry);
    }
  }
  bundle.close({ device: runner.info() });
}

/**
 * The step graph of a model request as a bundle: the original and fused graphs,
 * the origin map, the ids that matter, and the step's inputs (parameters, state,
 * batch k, cotangent 1) as float32 arrays. No GPU.
 */
function stepGraph(req, dir) {
  const { modelStep } = require('../src/builders/models');
  const { fusedStep } = require('../src/mi355x/trainer');
  const m = modelStep(req);
  const fs = fusedStep(m.step);
  const bundle = new Bundle(dir);
  const b = m.batch(req.batchIndex || 0);
  const values = Object.assign({}, m.params, m.state, { x: b.x, y: b.y });
  values[m.step.cotangent] = [1];
  const inputs = {};
  for (const k of Object.keys(values)) inputs[k] = bundle.put(values[k]);
  bundle.add({ name: req.model, graph: m.step.graph.toJSON(), fused: fs.graph.toJSON(), origin: fs.fusion.origin, inputs,
    loss: m.step.loss, logits: m.step.logits, outputs: m.step.outputs, stepInputs: m.step.inputs, names: m.step.names,
    launchesFused: fs.lowered.launches.length, info: m.info });
  bundle.close();
}

/**
 * Node-local run of a model's fused step: every launch reads the float32
 * reference operands given in `values.f32` (all fused-graph nodes, in node
 * order, as the checker computed them) and writes its own output (with canaries).
 */
async function gpuLocal(req, dir) {
  const { modelStep } = require('../src/builders/models');
  const { fusedStep } = require('../src/mi355x/trainer');
  const { HipRunner } = require('../src/mi355x/runner');
  const m = modelStep(req);
  const fs = fusedStep(m.step, { sabotage: req.sabotage });
  const raw = fs_.readFileSync(req.valuesFile);
  const data = new Float32Array(raw.buffer, raw.byteOffset, raw.byteLength / 4);
  const values = [];
  let off = 0;
  for (const node of fs.graph.nodes) {
    const n = node.shape.reduce((a, c) => a * c, 1);
    values.push(data.subarray(off, off + n));
    off += n;
  }
  if (off !== data.length) throw new Error(`values file holds ${data.length} floats, the fused graph needs ${off}`);
  const runner = HipRunner.create();
  const out = await runner.runLocal(fs.graph, fs.lowered, values, { canary: true });
  const bundle = new Bundle(dir);
  const gpu = {};
  for (const l of fs.lowered.launches) gpu[l.node] = bundle.put(out[l.node]);
  bundle.add({ name: req.model, gpu, canaryIntact: fs.lowered.launches.every((l) => out.canaryIntact[l.node]),
    launches: fs.lowered.launches.length });
  bundle.close({ device: runner.info() });
}

/**
 * Train a model for `steps` steps on the GPU with the fused trainer; with
 * `consistency`, also run the first steps through runner.run on the same fused
 * graph and compare loss and parameters bit for bit (the trainer's feedback
 * against the checked path, harness-m4.js:310-330).
 */
async function gpuTrain(req) {
  const { modelStep } = require('../src/builders/models');
  const { fusedStep, HipTrainer } = require('../src/mi355x/trainer');
  const { HipRunner } = require('../src/mi355x/runner');
  const m = modelStep(req);
  const fs = fusedStep(m.step);
  const runner = HipRunner.create();
  const trainer = new HipTrainer(runner, fs, m.params, m.state);
  const losses = [];
  let identical = null;
  const names = Object.keys(Object.assign({}, m.params, m.state));
  let inputs = null;
  if (req.consistency) {
    identical = true;
    inputs = {};
    for (const n of names) inputs[n] = Float32Array.from(Object.assign({}, m.params, m.state)[n]);
  }
  for (let t = 0; t < req.steps; t++) {
    const b = m.batch(req.sameBatch ? 0 : t);
    const loss = trainer.train(b.x, b.y);
    losses.push(loss);
    if (req.consistency && t < (req.consistencySteps || 3)) {
      const feed = Object.assign({}, inputs, { x: b.x, y: b.y });
      feed[fs.cotangent] = [1];
      const r = await runner.run(fs.graph, fs.lowered, feed);
      if (!Object.is(r.values[fs.loss][0], loss)) identical = false;
      for (const n of names) inputs[n] = r.values[fs.outputs[n]];
    }
  }
  if (req.consistency) {
    const now = trainer.read(names);
    for (const n of names) {
      const a = now[n], b = inputs[n];
      if ((req.consistencySteps || 3) >= req.steps) for (let i = 0; i < a.length; i++) if (!Object.is(a[i], b[i])) { identical = false; break; }
    }
  }
  const params = req.returnParams ? trainer.read(Object.keys(m.params)) : null;
  if (params) for (const k of Object.keys(params)) params[k] = Array.from(params[k]);
  trainer.destroy();
  return { losses, identical, params, launches: fs.lowered.launches.length, unfusedNodes: m.step.graph.nodes.length, info: m.info };
}

async function main() {
  const argv = process.argv.slice(2);
  const cmd = argv[0];
  const req = readRequest(argv);
  let out;
  switch (cmd) {
    case 'builder-cases': out = builderCases(); break;
    case 'grad':
      out = req.cases.map((c) => {
        const g = Graph.fromJSON(c.graph);
        const G = grad(g, c.outputs, g.inputs().map((n) => n.id));
        return { name: c.name, graph: G.graph.toJSON(), grads: G.grads, cotangents: G.cotangents };
      });
      break;
    case 'fuse':
      out = req.graphs.map((c) => {
        const g = Graph.fromJSON(c.graph);
        try {
          const f = fuse(g, { keep: c.keep || [], recompute: !!c.recompute, sabotage: c.sabotage });
          return Object.assign({ name: c.name, summary: fusionSummary(g, f) }, fusedOut(f));
        } catch (e) {
          return { name: c.name, error: String(e.message) };
        }
      });
      break;
    case 'lower': {
      const g = Graph.fromJSON(req.graph);
      const target = req.fuse ? fuse(g, { keep: req.fuse.keep || [] }).graph : g;
      const l = lowerMI355X(target, { sabotage: req.sabotage });
      out = { workspace: l.workspace, launches: l.launches.map((x) => Object.assign({}, x, { params: Array.from(x.params),
        kernels: x.kernels.map((k) => ({ name: k.name, grid: k.grid, block: k.block, lds: k.lds, source: req.sources ? k.source : undefined })) })) };
      break;
    }
    case 'model-fusion': out = modelFusion(); break;
    case 'direct-catalogue': out = directCatalogue(); break;
    case 'transformer-init': out = transformerInit(req); break;
    case 'chain-graphs': {
      const { chainWorkload } = require('../src/builders/chains');
      out = req.seeds.map((seed) => {
        const w = chainWorkload(seed, req.R, req.C);
        const one = (v) => {
          const f = fuse(v.graph, { keep: v.keep });
          const l = lowerMI355X(f.graph);
          return { graph: v.graph.toJSON(), keep: v.keep, cotangent: v.cotangent || null,
            fusedBytes: l.launches.reduce((s, x) => s + x.bytes, 0), fusedLaunches: l.launches.length };
        };
        return { seed, ops: w.ops, forward: one(w.forward), gradient: one(w.gradient) };
      });
      break;
    }
    case 'precompile': out = { kernels: precompileGroup(req.group || 'direct', req.arch) }; break;
    case 'gpu-direct': await gpuDirect(outDir(argv)); out = { ok: true }; break;
    case 'step-graph': stepGraph(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-local': await gpuLocal(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-train': out = await gpuTrain(req); break;
    case 'gpu-chains': await gpuChains(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-graphs': await gpuGraphs(req, outDir(argv)); out = { ok: true }; break;
    default:
      throw new Error(`unknown command '${cmd}'`);
  }
  process.stdout.write(JSON.stringify(out));
}

main().catch((e) => {
  process.stderr.write(`${e.stack || e}\n`);
  process.exit(1);
});
