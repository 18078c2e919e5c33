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
//   lower            request {graph, fuse?: {keep, recompute?}, sources?} -> launch records
//   model-fusion     fusion summaries of the reference's transformer forward pass and Adam step
//   direct-catalogue the direct adversarial cases: names, kinds, patterns, and what fuse() makes of each
//   transformer-init the reference transformer (golden config) forward + gradient graph and its inputs
//   random-programs  request {programs: [{seed, focus?, f32?}]} -> the reference's v2 random programs
//   corpus-fusion    request {from, to, sabotageTo?} -> fusion counts over corpus programs
//   config-graphs    request {c3: [{fn, R, C}], c4: [{act, M, K, N}]} -> forward and gradient graphs of configs 3 and 4
//   step-graph       (bundle) request {model, V?, B?, seed?, firstBatch?, params64?}: a model's step graph, fused, with its inputs
//   forward-graph    (bundle) request {model, V?, B?, seed?, firstBatch?, params64?}: a model's forward pass, fused, with its inputs
// GPU commands write a bundle (manifest.json + data.f32) under --out:
//   gpu-direct       request {sabotage?}: every direct case, fused, canary-padded, on the GPU
//   gpu-graphs       request {graphs: [{name, graph, inputs, keep, unfused?, perf?}]} fused (and unfused, and in the perf lowering) on the GPU
//   gpu-fuzz         request {from, to, recompute?}: the reference's corpus programs, fused / perf / unfused, on the GPU
//   gpu-configs      request {c3: [...], c4: [...], unfused} configs 3 and 4, kept outputs as oracle-computable slices
//   gpu-workloads    request {ids?, families?, allNodes?}: the workload sweep's variants run once, outputs for the gate
//   gpu-bench-selftest  the timing protocol's counters: a clean timed region, a planted leak that must trip
//   gpu-step-slices  request {model, B, sequences}: a full-batch step's launches with their operands, as per-sequence blocks
//   gpu-local        request {model, forward?, valuesFile, sets?, sabotage?, perf?}: a fused step or forward pass run
//                    node-locally on the checker's reference operands, one case per value set
//   grouped-batches  request {model, B}: the batched kernels of a step's split-K products, with their text

const fs = require('fs');
const fs_ = fs;
const path = require('path');
const { Graph } = require('../src/ir/graph');
const { size } = require('../src/ir/shapes');
const { grad } = require('../src/autodiff');
const { fuse, fusionSummary } = require('../src/fusion/fuse');
const { lowerMI355X, kernelSources } = require('../src/mi355x/lower');
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

// Attention graphs of the GPU tests: [B, H, TQ, TK, DH, DV], options, and whether the
// attention kernel takes them (the last is past its key limit and stays three launches).
const ATTENTION_CASES = [
  { name: 'ragged', dims: [2, 3, 37, 45, 20, 12], scale: 0.2, mask: true, fuses: true },
  { name: 'per-element', dims: [1, 2, 19, 33, 18, 10], scale: 0.25, mask: true, fuses: true },
  { name: 'query-blocks', dims: [2, 2, 130, 256, 32, 32], scale: 0.18, fuses: true },
  { name: 'pre-transposed', dims: [2, 2, 64, 64, 32, 32], scale: 0.18, mask: true, kTransposed: true, vTransposed: true, fuses: true },
  { name: 'too-many-keys', dims: [1, 1, 8, 1024, 16, 16], scale: 0.25, fuses: false },
  // Two independent attentions of one shape: the perf lowering batches their kernels.
  { name: 'twin', dims: [2, 2, 48, 64, 32, 32], scale: 0.18, mask: true, twice: true, fuses: true },
];

/**
 * Scaled-dot-product attention graphs built with the IR builder:
 * o = softmax(q · kᵀ · scale + mask) · v, k (and v) optionally given already
 * transposed; inputs uniform in [-2, 2] from a seeded generator.
 */
function attentionGraphs(cases) {
  const { Rng } = require('../src/testing/rng');
  return cases.map((c) => {
    const g = new Graph();
    const [B, H, TQ, TK, DH, DV] = c.dims;
    const one = (sfx) => {
      const q = g.input(`q${sfx}`, [B, H, TQ, DH]);
      const kt = c.kTransposed ? g.input(`kt${sfx}`, [B, H, DH, TK]) : g.transpose(g.input(`k${sfx}`, [B, H, TK, DH]), [0, 1, 3, 2]);
      const v = c.vTransposed ? g.transpose(g.input(`vt${sfx}`, [B, H, DV, TK]), [0, 1, 3, 2]) : g.input(`v${sfx}`, [B, H, TK, DV]);
      let s = g.matmul(q, kt);
      if (c.scale) s = g.mul(s, g.const(c.scale));
      if (c.mask) {
        const m = [];
        for (let i = 0; i < TQ; i++) for (let j = 0; j < TK; j++) m.push(j > i + (TK - TQ) ? -1e4 : 0);
        s = g.add(s, g.const(m, [TQ, TK]));
      }
      return g.matmul(g.softmax(s, 3), v);
    };
    const keep = [one('')];
    if (c.twice) keep.push(one('2'));
    const rng = new Rng(c.seed || 7);
    const inputs = {};
    for (const n of g.inputs()) inputs[n.attrs.name] = rng.array(size(n.shape), -2, 2);
    return { name: c.name, fuses: c.fuses, graph: g.toJSON(), keep, inputs };
  });
}

/**
 * The transformer's forward graph (reference or config-5 structure) with its
 * parameters (initParams) and one batch of one-hot tokens and targets.
 */
function transformerForward(req) {
  const cfg = req.config === 'c5' ? tf.C5_CONFIG : tf.REFERENCE_CONFIG;
  const V = req.V || 16, B = req.B || 2;
  const fwd = tf.buildForward(V, B, cfg);
  const inputs = {};
  const init = tf.initParams(V, req.seed || 1, cfg);
  for (const k of Object.keys(init)) inputs[k] = Array.from(init[k]);
  const { Rng } = require('../src/testing/rng');
  const rng = new Rng(req.seed || 1);
  const rows = B * cfg.T;
  const onehot = () => { const a = new Array(rows * V).fill(0); for (let i = 0; i < rows; i++) a[i * V + rng.int(0, V - 1)] = 1; return a; };
  inputs.x = onehot();
  inputs.y = onehot();
  return { graph: fwd.graph.toJSON(), keep: [fwd.logits, fwd.loss], inputs };
}

/** Compile, offline, the kernels a named group of GPU runs will ask for (same module text as on the box). */
function precompileGroup(group, arch, shard, shards) {
  const { precompile } = require('../src/mi355x/runner');
  if (group === 'direct') {
    const fused = fusedDirectCases().map((c) => fuse(c.graph).graph);
    let n = precompile(fused.map((g) => lowerMI355X(g)), arch);
    for (const sabotage of KERNEL_SABOTAGES) n += precompile(fused.map((g) => lowerMI355X(g, { sabotage })), arch);
    return n;
  }
  if (group === 'models') {
    // The trainer compiles a step's kernels as one module: the same text here.
    const { modelStep } = require('../src/builders/models');
    const { fusedStep } = require('../src/mi355x/trainer');
    const reqs = [{ model: 'mlp' }, { model: 'transformer', B: 1 }, { model: 'transformer', B: 64 }, { model: 'transformer-ref' },
      { model: 'transformer', B: 1, attention: true }, { model: 'transformer', B: 64, attention: true }];
    let n = 0;
    for (const r of reqs) {
      const m = modelStep(r);
      const fs = fusedStep(m.step, { attention: !!r.attention });
      // The bench's unfused step runs in the perf lowering as well.
      const unfused = lowerMI355X(m.step.graph, { perf: true, keep: [m.step.loss, m.step.logits].concat(Object.values(m.step.outputs)), rowFolds: false });
      n += precompile([fs.lowered], arch) + precompile([fs.checked], arch) + precompile([unfused], arch);
    }
    return n;
  }
  if (group === 'golden') {
    // The reference transformer's model-level checks at its golden size (V 16, batch 4):
    // the forward pass fused (plain and perf lowerings), and the step and the forward pass
    // under each kernel sabotage (plain lowering). The honest step is the models group's.
    const { modelForward } = require('../src/builders/models');
    const { fusedForward } = require('../src/mi355x/trainer');
    const { modelStep } = require('../src/builders/models');
    const { fusedStep } = require('../src/mi355x/trainer');
    const req = { model: 'transformer-ref' };
    const ff = fusedForward(modelForward(req).fwd);
    let n = precompile([ff.checked], arch) + precompile([ff.lowered], arch);
    for (const sabotage of KERNEL_SABOTAGES) {
      n += precompile([fusedForward(modelForward(req).fwd, { sabotage, perf: false }).checked], arch);
      n += precompile([fusedStep(modelStep(req).step, { sabotage, perf: false }).checked], arch);
    }
    return n;
  }
  if (group === 'configs') {
    // Configs 2, 3 and 4 as the bench and the GPU tests run them: fused and unfused.
    const { chainWorkload } = require('../src/builders/chains');
    const cfg = require('../src/builders/configs');
    const lists = [];
    const both = (v) => {
      const f = fuse(v.graph, { keep: v.keep });
      const fk = v.keep.map((id) => f.index.get(id));
      lists.push(lowerMI355X(f.graph), lowerMI355X(v.graph), lowerMI355X(f.graph, { perf: true, keep: fk }), lowerMI355X(v.graph, { perf: true, keep: v.keep, rowFolds: false }));
    };
    for (const R of [8192, 64]) {
      for (let seed = 0; seed < 8; seed++) { const w = chainWorkload(seed, R, 1024); both(w.forward); both(w.gradient); }
    }
    for (const fn of ['softmax', 'logSoftmax']) { const g = cfg.c3Graphs(fn, cfg.C3_SHAPE[0], cfg.C3_SHAPE[1]); both(g.forward); both(g.gradient); }
    for (const [M, K, N] of cfg.C4_SHAPES) {
      for (const act of ['relu', 'tanh']) { const g = cfg.c4Graphs(act, M, K, N); both(g.forward); both(g.gradient); }
    }
    return precompile(lists, arch);
  }
  if (group === 'sweep') {
    // The workload sweep's variants as the bench lowers them.
    const { workloads } = require('../src/builders/workloads');
    const lists = [];
    for (const w of workloads()) {
      const m = w.make();
      for (const v of w.variants) {
        if (v === 'unfused') { lists.push(lowerMI355X(m.graph, { perf: true, keep: m.outputs, rowFolds: false })); continue; }
        const f = fuse(m.graph, { keep: m.outputs, recompute: v === 'recompute' });
        lists.push(lowerMI355X(f.graph, { perf: true, keep: m.outputs.map((id) => f.index.get(id)) }));
      }
    }
    return precompile(lists, arch);
  }
  if (group === 'attention') {
    // The attention GPU tests' graphs (fused with and without the extension, plain and
    // perf lowerings) and the bench's forward passes.
    const graphs = attentionGraphs(ATTENTION_CASES).map((c) => ({ graph: Graph.fromJSON(c.graph), keep: c.keep }));
    const att = builderCases().find((c) => c.name === 'attention');
    graphs.push({ graph: Graph.fromJSON(att.graph), keep: att.outputs });
    for (const [config, V, B] of [['reference', 16, 2], ['reference', 16, 16], ['c5', 96, 2], ['c5', 96, 64]]) {
      const fw = transformerForward({ config, V, B });
      graphs.push({ graph: Graph.fromJSON(fw.graph), keep: fw.keep });
    }
    const lists = [];
    for (const { graph, keep } of graphs) {
      for (const attention of [false, true]) {
        const f = fuse(graph, { keep, attention });
        lists.push(lowerMI355X(f.graph), lowerMI355X(f.graph, { perf: true, keep: keep.map((id) => f.index.get(id)) }));
      }
      lists.push(lowerMI355X(graph, { perf: true, keep, rowFolds: false }));
    }
    return precompile(lists, arch);
  }
  if (group === 'scratch') {
    // The no-allocation entry point's GPU test: split-K matmuls, one translation unit.
    return precompile(scratchLowerings(SCRATCH_SHAPES), arch);
  }
  if (group === 'recompute') {
    // The recompute GPU tests: corpus programs 1..100 fused with recomputation (plain and
    // perf lowerings), and the fusion-loses workloads' fused and recompute variants in the
    // plain lowering (their perf lowerings are the sweep group's).
    const { corpusGraphs } = require('../src/testing/random_graph');
    const { workloads } = require('../src/builders/workloads');
    const lists = [];
    for (let i = 1; i <= 100; i++) {
      for (const c of corpusGraphs(i)) {
        const f = fuse(c.graph, { keep: c.keep, recompute: true });
        lists.push(lowerMI355X(f.graph), lowerMI355X(f.graph, { perf: true, keep: c.keep.map((id) => f.index.get(id)), absorb: true }));
      }
    }
    for (const w of workloads().filter((x) => x.variants.includes('recompute'))) {
      const m = w.make();
      for (const recompute of [false, true]) lists.push(lowerMI355X(fuse(m.graph, { keep: m.outputs, recompute }).graph));
    }
    return precompile(lists, arch);
  }
  if (group === 'fuzz') {
    // The GPU fuzzer's kernels (corpus programs 1..2000, fused and unfused), in
    // `shards` disjoint parts by kernel name so several processes can compile them.
    const { corpusGraphs } = require('../src/testing/random_graph');
    const { fnv } = require('../src/mi355x/codegen');
    const lists = [];
    for (let i = 1; i <= 2000; i++) {
      for (const c of corpusGraphs(i)) {
        const f = fuse(c.graph, { keep: c.keep });
        lists.push(lowerMI355X(f.graph), lowerMI355X(f.graph, { perf: true, keep: c.keep.map((id) => f.index.get(id)), absorb: true }), lowerMI355X(c.graph));
      }
    }
    const k = shards || 1, me = shard || 0;
    return precompile(lists, arch, (name) => parseInt(fnv(name), 16) % k === me);
  }
  throw new Error(`unknown precompile group '${group}'`);
}

/** Products whose K is split across workgroups (a workspace of partial sums): the scratch test's. */
const SCRATCH_SHAPES = [[256, 4096, 256], [128, 2048, 128]];

/** The plain lowering of matmul(x[M,K], w[K,N]) for each shape. */
function scratchLowerings(shapes) {
  return shapes.map(([M, K, N]) => {
    const g = new Graph();
    g.matmul(g.input('x', [M, K]), g.input('w', [K, N]));
    return lowerMI355X(g);
  });
}

/** The load modes (A, B) of a matmul launch's kernel, or null. */
function gemmModes(l) {
  // gemm_f32<TM, TN, BK, PF, AMODE, BMODE, SPLIT, ...>
  const m = l.kernels[0].source.match(/gemm_f32<([^>]*)>/);
  if (!m) return null;
  const a = m[1].split(',').map((x) => x.trim());
  return [Number(a[4]), Number(a[5])];
}

/** The K split (chunks, chunk length) of a matmul launch's kernel, or null. */
function gemmSplit(l) {
  // gemm_f32<...>(A, a, b, batch, M, K, N, chunks, chunkK, zid, tx, ty): the place is
  // (blockIdx.z, blockIdx.x, blockIdx.y), or (wg.z, wg.x, wg.y) where the tiles take
  // XCD-grouped places.
  const m = l.kernels[0].source.match(/(\d+)u, (\d+)u, (?:blockIdx\.z, blockIdx\.x, blockIdx\.y|wg\.z, wg\.x, wg\.y)\);/);
  return l.flops && m ? [Number(m[1]), Number(m[2])] : null;
}

/** The reference's four kernel sabotages (codegen-fused.js:22), as lowerMI355X applies them. */
const KERNEL_SABOTAGES = ['epilogue-before-bias', 'layernorm-tree-short', 'softmax-no-max', 'fused-bounds-off-by-one'];

async function gpuDirect(dir, req) {
  const { HipRunner } = require('../src/mi355x/runner');
  const sabotage = (req && req.sabotage) || undefined;
  if (sabotage && !KERNEL_SABOTAGES.includes(sabotage)) throw new Error(`unknown kernel sabotage '${sabotage}'`);
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  const cases = fusedDirectCases();
  const plans = cases.map((c) => { const f = fuse(c.graph); return { f, lowered: lowerMI355X(f.graph, { sabotage }) }; });
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
  bundle.close({ device: runner.info(), sabotage: sabotage || null });
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
    const f = fuse(g, { keep: c.keep || [], attention: !!c.attention });
    const lf = lowerMI355X(f.graph);
    const rf = await runner.run(f.graph, lf, inputs, { canary: true });
    const entry = { name: c.name, fused: f.graph.toJSON(), origin: f.origin, gpuFused: {}, canaryFused: rf.canaryIntact,
      kinds: lf.launches.map((l) => l.kind) };
    f.graph.nodes.forEach((n) => { entry.gpuFused[n.id] = bundle.put(rf.values[n.id]); });
    if (c.perf) {
      // The perf lowering: transposes read in place by the matmuls, reshapes sharing buffers.
      const keepF = (c.keep || []).map((id) => f.index.get(id));
      const lp = lowerMI355X(f.graph, { perf: true, keep: keepF });
      const rp = await runner.run(f.graph, lp, inputs, { canary: true });
      entry.gpuPerf = {};
      for (const id of keepF) entry.gpuPerf[id] = bundle.put(rp.values[id]);
      entry.perfFolded = lp.folded;
      entry.perfModes = lp.launches.filter((l) => l.flops && l.kind !== 'fused-attention').map(gemmModes);
      entry.perfViews = lp.launches.filter((l) => l.kind === 'fused-attention').map((l) => Object.keys(l.views || {}).sort());
      entry.perfBatches = (lp.batches || []).map((x) => ({ count: x.count, kind: lp.launches[x.start].kind, kernels: x.kernels.map((k) => k.name) }));
      entry.canaryPerf = rp.canaryIntact.every(Boolean);
    }
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

/** Sorted unique indices in [0, n): the two first and two last, `must`, and random ones up to `count` in all. */
function sampleIndices(n, must, count, seed) {
  const { Rng } = require('../src/testing/rng');
  const set = new Set([0, 1, n - 2, n - 1].filter((i) => i >= 0 && i < n).concat(must || []));
  const rng = new Rng(seed >>> 0);
  while (set.size < Math.min(count, n)) set.add(rng.int(0, n - 1));
  return Array.from(set).sort((a, b) => a - b);
}

function takeRows(a, C, rows) {
  const out = new Float32Array(rows.length * C);
  rows.forEach((r, k) => out.set(a.subarray(r * C, (r + 1) * C), k * C));
  return out;
}

function takeCols(a, R, C, cols) {
  const out = new Float32Array(R * cols.length);
  for (let r = 0; r < R; r++) for (let k = 0; k < cols.length; k++) out[r * cols.length + k] = a[r * C + cols[k]];
  return out;
}

/** The two graphs have the same nodes (op, inputs, attrs other than shapes) in the same order. */
function sameStructure(a, b) {
  if (a.nodes.length !== b.nodes.length) return false;
  return a.nodes.every((n, i) => n.op === b.nodes[i].op && n.inputs.join() === b.nodes[i].inputs.join());
}

/** Full-tensor properties of one kept output: non-finite counts and fused/unfused bitwise agreement. */
function tensorProps(f, u) {
  let nfF = 0, nfU = 0, same = 0;
  for (let i = 0; i < f.length; i++) if (!Number.isFinite(f[i])) nfF++;
  if (u) {
    const fb = new Uint32Array(f.buffer, f.byteOffset, f.length), ub = new Uint32Array(u.buffer, u.byteOffset, u.length);
    for (let i = 0; i < u.length; i++) { if (!Number.isFinite(u[i])) nfU++; if (fb[i] === ub[i]) same++; }
  }
  return { n: f.length, nonfiniteFused: nfF, nonfiniteUnfused: u ? nfU : null, bitwiseSame: u ? same : null };
}

/** Fused (and unfused) run of `graph` with canaries; the kept outputs of each, by kept position. */
async function runVariants(runner, graph, keep, inputs, unfused) {
  const f = fuse(graph, { keep });
  const lf = lowerMI355X(f.graph);
  let r = await runner.run(f.graph, lf, inputs, { canary: true });
  const out = { fused: keep.map((id) => r.values[f.index.get(id)]), canaryFused: r.canaryIntact.every(Boolean),
    fusedKinds: lf.launches.map((l) => l.kind), unfused: null, canaryUnfused: null, unfusedLaunches: null };
  r = null;
  // The perf lowering of the fused graph (transposes read in place, reshapes sharing
  // buffers): its kept outputs must equal the plain lowering's bit for bit.
  const lp = lowerMI355X(f.graph, { perf: true, keep: keep.map((id) => f.index.get(id)) });
  const rp = await runner.run(f.graph, lp, inputs, { canary: true });
  let perfSame = 0, perfTotal = 0;
  keep.forEach((id, k) => {
    const a = new Uint32Array(rp.values[f.index.get(id)].buffer), b = new Uint32Array(out.fused[k].buffer);
    perfTotal += a.length;
    for (let i = 0; i < a.length; i++) if (a[i] === b[i]) perfSame++;
  });
  Object.assign(out, { perfSame, perfTotal, perfLaunches: lp.launches.length, perfFolded: lp.folded.length,
    canaryPerf: rp.canaryIntact.every(Boolean) });
  if (unfused) {
    const lu = lowerMI355X(graph);
    const ru = await runner.run(graph, lu, inputs, { canary: true });
    out.unfused = keep.map((id) => ru.values[id]);
    out.canaryUnfused = ru.canaryIntact.every(Boolean);
    out.unfusedLaunches = lu.launches.length;
  }
  return out;
}

/**
 * Configs 3 and 4 on the GPU at the requested sizes, fused and unfused, with
 * canaries. Every kept output is returned through slices the oracle can compute
 * exactly: whole rows (config 3; config 4's y and dX) and whole columns
 * (config 4's y, dW and dbias), each with the graph the same builder makes at
 * the slice's size and the inputs restricted to it (rows of a row-wise softmax
 * depend only on their own inputs; row i of X·W on row i of X; column j of
 * X·W, of dW = Xᵀ·dZ and of dbias on column j of W, bias and dY). Full-tensor
 * properties over every element are computed here: non-finite counts,
 * fused/unfused bitwise agreement, the row sums of softmax and the row
 * log-sum-exp of logSoftmax.
 * Request: { c3: [{fn, R, C, rows}], c4: [{act, M, K, N, rows, cols}], unfused }.
 */
async function gpuConfigs(req, dir) {
  const cfg = require('../src/builders/configs');
  const { HipRunner } = require('../src/mi355x/runner');
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  for (const c of req.c3 || []) {
    const { R, C } = c;
    const ins = cfg.c3Inputs(R, C);
    const rows = c.rows === 'all' ? Array.from({ length: R }, (_, i) => i) : sampleIndices(R, ins.shifted, ins.shifted.length + c.rows, 31);
    const full = cfg.c3Graphs(c.fn, R, C), sub = cfg.c3Graphs(c.fn, rows.length, C);
    for (const kind of ['forward', 'gradient']) {
      const v = full[kind], s = sub[kind];
      if (!sameStructure(v.graph, s.graph)) throw new Error('config 3 sub-graph differs in structure');
      process.stderr.write(`gpu-configs: c3 ${c.fn} ${kind} [${R},${C}], ${rows.length} rows sampled\n`);
      const inputs = kind === 'forward' ? { x: ins.x } : { x: ins.x, d0: ins.dy };
      const r = await runVariants(runner, v.graph, v.keep, inputs, req.unfused);
      const props = v.keep.map((id, k) => tensorProps(r.fused[k], r.unfused && r.unfused[k]));
      // Row property of y over every row: sum of softmax = 1, log-sum-exp of logSoftmax = 0.
      const y = r.fused[0];
      let worstRow = 0;
      for (let row = 0; row < R; row++) {
        let acc = 0;
        for (let col = 0; col < C; col++) acc += c.fn === 'softmax' ? y[row * C + col] : Math.exp(y[row * C + col]);
        const dev = c.fn === 'softmax' ? Math.abs(acc - 1) : Math.abs(Math.log(acc));
        if (!(dev <= worstRow)) worstRow = dev;
      }
      const subInputs = {};
      for (const name of Object.keys(inputs)) subInputs[name] = bundle.put(takeRows(inputs[name], C, rows));
      const compare = v.keep.map((id, k) => ({ id, fused: bundle.put(takeRows(r.fused[k], C, rows)),
        unfused: r.unfused ? bundle.put(takeRows(r.unfused[k], C, rows)) : null }));
      bundle.add({ name: `c3-${c.fn}-${kind}-${R}x${C}`, config: 'c3', fn: c.fn, kind, shape: [R, C], rows: rows.length,
        shifted: ins.shifted.length, sample: { graph: s.graph.toJSON(), inputs: subInputs, compare },
        props, rowProperty: worstRow, canaryFused: r.canaryFused, canaryUnfused: r.canaryUnfused, fusedKinds: r.fusedKinds,
        unfusedLaunches: r.unfusedLaunches, perf: { same: r.perfSame, total: r.perfTotal, launches: r.perfLaunches, folded: r.perfFolded, canary: r.canaryPerf } });
    }
  }
  for (const c of req.c4 || []) {
    const { M, K, N } = c;
    const ins = cfg.c4Inputs(M, K, N);
    const all = c.rows === 'all';
    const rows = all ? Array.from({ length: M }, (_, i) => i) : sampleIndices(M, [], c.rows, 41);
    const cols = all ? [] : sampleIndices(N, [], c.cols, 43);
    const full = cfg.c4Graphs(c.act, M, K, N);
    const byRows = cfg.c4Graphs(c.act, rows.length, K, N);
    const byCols = all ? null : cfg.c4Graphs(c.act, M, K, cols.length);
    for (const kind of ['forward', 'gradient']) {
      const v = full[kind];
      if (!sameStructure(v.graph, byRows[kind].graph) || (byCols && !sameStructure(v.graph, byCols[kind].graph))) {
        throw new Error('config 4 sub-graph differs in structure');
      }
      process.stderr.write(`gpu-configs: c4 ${c.act} ${kind} ${M}x${K}x${N}, ${all ? 'all' : rows.length} rows, ${cols.length} cols sampled\n`);
      const inputs = kind === 'forward' ? { X: ins.X, W: ins.W, bias: ins.bias } : { X: ins.X, W: ins.W, bias: ins.bias, d0: ins.dY };
      const r = await runVariants(runner, v.graph, v.keep, inputs, req.unfused);
      const props = v.keep.map((id, k) => tensorProps(r.fused[k], r.unfused && r.unfused[k]));
      let outOfRange = 0;
      for (const t of [r.fused[0]].concat(r.unfused ? [r.unfused[0]] : [])) {
        for (let i = 0; i < t.length; i++) if (c.act === 'relu' ? !(t[i] >= 0) : !(Math.abs(t[i]) <= 1)) outOfRange++;
      }
      const samples = [];
      // Row slice: y and dX (kept as [y, dX, dW, dbias]); everything when all rows are taken.
      {
        const shapes = v.keep.map((id) => v.graph.nodes[id].shape);
        const take = (a, shape) => takeRows(a, shape[shape.length - 1], rows);
        const sel = all ? v.keep.map((id, k) => k) : (kind === 'forward' ? [0] : [0, 1]);
        const subInputs = { X: bundle.put(takeRows(ins.X, K, rows)), W: bundle.put(ins.W), bias: bundle.put(ins.bias) };
        if (kind === 'gradient') subInputs.d0 = bundle.put(takeRows(ins.dY, N, rows));
        samples.push({ slice: 'rows', n: rows.length, graph: byRows[kind].graph.toJSON(), inputs: subInputs,
          compare: sel.map((k) => ({ id: v.keep[k], fused: bundle.put(all ? r.fused[k] : take(r.fused[k], shapes[k])),
            unfused: r.unfused ? bundle.put(all ? r.unfused[k] : take(r.unfused[k], shapes[k])) : null })) });
      }
      // Column slice: y, dW and dbias.
      if (!all) {
        const shapes = v.keep.map((id) => v.graph.nodes[id].shape);
        const take = (a, shape) => (shape.length === 1 ? Float32Array.from(cols.map((j) => a[j])) : takeCols(a, shape[0], N, cols));
        const sel = kind === 'forward' ? [0] : [0, 2, 3];
        const subInputs = { X: bundle.put(ins.X), W: bundle.put(takeCols(ins.W, K, N, cols)), bias: bundle.put(Float32Array.from(cols.map((j) => ins.bias[j]))) };
        if (kind === 'gradient') subInputs.d0 = bundle.put(takeCols(ins.dY, M, N, cols));
        samples.push({ slice: 'cols', n: cols.length, graph: byCols[kind].graph.toJSON(), inputs: subInputs,
          compare: sel.map((k) => ({ id: v.keep[k], fused: bundle.put(take(r.fused[k], shapes[k])),
            unfused: r.unfused ? bundle.put(take(r.unfused[k], shapes[k])) : null })) });
      }
      bundle.add({ name: `c4-${c.act}-${kind}-${M}x${K}x${N}`, config: 'c4', act: c.act, kind, shape: [M, K, N],
        samples, props, outOfRange, canaryFused: r.canaryFused, canaryUnfused: r.canaryUnfused, fusedKinds: r.fusedKinds,
        unfusedLaunches: r.unfusedLaunches, perf: { same: r.perfSame, total: r.perfTotal, launches: r.perfLaunches, folded: r.perfFolded, canary: r.canaryPerf } });
    }
  }
  bundle.close({ device: runner.info() });
}

/**
 * The reference's GPU fuzzer over its corpus (src/gpu/harness-m4.js:126-172): for
 * corpus programs [from, to], the program and its gradient graph, each fused
 * (plain lowering), fused in the perf lowering, and unfused, on the GPU with
 * canaries. The bundle holds each graph, its fused graph and origin map, the
 * inputs, and every node's GPU value of each variant (the perf variant's kept
 * outputs only) for the checker.
 */
async function gpuFuzz(req, dir) {
  const { corpusGraphs } = require('../src/testing/random_graph');
  const { HipRunner } = require('../src/mi355x/runner');
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  for (let i = req.from; i <= req.to; i++) {
    for (const c of corpusGraphs(i)) {
      const inputs = {}, ins = {};
      for (const name of Object.keys(c.inputs)) { inputs[name] = Float32Array.from(c.inputs[name]); ins[name] = bundle.put(inputs[name]); }
      const f = fuse(c.graph, { keep: c.keep, recompute: !!req.recompute });
      const keepF = c.keep.map((id) => f.index.get(id));
      const rf = await runner.run(f.graph, lowerMI355X(f.graph), inputs, { canary: true });
      const rp = await runner.run(f.graph, lowerMI355X(f.graph, { perf: true, keep: keepF, absorb: true }), inputs, { canary: true });
      const ru = await runner.run(c.graph, lowerMI355X(c.graph), inputs, { canary: true });
      const entry = { program: i, label: c.label, graph: c.graph.toJSON(), fused: f.graph.toJSON(), origin: f.origin, keep: c.keep,
        inputs: ins, gpuFused: {}, gpuUnfused: {}, gpuPerf: {},
        canary: rf.canaryIntact.every(Boolean) && rp.canaryIntact.every(Boolean) && ru.canaryIntact.every(Boolean) };
      f.graph.nodes.forEach((n) => { entry.gpuFused[n.id] = bundle.put(rf.values[n.id]); });
      c.graph.nodes.forEach((n) => { entry.gpuUnfused[n.id] = bundle.put(ru.values[n.id]); });
      for (const id of keepF) entry.gpuPerf[id] = bundle.put(rp.values[id]);
      bundle.add(entry);
    }
    if (i % 100 === 0) process.stderr.write(`gpu-fuzz: program ${i}\n`);
  }
  bundle.close({ device: runner.info(), from: req.from, to: req.to, recompute: !!req.recompute });
}

/**
 * The reference's workload sweep (src/fusion/workloads.js:71-120) run once on the GPU
 * in the lowerings the bench times, for the checker (workloads.js:351-374: every
 * variant's outputs against the streamed float64 reference before it may be timed).
 * Per workload: the graph, its inputs, and per variant (unfused, fused, recompute; the
 * step's matmul-only variant is the fused variant's matmul launches and has no outputs
 * of its own) the kept outputs and the canary verdict. With `allNodes`, the fused and
 * recompute variants are also run in the plain lowering with every surviving node
 * returned, with the fused graph and its origin map (judgeFused, harness-m4.js:46-60).
 * Request: { ids?: [workload id...] (default all), families?: [...], allNodes? }.
 */
async function gpuWorkloads(req, dir) {
  const { workloads } = require('../src/builders/workloads');
  const { HipRunner } = require('../src/mi355x/runner');
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  const want = (w) => (!req.ids || req.ids.includes(w.id)) && (!req.families || req.families.includes(w.family));
  for (const w of workloads().filter(want)) {
    process.stderr.write(`gpu-workloads: ${w.id}\n`);
    const m = w.make();
    const ins = {};
    for (const k of Object.keys(m.inputs)) ins[k] = bundle.put(m.inputs[k]);
    const entry = { id: w.id, family: w.family, params: w.params, judge: w.judge, graph: m.graph.toJSON(), outputs: m.outputs,
      inputs: ins, variants: {} };
    for (const v of w.variants.filter((x) => x !== 'matmul-only')) {
      let graph = m.graph, keep = m.outputs, f = null;
      if (v !== 'unfused') {
        f = fuse(m.graph, { keep: m.outputs, recompute: v === 'recompute' });
        graph = f.graph;
        keep = m.outputs.map((id) => f.index.get(id));
      }
      // As the bench lowers each variant: the unfused graph with nothing folded into another launch.
      const lp = lowerMI355X(graph, Object.assign({ perf: true, keep }, v === 'unfused' ? { rowFolds: false } : {}));
      const r = await runner.run(graph, lp, m.inputs, { canary: true });
      const out = { outputs: keep.map((id) => bundle.put(r.values[id])), canary: r.canaryIntact.every(Boolean),
        launches: lp.launches.length, kinds: lp.launches.map((l) => l.kind) };
      if (req.allNodes && f) {
        const lf = lowerMI355X(graph);
        const rf = await runner.run(graph, lf, m.inputs, { canary: true });
        out.fused = graph.toJSON();
        out.origin = f.origin;
        out.nodes = graph.nodes.map((n) => bundle.put(rf.values[n.id]));
        out.canaryPlain = rf.canaryIntact.every(Boolean);
        out.plainLaunches = lf.launches.length;
      }
      entry.variants[v] = out;
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
      if (req.perf) {
        // The lowerings the bench times: broadcasts read in place by their consumers,
        // dead launches dropped; the kernel names are the ones a profile of the bench shows.
        const fk = v.keep.map((id) => f.index.get(id));
        for (const [key, g, keep] of [['fusedPerf', f.graph, fk], ['unfusedPerf', v.graph, v.keep]]) {
          const lp = lowerMI355X(g, { perf: true, keep });
          const rp = await runner.run(g, lp, inputs, { canary: true });
          entry[key] = {};
          v.keep.forEach((id, k) => { entry[key][id] = bundle.put(rp.values[keep[k]]); });
          entry[`${key}Canary`] = rp.canaryIntact.every(Boolean);
          entry[`${key}Kernels`] = [].concat(...lp.launches.map((l) => l.kernels.map((x) => x.name)));
        }
      }
      bundle.add(entry);
    }
  }
  bundle.close({ device: runner.info() });
}

/** Plain arrays of a name -> values map, at full (float64) precision, for a JSON manifest. */
const plainArrays = (m) => { const r = {}; for (const k of Object.keys(m)) r[k] = Array.from(m[k]); return r; };

/**
 * The step graph of a model request as a bundle: the original and fused graphs,
 * the origin map, the ids that matter, and the step's inputs (parameters, state,
 * batch k, cotangent 1) as float32 arrays. With `params64`, the initial parameters
 * and state also as float64 numbers in the manifest (a float64 trajectory starts
 * from them, as the reference's trainCpu3b does). No GPU.
 */
function stepGraph(req, dir) {
  const { modelStep } = require('../src/builders/models');
  const { fusedStep } = require('../src/mi355x/trainer');
  const m = modelStep(req);
  const fs = fusedStep(m.step, { attention: !!req.attention });
  const bundle = new Bundle(dir);
  const b = m.batch(req.batchIndex || 0);
  const values = Object.assign({}, m.params, m.state, { x: b.x, y: b.y });
  values[m.step.cotangent] = [1];
  const inputs = {};
  for (const k of Object.keys(values)) inputs[k] = bundle.put(values[k]);
  const entry = { name: req.model, graph: m.step.graph.toJSON(), fused: fs.graph.toJSON(), origin: fs.fusion.origin, inputs,
    loss: m.step.loss, logits: m.step.logits, outputs: m.step.outputs, stepInputs: m.step.inputs, names: m.step.names,
    stateNames: m.step.stateNames || [], cotangent: m.step.cotangent,
    launchesFused: fs.lowered.launches.length, launchesChecked: fs.checked.launches.length,
    launchesUnfused: lowerMI355X(m.step.graph).launches.length, info: m.info };
  if (req.params64) Object.assign(entry, { params64: plainArrays(m.params), state64: plainArrays(m.state) });
  bundle.add(entry);
  bundle.close();
}

/**
 * The forward pass of a model request (the transformer's logits and loss) as a bundle,
 * like step-graph: original and fused graphs (fused keeping the logits and the loss, as
 * src/gpu/harness-m4.js:281 does), the origin map, and the inputs (parameters, batch k) as
 * float32 arrays; with `params64`, the parameters as float64 numbers too. No GPU.
 */
function forwardGraph(req, dir) {
  const { modelForward } = require('../src/builders/models');
  const { fusedForward } = require('../src/mi355x/trainer');
  const m = modelForward(req);
  const ff = fusedForward(m.fwd);
  const bundle = new Bundle(dir);
  const b = m.batch(req.batchIndex || 0);
  const values = Object.assign({}, m.params, { x: b.x, y: b.y });
  const inputs = {};
  for (const k of Object.keys(values)) inputs[k] = bundle.put(values[k]);
  const entry = { name: req.model, graph: m.fwd.graph.toJSON(), fused: ff.graph.toJSON(), origin: ff.fusion.origin, inputs,
    loss: m.fwd.loss, logits: m.fwd.logits, launchesFused: ff.lowered.launches.length, launchesChecked: ff.checked.launches.length,
    launchesUnfused: lowerMI355X(m.fwd.graph).launches.length, info: m.info };
  if (req.params64) entry.params64 = plainArrays(m.params);
  bundle.add(entry);
  bundle.close();
}

/**
 * Node-local run of a model's fused step (or, with `forward`, of its fused forward pass):
 * every launch reads the float32 reference operands given in `valuesFile` (all fused-graph
 * nodes, in node order, as the checker computed them) and writes its own output (with
 * canaries). The file may hold `sets` such value sets back to back (the teacher-forced
 * check's steps, src/gpu/harness-m4.js:225-272): each is run as its own case, in order.
 * `sabotage` plants one of the reference's kernel sabotages in both lowerings;
 * `perf: false` runs the checked lowering alone.
 */
async function gpuLocal(req, dir) {
  const { modelStep, modelForward } = require('../src/builders/models');
  const { fusedStep, fusedForward } = require('../src/mi355x/trainer');
  const { HipRunner } = require('../src/mi355x/runner');
  const fs = req.forward ? fusedForward(modelForward(req).fwd, { sabotage: req.sabotage })
    : fusedStep(modelStep(req).step, { sabotage: req.sabotage, attention: !!req.attention });
  const raw = fs_.readFileSync(req.valuesFile);
  const data = new Float32Array(raw.buffer, raw.byteOffset, raw.byteLength / 4);
  const sets = req.sets || 1;
  const per = fs.graph.nodes.reduce((c, node) => c + node.shape.reduce((a, d) => a * d, 1), 0);
  if (per * sets !== data.length) throw new Error(`values file holds ${data.length} floats, ${sets} value sets of the fused graph need ${per * sets}`);
  const runner = HipRunner.create();
  const bundle = new Bundle(dir);
  const lowerings = req.perf === false ? [['gpu', fs.checked]] : [['gpu', fs.checked], ['gpuPerf', fs.lowered]];
  for (let s = 0; s < sets; s++) {
    const values = [];
    let off = s * per;
    for (const node of fs.graph.nodes) {
      const n = node.shape.reduce((a, c) => a * c, 1);
      values.push(data.subarray(off, off + n));
      off += n;
    }
    // The checked lowering (every node launched) and the trainer's perf lowering.
    const entry = { name: req.model, set: s };
    for (const [key, lowered] of lowerings) {
      const out = await runner.runLocal(fs.graph, lowered, values, { canary: true });
      entry[key] = {};
      for (const l of lowered.launches) entry[key][l.node] = bundle.put(out[l.node]);
      entry[`${key}Canary`] = lowered.launches.every((l) => out.canaryIntact[l.node]);
      entry[`${key}Launches`] = lowered.launches.length;
    }
    entry.canaryIntact = lowerings.every(([key]) => entry[`${key}Canary`]);
    entry.rowFolds = rowFoldsOf(fs.lowered);
    entry.formed = formedOf(fs.lowered);
    entry.absorbed = absorbedOf(fs.lowered);
    entry.loadOps = loadOpsOf(fs.lowered);
    entry.aliases = fs.lowered.aliases;
    entry.folded = fs.lowered.folded;
    entry.dead = fs.lowered.dead;
    bundle.add(entry);
    if (sets > 1) process.stderr.write(`gpu-local: ${req.model}${req.forward ? ' forward' : ''} set ${s + 1}/${sets}\n`);
  }
  bundle.close({ device: runner.info() });
}

/**
 * Train a model for `steps` steps on the GPU with the fused trainer; with
 * `consistency`, also run the first steps through runner.run on the same fused
 * graph and compare loss and parameters bit for bit (the trainer's feedback
 * against the checked path, harness-m4.js:310-330).
 */
/**
 * Config 2's programs (seeds 0..P-1, forward and gradient, perf lowering) run one after
 * another on one stream, then, with every kept output a launch writes overwritten
 * first, as one concurrent group over each of `streams`: the outputs must be the same
 * bits.
 */
async function gpuConcurrent(req) {
  const { HipRunner, Concurrent, CANARY_BITS } = require('../src/mi355x/runner');
  const { chainWorkload, chainInputs } = require('../src/builders/chains');
  const runner = HipRunner.create();
  const programs = [], kept = [];
  for (let seed = 0; seed < req.programs; seed++) {
    const w = chainWorkload(seed, req.R, req.C);
    const inputs = chainInputs(seed, req.R, req.C);
    for (const kind of ['forward', 'gradient']) {
      const v = w[kind];
      const f = fuse(v.graph, { keep: v.keep });
      const keep = v.keep.map((id) => f.index.get(id));
      const p = runner.prepare(f.graph, lowerMI355X(f.graph, { perf: true, keep }));
      for (const n of f.graph.nodes) if (n.op === 'input') p.write(n.id, inputs[n.attrs.name]);
      programs.push(p);
      kept.push(keep);
    }
  }
  const readAll = () => programs.map((p, i) => kept[i].map((id) => p.read(id)));
  for (const p of programs) p.run();
  runner.a.sync();
  const want = readAll();
  const out = { programs: programs.length, streams: {} };
  for (const S of req.streams) {
    // Overwrite every kept output a launch writes (kept constants stay: no launch writes them).
    programs.forEach((p, i) => {
      const written = new Set(p.launches.map((l) => l.node));
      for (const id of kept[i]) if (written.has(id)) runner.a.fill32(p.bufs[id], 0, CANARY_BITS, p.n[id]);
    });
    const g = new Concurrent(runner, programs, S);
    g.run();
    runner.a.sync();
    const got = readAll();
    let same = 0, total = 0;
    got.forEach((outs, i) => outs.forEach((a, k) => {
      const x = new Uint32Array(a.buffer), y = new Uint32Array(want[i][k].buffer);
      total += x.length;
      for (let q = 0; q < x.length; q++) if (x[q] === y[q]) same++;
    }));
    out.streams[S] = { same, total, load: g.load };
  }
  for (const p of programs) p.destroy();
  return out;
}

/**
 * The batch axis of a node: the one dimension where its shape at the full batch differs
 * from its shape in the one-sequence twin graph (the same builder at B = 1), or -1 for
 * a node whose shape does not depend on the batch (parameters, their gradients and
 * updates, the loss).
 */
function batchAxis(full, twin) {
  const diff = [];
  for (let d = 0; d < full.length; d++) if (full[d] !== twin[d]) diff.push(d);
  if (full.length !== twin.length || diff.length > 1) throw new Error(`shapes ${full} / ${twin}: not one batch axis`);
  return diff.length ? diff[0] : -1;
}

/** Block `b` (of size twin[p]) along axis p of a row-major array of shape `shape`. */
function takeBlock(a, shape, p, q, b) {
  let outer = 1, inner = 1;
  for (let d = 0; d < p; d++) outer *= shape[d];
  for (let d = p + 1; d < shape.length; d++) inner *= shape[d];
  const span = q * inner, slab = shape[p] * inner;
  const out = new Float32Array(outer * span);
  for (let o = 0; o < outer; o++) out.set(a.subarray(o * slab + b * span, o * slab + (b + 1) * span), o * span);
  return out;
}

/**
 * A training step at its full batch, judged node-locally on the GPU's own operands
 * (the check of harness-m4.js:182-223 with every launch's operands taken from one
 * run of the checked lowering instead of the float64 reference, so that no full-size
 * float64 evaluation of the step is needed). The checked lowering (one launch per
 * node) runs once with canaries and every node is read back; the trainer's perf
 * lowering (split-K weight gradients, batched dispatches, read-in-place transposes)
 * then runs node-locally on those values. The bundle holds, for the checker:
 *  - per launched node whose shape carries the batch: its block for each sampled
 *    sequence, and the same blocks of its operands (a sequence's rows depend only on
 *    that sequence's operand rows and on the parameters);
 *  - per launched node whose shape does not (weight and bias gradients and their SGD
 *    updates, the loss): its whole value and its operands' whole values;
 *  - the fused graph at the full batch and its one-sequence twin (shapes of a block).
 * Request: { model, B, sequences: [b...], batchIndex? }.
 */
async function gpuStepSlices(req, dir) {
  const { modelStep } = require('../src/builders/models');
  const { fusedStep } = require('../src/mi355x/trainer');
  const { HipRunner } = require('../src/mi355x/runner');
  const m = modelStep(req);
  const fs = fusedStep(m.step, { attention: !!req.attention });
  const twin = fusedStep(modelStep(Object.assign({}, req, { B: 1 })).step, { attention: !!req.attention });
  if (!sameStructure(fs.graph, twin.graph)) throw new Error('the one-sequence twin differs in structure');
  const nodes = fs.graph.nodes;
  const axis = nodes.map((n, i) => batchAxis(n.shape, twin.graph.nodes[i].shape));
  const B = req.B;
  const seqs = req.sequences;
  for (const b of seqs) if (!(b >= 0 && b < B)) throw new Error(`sequence ${b} outside the batch`);
  const runner = HipRunner.create();
  const batch = m.batch(req.batchIndex || 0);
  const feed = Object.assign({}, m.params, m.state, { x: batch.x, y: batch.y });
  feed[fs.cotangent] = [1];
  process.stderr.write(`gpu-step-slices: checked lowering, ${fs.checked.launches.length} launches, every node read back\n`);
  const r = await runner.run(fs.graph, fs.checked, feed, { canary: true });
  process.stderr.write(`gpu-step-slices: perf lowering node-local, ${fs.lowered.launches.length} launches\n`);
  const perf = await runner.runLocal(fs.graph, fs.lowered, r.values, { canary: true });
  const bundle = new Bundle(dir);
  // What each launched node needs: blocks (batch-carrying output) or whole values.
  const wantBlocks = new Set(), wantWhole = new Set();
  const launched = fs.checked.launches.map((l) => l.node);
  const need = (id, ins) => {
    if (axis[id] >= 0) {
      wantBlocks.add(id);
      for (const i of ins) (axis[i] >= 0 ? wantBlocks : wantWhole).add(i);
    } else {
      wantWhole.add(id);
      for (const i of ins) wantWhole.add(i);
    }
  };
  for (const id of launched) need(id, nodes[id].inputs);
  // A perf launch that forms values in place (absorbed producers, row folds) is judged on
  // the operands of what it forms: a column sum that forms its operand is judged whole on
  // that producer's operands whole, though the producer's own launch takes their blocks.
  for (const l of fs.lowered.launches) {
    const ins = new Set(nodes[l.node].inputs);
    const walk = (records) => {
      for (const a of records || []) {
        for (const i of nodes[a.producer].inputs) ins.add(i);
        walk(a.absorbed);
      }
    };
    walk(l.absorbed);
    for (const f of l.rowFolds || []) {
      for (const i of nodes[f.reduction].inputs) ins.add(i);
      if (f.producer !== undefined) for (const i of nodes[f.producer].inputs) ins.add(i);
    }
    need(l.node, ins);
  }
  const put = (a, id) => {
    const entry = {};
    if (wantWhole.has(id)) entry.whole = bundle.put(a);
    if (wantBlocks.has(id)) {
      const q = twin.graph.nodes[id].shape[axis[id]];
      entry.blocks = seqs.map((b) => bundle.put(takeBlock(a, nodes[id].shape, axis[id], q, b)));
    }
    return entry;
  };
  const values = {}, perfOut = {};
  for (let id = 0; id < nodes.length; id++) if (wantBlocks.has(id) || wantWhole.has(id)) values[id] = put(r.values[id], id);
  for (const l of fs.lowered.launches) perfOut[l.node] = put(perf[l.node], l.node);
  bundle.add({ name: `${req.model}-B${B}`, graph: fs.graph.toJSON(), twin: twin.graph.toJSON(), axis, sequences: seqs,
    launched, perfLaunched: fs.lowered.launches.map((l) => l.node), values, perf: perfOut,
    canaryChecked: r.canaryIntact.every(Boolean),
    canaryPerf: fs.lowered.launches.every((l) => perf.canaryIntact[l.node]),
    loss: r.values[fs.loss][0], dispatchKinds: fs.lowered.launches.map((l) => l.kind),
    splitK: fs.lowered.launches.filter((l) => l.kernels.some((k) => /_red$/.test(k.name))).length,
    batches: (fs.lowered.batches || []).length, aliases: fs.lowered.aliases, folded: fs.lowered.folded, dead: fs.lowered.dead,
    rowFolds: rowFoldsOf(fs.lowered), absorbed: absorbedOf(fs.lowered), formed: formedOf(fs.lowered) });
  bundle.close({ device: runner.info() });
}

/** {chain node: [{ reduction, pos }]}: the row reductions a perf lowering folded into their chains. */
function rowFoldsOf(lowered) {
  const out = {};
  for (const l of lowered.launches) if (l.rowFolds) out[l.node] = l.rowFolds;
  return out;
}

/** {reader node: [{ slot, op, node, source }]}: the ops a perf lowering's matmuls apply to operands as they load them. */
function loadOpsOf(lowered) {
  const out = {};
  for (const l of lowered.launches) {
    for (const [slot, v] of Object.entries(l.views || {})) {
      if (!v.view.op) continue;
      if (!out[l.node]) out[l.node] = [];
      out[l.node].push({ slot, op: v.view.op, node: v.opNode, source: v.source });
    }
  }
  return out;
}

/** {reader node: [{ producer, pos, producerPos, absorbed? }]}: the producers a perf lowering's launches form. */
function absorbedOf(lowered) {
  const out = {};
  for (const l of lowered.launches) if (l.absorbed) out[l.node] = l.absorbed;
  return out;
}

/** {reader node: [{ value, rowFolds?, absorbed? }]}: the values a perf lowering's launches form. */
function formedOf(lowered) {
  const out = {};
  for (const l of lowered.launches) if (l.formed) out[l.node] = l.formed;
  return out;
}

/**
 * The timing protocol's counters and their self-test (src/fusion/bench.js:122-132,
 * 175-192 there: a deliberate leak inside the timed region must be caught): a small fused
 * program timed once as the bench times it (nothing may be created or copied inside the
 * repetitions), then again with `leak` (an allocation and a free inside every
 * repetition), which must throw; and a timed region around an upload, which must throw
 * unless uploads are allowed (a training step's batch).
 */
async function gpuBenchSelftest() {
  const { HipRunner } = require('../src/mi355x/runner');
  const { HipBench, TimedRegionError } = require('../src/mi355x/bench');
  const { chainWorkload, chainInputs } = require('../src/builders/chains');
  const runner = HipRunner.create();
  const bench = new HipBench(runner);
  const w = chainWorkload(0, 64, 1024), inputs = chainInputs(0, 64, 1024);
  const f = fuse(w.forward.graph, { keep: w.forward.keep });
  const lf = lowerMI355X(f.graph, { perf: true, keep: w.forward.keep.map((id) => f.index.get(id)) });
  const p = runner.prepare(f.graph, lf);
  for (const n of f.graph.nodes) if (n.op === 'input') p.write(n.id, inputs[n.attrs.name]);
  const out = { clean: null, leak: null, upload: null, uploadAllowed: null };
  const t = bench.time({ fused: p }, { reps: 4, warmup: 1 });
  out.clean = { k: t.k, checked: bench.checked };
  const trips = (fn) => {
    try { fn(); return { threw: false }; } catch (e) {
      return { threw: e instanceof TimedRegionError, created: e.created || null, message: e.message };
    }
  };
  out.leak = trips(() => bench.time({ fused: p }, { reps: 2, warmup: 0, leak: true }));
  const h = runner.a.malloc(16);
  out.upload = trips(() => bench.region(() => runner.a.h2d(h, 0, new Float32Array(4))));
  out.uploadAllowed = trips(() => bench.region(() => runner.a.h2d(h, 0, new Float32Array(4)), ['h2d']));
  runner.a.free(h);
  out.checked = bench.checked;
  p.destroy();
  bench.destroy();
  return out;
}

async function gpuTrain(req) {
  const { modelStep } = require('../src/builders/models');
  const { fusedStep, HipTrainer } = require('../src/mi355x/trainer');
  const { HipRunner } = require('../src/mi355x/runner');
  const m = modelStep(req);
  const fs = fusedStep(m.step, { attention: !!req.attention });
  const runner = HipRunner.create();
  const trainer = new HipTrainer(runner, fs, m.params, m.state, { graph: !!req.graph, arena: !!req.arena, streams: req.streams || 1 });
  const plan = trainer.program.arena;
  const dispatches = trainer.program.dispatches;
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
      // The checked path: the plain lowering (one launch per node), against the trainer's perf lowering.
      const r = await runner.run(fs.graph, fs.checked, feed);
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
  return { losses, identical, params, launches: fs.lowered.launches.length, checkedLaunches: fs.checked.launches.length,
    folded: fs.lowered.folded.length, aliases: fs.lowered.aliases.length, unfusedNodes: m.step.graph.nodes.length, info: m.info,
    arena: plan ? { bytes: plan.size, unshared: plan.unshared, buffers: plan.buffers.length } : null,
    batches: (fs.lowered.batches || []).length, dispatches,
    batchSaves: (fs.lowered.batches || []).reduce((c, b) => c + (b.count - 1) * b.kernels.length, 0),
    kernels: fs.lowered.launches.reduce((c, l) => c + l.kernels.length, 0) };
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
          const f = fuse(g, { keep: c.keep || [], recompute: !!c.recompute, sabotage: c.sabotage, attention: !!c.attention });
          return Object.assign({ name: c.name, summary: fusionSummary(g, f) }, fusedOut(f));
        } catch (e) {
          return { name: c.name, error: String(e.message) };
        }
      });
      break;
    case 'lower': {
      const g = Graph.fromJSON(req.graph);
      const target = req.fuse ? fuse(g, { keep: req.fuse.keep || [], recompute: !!req.fuse.recompute }).graph : g;
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
    case 'random-programs': {
      // The reference's v2 random programs (the fuzzing corpus generator), as graphs and outputs.
      const { randomProgram } = require('../src/testing/random_graph');
      out = req.programs.map((r) => {
        const p = randomProgram(r.seed, { focus: r.focus || undefined, f32: !!r.f32 });
        return { seed: r.seed, focus: p.focus, graph: p.graph.toJSON(), outputs: p.outputs, inputs: p.inputs, bounds: p.bounds };
      });
      break;
    }
    case 'corpus-fusion': {
      // The fusion pass over corpus programs [from, to]: the counts the reference records
      // (measurements.json m4.semantics.corpus, m4.passSabotage, gpu-m4.json fuzz structure).
      const { corpusGraphs } = require('../src/testing/random_graph');
      const sem = { graphs: 0, withFused: 0, fusedNodes: 0, byPattern: {} };
      const fz = { runs: 0, fusedRuns: 0, byKind: {}, byPattern: {} };
      const sab = { graphs: 0, changed: 0, threw: 0 };
      for (let i = req.from; i <= req.to; i++) {
        for (const c of corpusGraphs(i)) {
          const f = fuse(c.graph, { keep: c.keep });
          const fusedNodes = f.graph.nodes.filter((n) => n.op === 'fused');
          sem.graphs++;
          if (fusedNodes.length) sem.withFused++;
          sem.fusedNodes += fusedNodes.length;
          for (const n of fusedNodes) sem.byPattern[n.attrs.pattern] = (sem.byPattern[n.attrs.pattern] || 0) + 1;
          // The GPU fuzzer runs a matmul program twice (the reference's naive and tiled matmuls).
          const reps = c.graph.nodes.some((n) => n.op === 'matmul') ? 2 : 1;
          const kinds = new Set(fusedNodes.map((n) => n.attrs.kind)), patterns = new Set(fusedNodes.map((n) => n.attrs.pattern));
          fz.runs += reps;
          if (fusedNodes.length) fz.fusedRuns += reps;
          for (const k of kinds) fz.byKind[k] = (fz.byKind[k] || 0) + reps;
          for (const q of patterns) fz.byPattern[q] = (fz.byPattern[q] || 0) + reps;
          if (i <= (req.sabotageTo || 0)) {
            sab.graphs++;
            try {
              const bad = fuse(c.graph, { keep: c.keep, sabotage: 'fusion-absorbs-shared' });
              if (JSON.stringify(bad.graph.toJSON().nodes) !== JSON.stringify(f.graph.toJSON().nodes)) sab.changed++;
            } catch (e) {
              sab.threw++;
              sab.changed++;
            }
          }
        }
      }
      out = { semantics: sem, fuzz: fz, passSabotage: sab };
      break;
    }
    case 'config-graphs': {
      // Forward and gradient graphs of configs 2, 3 and 4 at the requested sizes.
      const cfg = require('../src/builders/configs');
      const { chainWorkload } = require('../src/builders/chains');
      const one = (v) => ({ graph: v.graph.toJSON(), keep: v.keep });
      out = {
        c2: (req.c2 || []).map((c) => { const w = chainWorkload(c.seed, c.R, c.C); return { seed: c.seed, R: c.R, C: c.C, forward: one(w.forward), gradient: one(w.gradient) }; }),
        c3: (req.c3 || []).map((c) => { const g = cfg.c3Graphs(c.fn, c.R, c.C); return { fn: c.fn, R: c.R, C: c.C, forward: one(g.forward), gradient: one(g.gradient) }; }),
        c4: (req.c4 || []).map((c) => { const g = cfg.c4Graphs(c.act, c.M, c.K, c.N); return { act: c.act, M: c.M, K: c.K, N: c.N, forward: one(g.forward), gradient: one(g.gradient) }; }),
      };
      break;
    }
    case 'scratch-kernels': {
      // The split-K matmuls of the no-allocation entry point's test: one translation unit
      // (as the build precompiles it), and per shape its kernels in launch order with their
      // launch shapes, parameters and workspace bytes.
      const { translationUnit } = require('../src/mi355x/runner');
      const lists = scratchLowerings(SCRATCH_SHAPES);
      const m = new Map();
      for (const l of lists) for (const [name, src] of kernelSources(l)) m.set(name, src);
      out = { unit: translationUnit(m), shapes: SCRATCH_SHAPES, launches: lists.map((l) => {
        const x = l.launches[0];
        return { workspace: l.workspace, params: Array.from(x.params),
          kernels: x.kernels.map((k) => ({ name: k.name, grid: k.grid, block: k.block, lds: k.lds })) };
      }) };
      break;
    }
    case 'kernel-unit': {
      // One translation unit of every kernel the standard runs launch (config 5's step in
      // both lowerings, configs 2-4 fused in the perf lowering, the forward pass with
      // attention fused), as the runner compiles them: for resource checks of the code.
      const { translationUnit } = require('../src/mi355x/runner');
      const { modelStep } = require('../src/builders/models');
      const { fusedStep } = require('../src/mi355x/trainer');
      const { chainWorkload } = require('../src/builders/chains');
      const cfg = require('../src/builders/configs');
      const m = new Map();
      const add = (lw) => { for (const [name, src] of kernelSources(lw)) m.set(name, src); };
      const perf = (v, fuseOpts) => {
        const f = fuse(v.graph, Object.assign({ keep: v.keep }, fuseOpts || {}));
        add(lowerMI355X(f.graph, { perf: true, keep: v.keep.map((id) => f.index.get(id)) }));
      };
      const fs = fusedStep(modelStep({ model: 'transformer', B: 64 }).step);
      add(fs.lowered);
      add(fs.checked);
      // The step with attention and its gradient fused (its joint gradient kernel included).
      const fa = fusedStep(modelStep({ model: 'transformer', B: 64 }).step, { attention: true });
      add(fa.lowered);
      add(fa.checked);
      for (let s2 = 0; s2 < 8; s2++) { const w = chainWorkload(s2, 8192, 1024); perf(w.forward); perf(w.gradient); }
      for (const fn of ['softmax', 'logSoftmax']) { const g = cfg.c3Graphs(fn, cfg.C3_SHAPE[0], cfg.C3_SHAPE[1]); perf(g.forward); perf(g.gradient); }
      for (const [M, K, N] of cfg.C4_SHAPES) for (const act of ['relu', 'tanh']) { const g = cfg.c4Graphs(act, M, K, N); perf(g.forward); perf(g.gradient); }
      const fw = transformerForward({ config: 'c5', V: 96, B: 64 });
      perf({ graph: Graph.fromJSON(fw.graph), keep: fw.keep }, { attention: true });
      out = { kernels: Array.from(m.keys()), unit: translationUnit(m) };
      break;
    }
    case 'schedule-check': {
      // Stream schedules of model steps and corpus programs (perf lowering) at 2..4 streams,
      // checked by replaying them with vector clocks; with `plant`, one wait dropped.
      const { scheduleLaunches } = require('../src/mi355x/schedule');
      const { checkSchedule } = require('../src/testing/schedule_check');
      out = [];
      const one = (name, graph, keep) => {
        const lw = lowerMI355X(graph, { perf: true, keep, absorb: true });
        const alias = new Map(lw.aliases);
        const owner = (id) => (alias.has(id) ? alias.get(id) : id);
        for (const streams of [2, 3, 4]) {
          const sc = scheduleLaunches(lw.launches, streams, owner);
          const rec = { name, streams, launches: lw.launches.length, criticalPath: sc.criticalPath, waits: sc.waits.length,
            used: new Set(sc.streamOf).size, check: checkSchedule(lw.launches, sc, owner) };
          if (req.plant && sc.waits.length) {
            const k = sc.waitBegin.findIndex((b, i) => i < sc.streamOf.length && sc.waitBegin[i + 1] > b);
            const broken = Object.assign({}, sc, { waits: sc.waits.slice(), waitBegin: sc.waitBegin.slice() });
            // Drop the first wait of kernel k: shift the later ranges down by one.
            broken.waits = Uint32Array.from([...sc.waits.slice(0, sc.waitBegin[k]), ...sc.waits.slice(sc.waitBegin[k] + 1)]);
            for (let i = k + 1; i < broken.waitBegin.length; i++) broken.waitBegin[i]--;
            rec.planted = checkSchedule(lw.launches, broken, owner);
          }
          out.push(rec);
        }
      };
      const { modelStep } = require('../src/builders/models');
      const { fusedStep } = require('../src/mi355x/trainer');
      for (const r of req.models || []) {
        const m = modelStep(r);
        const f = fusedStep(m.step, { attention: !!r.attention });
        one(`${r.model}-${r.B || ''}${r.attention ? '-attention' : ''}`, f.graph, [f.loss, f.logits].concat(Object.values(f.outputs)));
      }
      if (req.corpus) {
        const { corpusGraphs } = require('../src/testing/random_graph');
        for (let i = req.corpus.from; i <= req.corpus.to; i++) {
          for (const c of corpusGraphs(i)) {
            const f = fuse(c.graph, { keep: c.keep });
            one(`corpus-${i}-${c.label}`, f.graph, c.keep.map((id) => f.index.get(id)));
          }
        }
      }
      break;
    }
    case 'arena-check': {
      // Arena plans of model steps and corpus programs (perf lowering), checked by running
      // each launch list abstractly over the arena's bytes.
      const { planArena } = require('../src/mi355x/arena');
      const { simulateArena, peakLive } = require('../src/testing/arena_check');
      const one = (name, graph, keep) => {
        const lowered = lowerMI355X(graph, { perf: true, keep, absorb: true });
        const plan = planArena(graph, lowered, { keep });
        const res = { name, launches: lowered.launches.length, buffers: plan.buffers.length, bytes: plan.size,
          unshared: plan.unshared, peak: peakLive(lowered, plan), check: simulateArena(graph, lowered, plan) };
        if (req.plant) {
          // A planted mistake: one buffer moved onto another that is live at the same
          // time (the first such pair); the simulation must refuse the plan.
          const bs = plan.buffers;
          let pair = null;
          for (const a of bs) {
            if (a.pinned) continue;
            const b = bs.find((x) => x !== a && x.lo <= a.hi && a.lo <= x.hi && x.bytes >= a.bytes);
            if (b) { pair = [a, b]; break; }
          }
          if (pair) {
            const saved = pair[0].offset;
            pair[0].offset = pair[1].offset;
            res.planted = { moved: pair[0].id, onto: pair[1].id, check: simulateArena(graph, lowered, plan) };
            pair[0].offset = saved;
          }
          // A plan that takes the members of each batched launch one after another:
          // its reuse of a member's last operand for a later member's output is a race.
          if ((lowered.batches || []).length) {
            const blind = planArena(graph, Object.assign({}, lowered, { batches: [] }), { keep });
            res.batchBlind = simulateArena(graph, lowered, blind);
          }
        }
        return res;
      };
      out = [];
      const { modelStep } = require('../src/builders/models');
      const { fusedStep } = require('../src/mi355x/trainer');
      for (const r of req.models || []) {
        const m = modelStep(r);
        const f = fusedStep(m.step, { attention: !!r.attention });
        out.push(one(`${r.model}-${r.B || ''}${r.attention ? '-attention' : ''}`, f.graph, [f.loss, f.logits].concat(Object.values(f.outputs))));
      }
      if (req.corpus) {
        const { corpusGraphs } = require('../src/testing/random_graph');
        for (let i = req.corpus.from; i <= req.corpus.to; i++) {
          for (const c of corpusGraphs(i)) {
            const f = fuse(c.graph, { keep: c.keep });
            out.push(one(`corpus-${i}-${c.label}`, f.graph, c.keep.map((id) => f.index.get(id))));
          }
        }
      }
      break;
    }
    case 'grouped-batches': {
      // The batched forms of a model step's split-K products (their workgroups take
      // XCD-grouped places): each batched kernel's text and its members' z extent.
      const { modelStep } = require('../src/builders/models');
      const { fusedStep } = require('../src/mi355x/trainer');
      const { kernelSources } = require('../src/mi355x/lower');
      const fs = fusedStep(modelStep(req).step, { attention: !!req.attention });
      const src = kernelSources(fs.lowered);
      const kernels = [];
      let batches = 0;
      for (const b of fs.lowered.batches || []) {
        const l = fs.lowered.launches[b.start];
        if (!(l.kernels.length === 2 && /_red$/.test(l.kernels[1].name))) continue;
        batches++;
        const k = b.kernels[0];
        kernels.push({ name: k.name, z: l.kernels[0].grid[2], source: src.get(k.name) });
      }
      out = { batches, kernels };
      break;
    }
    case 'ragged-batches': {
      // The ragged batches of model steps and corpus programs (perf lowering): each batched
      // kernel's text, grid and workgroup size, and its members' kernel grids in order.
      const { modelStep } = require('../src/builders/models');
      const { fusedStep } = require('../src/mi355x/trainer');
      const lowerings = [];
      for (const r of req.models || []) {
        const fs = fusedStep(modelStep(r).step, { attention: !!r.attention });
        lowerings.push([`${r.model}-${r.B || ''}`, fs.lowered]);
      }
      if (req.corpus) {
        const { corpusGraphs } = require('../src/testing/random_graph');
        for (let i = req.corpus.from; i <= req.corpus.to; i++) {
          for (const c of corpusGraphs(i)) {
            const f = fuse(c.graph, { keep: c.keep });
            lowerings.push([`corpus-${i}-${c.label}`, lowerMI355X(f.graph, { perf: true, keep: c.keep.map((id) => f.index.get(id)), absorb: true })]);
          }
        }
      }
      out = [];
      for (const [name, lo] of lowerings) {
        for (const b of lo.batches || []) {
          if (!b.ragged) continue;
          const k = b.kernels[0];
          out.push({ name, kernel: k.name, source: k.source, grid: k.grid, block: k.block,
            members: lo.launches.slice(b.start, b.start + b.count).map((l) => ({ kernel: l.kernels[0].name, grid: l.kernels[0].grid, block: l.kernels[0].block })) });
        }
      }
      break;
    }
    case 'batch-check': {
      // Batched launches of model steps and corpus programs (perf lowering), checked against
      // the plain order; with `plant`, the planted mistakes of batch_check.js as well.
      const { checkBatches, plantBatchMistake } = require('../src/testing/batch_check');
      const one = (name, graph, keep) => {
        const plain = lowerMI355X(graph, { perf: true, keep, batch: false, absorb: true });
        const batched = lowerMI355X(graph, { perf: true, keep, absorb: true });
        const res = { name, launches: batched.launches.length, check: checkBatches(plain, batched) };
        if (req.plant) {
          for (const kind of ['dependent', 'early', 'grid', 'body']) {
            const bad = plantBatchMistake(batched, kind);
            if (bad) res[kind] = checkBatches(plain, bad);
          }
        }
        return res;
      };
      out = [];
      const { modelStep } = require('../src/builders/models');
      const { fusedStep } = require('../src/mi355x/trainer');
      for (const r of req.models || []) {
        const f = fusedStep(modelStep(r).step, { attention: !!r.attention });
        out.push(one(`${r.model}-${r.B || ''}${r.attention ? '-attention' : ''}`, f.graph, [f.loss, f.logits].concat(Object.values(f.outputs))));
      }
      if (req.corpus) {
        const { corpusGraphs } = require('../src/testing/random_graph');
        for (let i = req.corpus.from; i <= req.corpus.to; i++) {
          for (const c of corpusGraphs(i)) {
            const f = fuse(c.graph, { keep: c.keep });
            out.push(one(`corpus-${i}-${c.label}`, f.graph, c.keep.map((id) => f.index.get(id))));
          }
        }
      }
      break;
    }
    case 'concurrent-check': {
      // A concurrent group over stand-in programs (no device): stream assignment, the
      // concatenated launch arrays, and the refusal of programs that share a written buffer.
      const { Concurrent } = require('../src/mi355x/runner');
      const fake = (i, bytes, kernels, shareWith) => {
        const launches = bytes.map((b, j) => ({ node: j + 1, inputs: [0], bytes: b }));
        const bufs = [1000 * (i + 1)].concat(bytes.map((_, j) => (shareWith !== undefined && j === 0 ? 1000 * (shareWith + 1) + 1 : 1000 * (i + 1) + j + 1)));
        const args = new Uint8Array(kernels * 16).map((_, q) => (i * 16 + q) % 256);
        return { dag: null, launches, bufs, ws: 900000 + i, count: kernels, fns: new Float64Array(kernels).fill(i + 1),
          dims: new Uint32Array(kernels * 7).fill(i), args, offsets: Uint32Array.from({ length: kernels + 1 }, (_, q) => q * 16) };
      };
      const runner = { a: {} };
      const programs = (req.bytes || [[5], [3, 3], [4], [1], [2, 2]]).map((b, i) => fake(i, b, b.length + 1));
      const g = new Concurrent(runner, programs, req.streams || 2);
      let refused = null;
      try { new Concurrent(runner, [fake(0, [1], 1), fake(1, [1], 1, 0)], 2); } catch (e) { refused = String(e.message); }
      out = { load: g.load, streamOf: Array.from(g.streamOf), fns: Array.from(g.fns), offsets: Array.from(g.offsets),
        args: Array.from(g.args), refused };
      break;
    }
    case 'attention-graphs': out = attentionGraphs(req.cases || ATTENTION_CASES); break;
    case 'transformer-forward': out = transformerForward(req); break;
    case 'chain-map': {
      // The index maps of values read through chains of transposes and reshapes (lower.js
      // chainMap): for each { shape, chain: [["transpose", perm] | ["reshape", shape]] }, the
      // factor lists per dimension of the chain's value, or null where no such map exists.
      const { chainMap } = require('../src/mi355x/lower');
      out = req.cases.map((c) => {
        const g = new Graph();
        let x = g.input('s', c.shape);
        const ids = [];
        for (const [op, arg] of c.chain) {
          // The builder returns its operand for an identity transpose or reshape.
          const y = op === 'transpose' ? g.transpose(x, arg) : g.reshape(x, arg);
          if (y !== x) ids.push(y);
          x = y;
        }
        return { map: chainMap(g, 0, ids), shape: g.nodes[x].shape };
      });
      break;
    }
    case 'perf-lower': {
      // The perf lowering of a model step or of a graph: launches, aliases, folded nodes, operand views.
      // A model's fused step as the trainer lowers it (producers absorbed); a graph with
      // absorb: true likewise.
      let g, keep, absorb = !!req.absorb;
      if (req.model && req.unfused) {
        // The model's step graph without fusion (the bench's unfused step).
        const { modelStep } = require('../src/builders/models');
        const st = modelStep(req).step;
        g = st.graph;
        keep = [st.loss, st.logits].concat(Object.values(st.outputs));
      } else if (req.model) {
        const { modelStep } = require('../src/builders/models');
        const { fusedStep } = require('../src/mi355x/trainer');
        const fs = fusedStep(modelStep(req).step, { attention: !!req.attention });
        g = fs.graph;
        keep = [fs.loss, fs.logits].concat(Object.values(fs.outputs));
        absorb = true;
      } else if (req.workload) {
        // A sweep workload's graph, unfused (as given).
        const { workloads } = require('../src/builders/workloads');
        const m = workloads().find((w) => w.id === req.workload).make();
        g = m.graph;
        keep = m.outputs;
      } else {
        g = Graph.fromJSON(req.graph);
        keep = req.keep || [];
        if (req.fuse) {
          // The graph fused first (with the recompute option as asked); ids are the fused graph's.
          const f = fuse(g, { keep, recompute: !!req.fuse.recompute });
          g = f.graph;
          keep = keep.map((id) => f.index.get(id));
        }
      }
      const l = lowerMI355X(g, { perf: true, keep, absorb });
      const plain = new Map(lowerMI355X(g).launches.map((x) => [x.node, x]));
      out = { graph: g.toJSON(), keep, aliases: l.aliases, folded: l.folded, dead: l.dead, rowFolds: rowFoldsOf(l), absorbed: absorbedOf(l), formed: formedOf(l), loadOps: loadOpsOf(l),
        launches: l.launches.map((x) => ({ node: x.node, kind: x.kind, inputs: x.inputs, params: x.params.length, views: x.views || null, modes: gemmModes(x),
          split: gemmSplit(x), plainSplit: gemmSplit(plain.get(x.node)) })),
        batches: (l.batches || []).map((b) => ({ start: b.start, count: b.count, joint: !!b.joint, kernels: b.kernels.map((k) => k.name) })) };
      if (req.sources) out.sources = Object.fromEntries(kernelSources(l));
      break;
    }
    case 'precompile': out = { kernels: precompileGroup(req.group || 'direct', req.arch, req.shard, req.shards) }; break;
    case 'gpu-direct': await gpuDirect(outDir(argv), req); out = { ok: true }; break;
    case 'step-graph': stepGraph(req, outDir(argv)); out = { ok: true }; break;
    case 'forward-graph': forwardGraph(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-local': await gpuLocal(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-workloads': await gpuWorkloads(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-step-slices': await gpuStepSlices(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-train': out = await gpuTrain(req); break;
    case 'gpu-bench-selftest': out = await gpuBenchSelftest(); break;
    case 'gpu-concurrent': out = await gpuConcurrent(req); break;
    case 'gpu-chains': await gpuChains(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-graphs': await gpuGraphs(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-configs': await gpuConfigs(req, outDir(argv)); out = { ok: true }; break;
    case 'gpu-fuzz': await gpuFuzz(req, outDir(argv)); out = { ok: true }; break;
    default:
      throw new Error(`unknown command '${cmd}'`);
  }
  process.stdout.write(JSON.stringify(out));
}

main().catch((e) => {
  process.stderr.write(`${e.stack || e}\n`);
  process.exit(1);
});
