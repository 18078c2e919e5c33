'use strict';
// The reference's timed workload sweep (src/fusion/workloads.js:71-120 in
// abho7/tensor-compiler-webgpu), the graph workloads of it: unary and binary
// elementwise chains, matmul + bias -> relu | gelu at its matmul shapes,
// LayerNorm and softmax over its row grid (rows capped at 2^22 elements), the
// broadcast-recompute and lost-reuse workloads built so that fusion loses, and
// the reference transformer's forward pass and training step. Each workload
// names its variants: unfused (one launch per node), fused, recompute (the
// fusion pass with recomputation allowed) and, for the step, matmul-only (its
// matmul launches alone). The reference's hand-written WGSL baselines are a
// WebGPU comparison with no counterpart here.

const { Graph } = require('../ir/graph');
const { size } = require('../ir/shapes');
const { Rng } = require('../testing/rng');
const { layerNormGraph, geluGraph, unaryChain } = require('./direct_cases');
const tf = require('./transformer');

const CHAIN_LENGTHS = [1, 2, 4, 8, 16];
const CHAIN_SIZES = [1000, 65537, 1048573, 4194301];
const BINARY_LENGTHS = [1, 2, 4, 8];
const BINARY_SIZES = [65537, 4194301];
const MATMUL_SHAPES = [[512, 64, 64], [512, 64, 256], [512, 256, 64], [1000, 63, 257], [4096, 64, 256], [128, 1024, 128], [2048, 512, 512]];
const ROW_C = [1, 7, 64, 65, 256, 1000, 4096];
const ROW_R = [1, 64, 4096, 65536];
const ROW_CAP = 2 ** 22;
const BROADCAST_R = [16, 256, 4096];
const REUSE_SIZE = 1048573;

/** Inputs uniform in [lo, hi] (default [-2, 2]) from Rng(seed), in input order. */
function drawInputs(graph, seed, ranges) {
  const rng = new Rng(seed);
  const out = {};
  for (const n of graph.inputs()) {
    const r = (ranges && ranges[n.attrs.name]) || [-2, 2];
    out[n.attrs.name] = Float32Array.from(rng.array(size(n.shape), r[0], r[1]));
  }
  return out;
}

function graphWorkload(id, family, params, build, options) {
  const o = options || {};
  return {
    // Outputs judged against the composed float32 budget of the whole graph.
    id, family, params, judge: 'composed', variants: o.variants || ['unfused', 'fused'],
    make() {
      const g = new Graph();
      const outputs = [].concat(build(g));
      return { graph: g, outputs, inputs: drawInputs(g, o.seed || 1, o.ranges) };
    },
  };
}

function binaryChain(g, n, L) {
  let y = g.input('x0', [n]);
  const ops = ['add', 'mul', 'sub'];
  for (let k = 1; k <= L; k++) y = g[ops[(k - 1) % 3]](y, g.input(`x${k}`, [n]));
  return y;
}

/** The reference transformer's forward pass or Adam step at (V, B), its seeding and a random batch. */
function modelWorkload(what, V, B) {
  return {
    // The model's composed budget is infinite at its logits (layer norm divides by a
    // deviation whose bound exceeds it), so its variants are compared with each other
    // and must be finite (the reference's revision R6).
    id: `${what}-V${V}-B${B}`, family: what === 'step' ? 'training-step' : 'forward', params: { V, B }, judge: 'compare',
    variants: what === 'step' ? ['unfused', 'fused', 'matmul-only'] : ['unfused', 'fused'],
    make() {
      const cfg = tf.REFERENCE_CONFIG;
      const rng = new Rng(V * 1000 + B);
      const rows = B * cfg.T;
      const tokens = Array.from({ length: rows }, () => rng.int(0, V - 1));
      const targets = Array.from({ length: rows }, () => rng.int(0, V - 1));
      const onehot = (ids) => { const a = new Float32Array(ids.length * V); ids.forEach((t, i) => { a[i * V + t] = 1; }); return a; };
      const params = {};
      const init = tf.initParams(V, 1, cfg);
      for (const k of Object.keys(init)) params[k] = Float32Array.from(init[k]);
      if (what === 'forward') {
        const f = tf.buildForward(V, B, cfg);
        return { graph: f.graph, outputs: [f.logits, f.loss], inputs: Object.assign({}, params, { x: onehot(tokens), y: onehot(targets) }) };
      }
      const s = tf.buildStep(V, B, cfg, tf.ADAM_3B);
      const state = tf.adamInitialState(s.names, s.shapes);
      const inputs = Object.assign({}, params, state, { x: onehot(tokens), y: onehot(targets) });
      inputs[s.cotangent] = new Float32Array([1]);
      return { graph: s.graph, outputs: [s.loss].concat(Object.values(s.outputs)), inputs };
    },
  };
}

/** Every graph workload of the sweep, in the reference's order. */
function workloads() {
  const w = [];
  for (const n of CHAIN_SIZES) for (const L of CHAIN_LENGTHS) {
    w.push(graphWorkload(`chain-unary-L${L}-n${n}`, 'chain-unary', { L, n }, (g) => unaryChain(g, g.input('x', [n]), L)));
  }
  for (const n of BINARY_SIZES) for (const L of BINARY_LENGTHS) {
    w.push(graphWorkload(`chain-binary-L${L}-n${n}`, 'chain-binary', { L, n }, (g) => binaryChain(g, n, L)));
  }
  for (const [M, K, N] of MATMUL_SHAPES) for (const act of ['relu', 'gelu']) {
    w.push(graphWorkload(`matmul-${act}-${M}x${K}x${N}`, 'matmul-epilogue', { M, K, N, act }, (g) => {
      const y = g.add(g.matmul(g.input('a', [M, K]), g.input('w', [K, N])), g.input('bias', [N]));
      return act === 'relu' ? g.relu(y) : geluGraph(g, y);
    }, { ranges: { w: [-1 / Math.sqrt(K), 1 / Math.sqrt(K)] } }));
  }
  for (const pattern of ['layernorm', 'softmax']) for (const C of ROW_C) for (const R of ROW_R) {
    if (R * C > ROW_CAP) continue;
    w.push(graphWorkload(`${pattern}-R${R}-C${C}`, pattern, { R, C }, (g) => (pattern === 'layernorm'
      ? layerNormGraph(g, g.input('x', [R, C]), g.input('g', [C]), g.input('b', [C]))
      : g.softmax(g.input('x', [R, C]), 1))));
  }
  for (const R of BROADCAST_R) {
    w.push(graphWorkload(`broadcast-recompute-R${R}`, 'broadcast-recompute', { R, C: 256, ops: 16 },
      (g) => g.add(g.input('y', [R, 256]), unaryChain(g, g.input('p', [256]), 16)), { variants: ['unfused', 'fused', 'recompute'] }));
  }
  for (const ops of [1, 16]) {
    w.push(graphWorkload(`lost-reuse-${ops}op`, 'lost-reuse', { ops, consumers: 4, n: REUSE_SIZE }, (g) => {
      const t = unaryChain(g, g.input('x', [REUSE_SIZE]), ops);
      return [g.mul(t, g.const(2)), g.add(t, g.const(1)), g.tanh(t), g.exp(g.neg(t))];
    }, { variants: ['unfused', 'fused', 'recompute'] }));
  }
  for (const [V, B] of [[16, 8], [75, 16]]) w.push(modelWorkload('forward', V, B));
  for (const [V, B] of [[16, 8], [16, 16], [75, 16]]) w.push(modelWorkload('step', V, B));
  return w;
}

module.exports = { workloads, CHAIN_LENGTHS, CHAIN_SIZES, MATMUL_SHAPES, ROW_C, ROW_R, ROW_CAP };
