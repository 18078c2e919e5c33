'use strict';
// Benchmark config 1: the MLP training step as one IR graph — X [128, 64] ->
// dense 64->128 tanh -> dense 128->10, log-softmax cross-entropy against
// one-hot labels, autodiff's gradient graph, plain SGD (p - 0.1·g) — built the
// way the reference builds its MLP step (src/train/step.js:60-127 in
// abho7/tensor-compiler-webgpu: forward, mean NLL, grad, optimizer as IR ops).
// Differences the config asks for: tanh instead of relu (so the activation
// epilogue survives fusion in the step graph), plain SGD instead of momentum
// with weight decay, N(0, 1/fan_in) weights, zero biases.

const { Graph } = require('../ir/graph');
const { grad } = require('../autodiff');
const { Rng } = require('../testing/rng');

const PARAMS = ['W1', 'b1', 'W2', 'b2'];
const C1 = { batch: 128, inputs: 64, hidden: 128, classes: 10, lr: 0.1, seed: 0 };

function shapes(c) { return { W1: [c.inputs, c.hidden], b1: [c.hidden], W2: [c.hidden, c.classes], b2: [c.classes] }; }

function buildMlpStep(c) {
  const cfg = c || C1;
  const g = new Graph();
  const s = shapes(cfg);
  const ids = {};
  for (const p of PARAMS) ids[p] = g.input(p, s[p]);
  ids.x = g.input('x', [cfg.batch, cfg.inputs]);
  ids.y = g.input('y', [cfg.batch, cfg.classes]);
  const h = g.tanh(g.add(g.matmul(ids.x, ids.W1), ids.b1));
  const logits = g.add(g.matmul(h, ids.W2), ids.b2);
  const logp = g.logSoftmax(logits, 1);
  const loss = g.div(g.neg(g.sum(g.sum(g.mul(ids.y, logp), 1), 0)), g.const(cfg.batch));
  const G = grad(g, [loss], PARAMS.map((p) => ids[p]));
  const B = G.graph;
  const outputs = {};
  PARAMS.forEach((p, k) => { outputs[p] = B.sub(ids[p], B.mul(B.const(cfg.lr), G.grads[k])); });
  const inputs = {};
  for (const p of PARAMS) inputs[p] = ids[p];
  inputs.x = ids.x;
  inputs.y = ids.y;
  return { graph: B, names: PARAMS, stateNames: [], loss, logits, inputs, outputs, cotangent: G.cotangents[0], grads: G.grads };
}

/** Config 1's data and parameters from `seed`: X = randint(0..16)/16, labels in 0..9, W ~ N(0, 1/fan_in), b = 0. */
function mlpData(c) {
  const cfg = c || C1;
  const rng = new Rng(cfg.seed);
  const s = shapes(cfg);
  const params = {
    W1: rng.normalF32(s.W1[0] * s.W1[1], 1 / Math.sqrt(cfg.inputs)), b1: new Float32Array(cfg.hidden),
    W2: rng.normalF32(s.W2[0] * s.W2[1], 1 / Math.sqrt(cfg.hidden)), b2: new Float32Array(cfg.classes),
  };
  const x = new Float32Array(cfg.batch * cfg.inputs);
  for (let i = 0; i < x.length; i++) x[i] = rng.int(0, 16) / 16;
  const y = new Float32Array(cfg.batch * cfg.classes);
  const labels = [];
  for (let r = 0; r < cfg.batch; r++) { const l = rng.int(0, cfg.classes - 1); labels.push(l); y[r * cfg.classes + l] = 1; }
  return { params, x, y, labels };
}

module.exports = { buildMlpStep, mlpData, C1, PARAMS };
