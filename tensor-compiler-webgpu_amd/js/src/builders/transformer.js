'use strict';
// A decoder-only, pre-LayerNorm character transformer as one IR graph, and its
// training step (forward, loss, autodiff's backward, optimizer update, all IR).
//
// The structure is the reference's (src/m3b/model.js:29-145 and
// src/m3b/step.js:18-32, src/m3b/adam.js:56-80 in abho7/tensor-compiler-webgpu):
// one-hot tokens [B·T, V] through a matmul embedding, learned positions, per
// block LayerNorm -> attention (heads by reshape/transpose, scores scaled by
// 1/sqrt(dh), causal mask -1e4, softmax) -> residual, LayerNorm -> MLP ->
// residual, final LayerNorm and head, mean next-token cross-entropy. The
// reference fixes its sizes in a module constant (T 64, d 64, L 2, ff 256,
// GELU); here they are a config, so that the same construction builds both the
// reference's model (to pin the fusion pass against its recorded counts) and
// benchmark config 5 (V 96, d 256, H 4, L 4, ff 1024 ReLU, T 128).

const { Graph } = require('../ir/graph');
const { grad } = require('../autodiff');
const { Rng } = require('../testing/rng');
const { layerNormGraph, geluGraph } = require('./direct_cases');

const REFERENCE_CONFIG = { T: 64, d: 64, H: 4, dh: 16, L: 2, ff: 256, eps: 1e-5, mask: -1e4, act: 'gelu' };
const C5_CONFIG = { T: 128, d: 256, H: 4, dh: 64, L: 4, ff: 1024, eps: 1e-5, mask: -1e4, act: 'relu' };
const ADAM_3B = { kind: 'adam', lr: 2e-3, beta1: 0.9, beta2: 0.999, eps: 1e-8, weightDecay: 0 };

const count = (shape) => shape.reduce((a, b) => a * b, 1);

/** Parameters in their fixed order: [name, shape, init] (model.js:29-45). */
function paramSpec(V, cfg) {
  const { T, d, L, ff } = cfg;
  const linear = (fanIn) => ['uniform', 1 / Math.sqrt(fanIn)];
  const spec = [['tok', [V, d], ['uniform', 1]], ['pos', [T, d], ['uniform', 1]]];
  for (let l = 0; l < L; l++) {
    const p = `b${l}.`;
    spec.push(
      [`${p}ln1.g`, [d], ['ones']], [`${p}ln1.b`, [d], ['zeros']],
      [`${p}wq`, [d, d], linear(d)], [`${p}wk`, [d, d], linear(d)], [`${p}wv`, [d, d], linear(d)],
      [`${p}wo`, [d, d], linear(d)], [`${p}bo`, [d], linear(d)],
      [`${p}ln2.g`, [d], ['ones']], [`${p}ln2.b`, [d], ['zeros']],
      [`${p}w1`, [d, ff], linear(d)], [`${p}b1`, [ff], linear(d)],
      [`${p}w2`, [ff, d], linear(ff)], [`${p}b2`, [d], linear(ff)],
    );
  }
  spec.push(['lnf.g', [d], ['ones']], ['lnf.b', [d], ['zeros']], ['head', [d, V], linear(d)], ['headb', [V], linear(d)]);
  return spec;
}

/** The reference's initialisation (model.js:54-62): uniform per spec from Rng((seed·7001 + 13) >>> 0). */
function initParams(V, seed, cfg) {
  const rng = new Rng((seed * 7001 + 13) >>> 0);
  const out = {};
  for (const [name, shape, init] of paramSpec(V, cfg)) {
    const n = count(shape);
    out[name] = init[0] === 'uniform' ? rng.array(n, -init[1], init[1]) : new Array(n).fill(init[0] === 'ones' ? 1 : 0);
  }
  return out;
}

/** Config 5's initialisation: every weight and bias N(0, std^2) from `seed`; LayerNorm gains 1, biases 0. */
function initNormal(V, seed, std, cfg) {
  const rng = new Rng(seed >>> 0);
  const out = {};
  for (const [name, shape, init] of paramSpec(V, cfg)) {
    const n = count(shape);
    if (init[0] === 'uniform') out[name] = rng.normalF32(n, std);
    else out[name] = new Float32Array(n).fill(init[0] === 'ones' ? 1 : 0);
  }
  return out;
}

function causalMask(T, mask) {
  const m = new Array(T * T);
  for (let i = 0; i < T; i++) for (let j = 0; j < T; j++) m[i * T + j] = j <= i ? 0 : mask;
  return m;
}

function attention(g, a, p, B, cfg) {
  const { T, d, H, dh } = cfg;
  const heads = (w) => g.transpose(g.reshape(g.matmul(a, p[w]), [B, T, H, dh]), [0, 2, 1, 3]);
  const q = heads('wq'), k = heads('wk'), v = heads('wv');
  let s = g.matmul(q, g.transpose(k, [0, 1, 3, 2]));
  s = g.mul(s, g.const(1 / Math.sqrt(dh)));
  s = g.add(s, g.const(causalMask(T, cfg.mask), [T, T]));
  const probs = g.softmax(s, 3);
  const o = g.matmul(probs, v);
  const merged = g.reshape(g.transpose(o, [0, 2, 1, 3]), [B * T, d]);
  return g.add(g.matmul(merged, p.wo), p.bo);
}

const BLOCK_KEYS = ['ln1.g', 'ln1.b', 'wq', 'wk', 'wv', 'wo', 'bo', 'ln2.g', 'ln2.b', 'w1', 'b1', 'w2', 'b2'];

/** Logits [B·T, V] of the model on graph `g` (model.js:112-124). */
function logitsOf(g, ids, V, B, cfg) {
  const { T, d, L } = cfg;
  const act = (x) => (cfg.act === 'relu' ? g.relu(x) : geluGraph(g, x));
  let h = g.reshape(g.add(g.reshape(g.matmul(ids.x, ids.tok), [B, T, d]), ids.pos), [B * T, d]);
  for (let l = 0; l < L; l++) {
    const p = {};
    for (const k of BLOCK_KEYS) p[k] = ids[`b${l}.${k}`];
    h = g.add(h, attention(g, layerNormGraph(g, h, p['ln1.g'], p['ln1.b'], cfg.eps), p, B, cfg));
    const m = layerNormGraph(g, h, p['ln2.g'], p['ln2.b'], cfg.eps);
    h = g.add(h, g.add(g.matmul(act(g.add(g.matmul(m, p.w1), p.b1)), p.w2), p.b2));
  }
  return g.add(g.matmul(layerNormGraph(g, h, ids['lnf.g'], ids['lnf.b'], cfg.eps), ids.head), ids.headb);
}

/** Mean next-token cross-entropy over the B·T rows; `y` one-hot (model.js:127-130). */
function lossOf(g, logits, y, rows) {
  const logp = g.logSoftmax(logits, 1);
  return g.div(g.neg(g.sum(g.sum(g.mul(y, logp), 1), 0)), g.const(rows));
}

function buildForward(V, B, cfg) {
  const g = new Graph();
  const ids = {};
  for (const [name, shape] of paramSpec(V, cfg)) ids[name] = g.input(name, shape);
  ids.x = g.input('x', [B * cfg.T, V]);
  ids.y = g.input('y', [B * cfg.T, V]);
  const logits = logitsOf(g, ids, V, B, cfg);
  const loss = lossOf(g, logits, ids.y, B * cfg.T);
  return { graph: g, ids, logits, loss };
}

/** Adam as IR ops (adam.js:56-80), state per parameter m and v, then the two beta powers. */
function adamUpdate(B, names, ids, grads, state, opt) {
  const c = (v) => B.const(v);
  const outputs = {};
  const decayed = (p) => B.add(grads[p], B.mul(c(opt.weightDecay), ids[p]));
  const b1 = B.mul(state.beta1Pow, c(opt.beta1));
  const b2 = B.mul(state.beta2Pow, c(opt.beta2));
  outputs.beta1Pow = b1;
  outputs.beta2Pow = b2;
  const bc1 = B.sub(c(1), b1);
  const bc2 = B.sub(c(1), b2);
  const stepSize = B.div(c(opt.lr), bc1);
  const sqrtBc2 = B.sqrt(bc2);
  for (const p of names) {
    const gp = decayed(p);
    const m = B.add(B.mul(c(opt.beta1), state[`${p}.m`]), B.mul(c(1 - opt.beta1), gp));
    const v = B.add(B.mul(c(opt.beta2), state[`${p}.v`]), B.mul(c(1 - opt.beta2), B.mul(gp, gp)));
    const denom = B.add(B.div(B.sqrt(v), sqrtBc2), c(opt.eps));
    outputs[p] = B.sub(ids[p], B.mul(stepSize, B.div(m, denom)));
    outputs[`${p}.m`] = m;
    outputs[`${p}.v`] = v;
  }
  return outputs;
}

function adamStateSpec(names, shapes) {
  const spec = [];
  for (const p of names) spec.push([`${p}.m`, shapes[p]], [`${p}.v`, shapes[p]]);
  spec.push(['beta1Pow', []], ['beta2Pow', []]);
  return spec;
}

function adamInitialState(names, shapes) {
  const out = {};
  for (const [name, shape] of adamStateSpec(names, shapes)) out[name] = new Array(count(shape)).fill(name.endsWith('Pow') ? 1 : 0);
  return out;
}

/** Plain SGD as IR ops: p - lr·g. */
function sgdUpdate(B, names, ids, grads, lr) {
  const outputs = {};
  for (const p of names) outputs[p] = B.sub(ids[p], B.mul(B.const(lr), grads[p]));
  return outputs;
}

/**
 * The training step graph. opt: ADAM_3B-like ({kind: 'adam', ...}) or
 * {kind: 'sgd', lr}. Returns { graph, names, stateNames, loss, logits, grads,
 * inputs: {name: id}, outputs: {name: id}, cotangent }.
 */
function buildStep(V, B, cfg, opt) {
  const f = buildForward(V, B, cfg);
  const spec = paramSpec(V, cfg);
  const names = spec.map((s) => s[0]);
  const shapes = {};
  for (const [n, s] of spec) shapes[n] = s;
  const G = grad(f.graph, [f.loss], names.map((n) => f.ids[n]));
  const g = G.graph;
  const grads = {};
  names.forEach((n, k) => { grads[n] = G.grads[k]; });
  const state = {};
  let outputs;
  if (opt.kind === 'adam') {
    for (const [name, shape] of adamStateSpec(names, shapes)) state[name] = g.input(name, shape);
    outputs = adamUpdate(g, names, f.ids, grads, state, opt);
  } else {
    outputs = sgdUpdate(g, names, f.ids, grads, opt.lr);
  }
  const inputs = {};
  for (const n of names) inputs[n] = f.ids[n];
  inputs.x = f.ids.x;
  inputs.y = f.ids.y;
  Object.assign(inputs, state);
  return { graph: g, names, stateNames: Object.keys(state), loss: f.loss, logits: f.logits, grads, inputs, outputs,
    cotangent: G.cotangents[0], shapes };
}

/** One-hot x and y [B·T, V] for sequences of T + 1 tokens (m3b/data.js:62-72): targets are x[t+1]. */
function encodeBatch(seqs, V, T) {
  const x = new Float32Array(seqs.length * T * V), y = new Float32Array(seqs.length * T * V);
  seqs.forEach((s, b) => {
    for (let t = 0; t < T; t++) {
      x[(b * T + t) * V + s[t]] = 1;
      y[(b * T + t) * V + s[t + 1]] = 1;
    }
  });
  return { x, y };
}

module.exports = { REFERENCE_CONFIG, C5_CONFIG, ADAM_3B, paramSpec, initParams, initNormal, causalMask, buildForward,
  buildStep, adamUpdate, adamInitialState, adamStateSpec, sgdUpdate, encodeBatch, logitsOf, lossOf };
