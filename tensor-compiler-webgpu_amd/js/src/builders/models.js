'use strict';
// The training steps of the benchmark's model configs (1 and 5), with their data:
//   mlp            config 1: X [128, 64], 64 -> 128 tanh -> 10, log-softmax CE, SGD 0.1
//   transformer    config 5: V 96, d 256, H 4, L 4, ff 1024 ReLU, T 128, batch B (64 at
//                  full size), N(0, 0.02) weights from seed 0, plain SGD (lr 0.05)
//   transformer-ref the reference's own model (V 16, T 64, d 64, L 2, ff 256 GELU, Adam,
//                  uniform init from its seeding), the config its PyTorch goldens use
// Token ids are uniform in 0..V-1; targets are the next token (x[t+1]).

const tf = require('./transformer');
const mlp = require('./mlp');
const { Rng } = require('../testing/rng');

const C5_LR = 0.05;

/** Sequences of T + 1 uniform token ids in 0..V-1 for batch `b` of `seed`. */
function randomTokens(B, T, V, seed) {
  const rng = new Rng((seed * 9176 + 5) >>> 0);
  const seqs = [];
  for (let b = 0; b < B; b++) {
    const s = new Array(T + 1);
    for (let t = 0; t <= T; t++) s[t] = rng.int(0, V - 1);
    seqs.push(s);
  }
  return seqs;
}

/**
 * { step, params, state, batch(k) -> {x, y}, info } for a model request
 * { model, B?, V?, seed?, cfg? (overrides of the transformer config), firstBatch?, batches? }.
 */
function modelStep(req) {
  const model = req.model || 'mlp';
  if (model === 'mlp') {
    const c = Object.assign({}, mlp.C1, req.cfg || {});
    const step = mlp.buildMlpStep(c);
    const d = mlp.mlpData(c);
    return { step, params: d.params, state: {}, batch: () => ({ x: d.x, y: d.y }), info: { config: 'C1', cfg: c } };
  }
  if (model === 'transformer') {
    const cfg = Object.assign({}, tf.C5_CONFIG, req.cfg || {});
    const V = req.V || 96, B = req.B || 64, seed = req.seed || 0;
    const lr = req.lr || C5_LR;
    const step = tf.buildStep(V, B, cfg, { kind: 'sgd', lr });
    const params = tf.initNormal(V, seed, 0.02, cfg);
    const batch = (k) => tf.encodeBatch(randomTokens(B, cfg.T, V, seed * 1000 + (k || 0)), V, cfg.T);
    return { step, params, state: {}, batch, info: { config: 'C5', V, B, cfg, lr, init: 'N(0, 0.02) weights, LayerNorm gains 1 and biases 0' } };
  }
  if (model === 'transformer-ref') {
    const cfg = Object.assign({}, tf.REFERENCE_CONFIG, req.cfg || {});
    const V = req.V || 16, B = req.B || 4, seed = req.seed || 1;
    const step = tf.buildStep(V, B, cfg, tf.ADAM_3B);
    const params = tf.initParams(V, seed, cfg);
    const spec = tf.paramSpec(V, cfg);
    const shapes = {};
    for (const [n, s] of spec) shapes[n] = s;
    const state = tf.adamInitialState(step.names, shapes);
    // `batches`: every step's sequences given (a golden run's schedule); else `firstBatch`
    // for step 0 and seeded random tokens after.
    const batch = (k) => (req.batches ? tf.encodeBatch(req.batches[(k || 0) % req.batches.length], V, cfg.T)
      : req.firstBatch && !k ? tf.encodeBatch(req.firstBatch, V, cfg.T)
        : tf.encodeBatch(randomTokens(B, cfg.T, V, seed * 1000 + (k || 0)), V, cfg.T));
    return { step, params, state, batch, info: { config: 'reference transformer', V, B, cfg } };
  }
  throw new Error(`unknown model '${model}'`);
}

/**
 * { fwd, params, batch(k) -> {x, y}, info } for a forward-pass request { model, B?, V?, seed?,
 * firstBatch? }: the transformer's forward graph (logits and loss from the parameters) with
 * the same parameters and batches as modelStep's.
 */
function modelForward(req) {
  const model = req.model || 'transformer-ref';
  if (model !== 'transformer' && model !== 'transformer-ref') throw new Error(`no forward pass for model '${model}'`);
  const ref = model === 'transformer-ref';
  const cfg = Object.assign({}, ref ? tf.REFERENCE_CONFIG : tf.C5_CONFIG, req.cfg || {});
  const V = req.V || (ref ? 16 : 96), B = req.B || (ref ? 4 : 64), seed = req.seed || (ref ? 1 : 0);
  const fwd = tf.buildForward(V, B, cfg);
  const params = ref ? tf.initParams(V, seed, cfg) : tf.initNormal(V, seed, 0.02, cfg);
  const batch = (k) => (req.firstBatch && !k ? tf.encodeBatch(req.firstBatch, V, cfg.T)
    : tf.encodeBatch(randomTokens(B, cfg.T, V, seed * 1000 + (k || 0)), V, cfg.T));
  return { fwd, params, batch, info: { config: ref ? 'reference transformer' : 'C5', V, B, cfg } };
}

module.exports = { modelStep, modelForward, randomTokens, C5_LR };
