'use strict';
// Graphs and seeded inputs of benchmark configs 3 and 4, shared by the bench and
// by the parity runs, so that both see the same values.
//
//   config 3  softmax / logSoftmax over x [R, C] (full size [16384, 4096]),
//             x ~ N(0, 4) (std 2), the first 1 % of a seeded permutation of the
//             rows shifted by +800, cotangent dy ~ N(0, 1); forward graph keeps y,
//             gradient graph keeps y and dx.
//   config 4  act(X[M,K] · W[K,N] + bias[N]), act in {relu, tanh}; X, W ~ N(0, 1/K)
//             (variance 1/K), bias ~ N(0, 0.1) (variance 0.1), cotangent
//             dY ~ N(0, 1); gradient graph keeps y, dX, dW, dbias.
//
// The graphs come from the restated builder and autodiff (src/ir/graph.js,
// src/autodiff.js of the reference), the composites from graph.js:133-146.

const { Graph } = require('../ir/graph');
const { grad } = require('../autodiff');
const { Rng } = require('../testing/rng');

const C3_SHAPE = [16384, 4096];
const C4_SHAPES = [[512, 512, 512], [4096, 4096, 4096], [8192, 1024, 4096]];

/** Config 3's inputs at [R, C]: { x, dy, shifted (row ids) }. */
function c3Inputs(R, C) {
  const rng = new Rng(3);
  const x = rng.normalF32(R * C, 2);
  const shifted = rng.shuffle(Array.from({ length: R }, (_, i) => i)).slice(0, Math.round(R / 100));
  for (const r of shifted) for (let c = 0; c < C; c++) x[r * C + c] += 800;
  const dy = rng.normalF32(R * C, 1);
  return { x, dy, shifted };
}

/** Config 3's forward and gradient graphs for `fn` ('softmax' | 'logSoftmax') at [R, C]. */
function c3Graphs(fn, R, C) {
  const g = new Graph();
  const xi = g.input('x', [R, C]);
  const y = g[fn](xi, 1);
  const G = grad(g, [y], [xi]);
  return {
    forward: { graph: g, keep: [y], inputs: ['x'] },
    gradient: { graph: G.graph, keep: [y, G.grads[0]], inputs: ['x', 'd0'] },
  };
}

/** Config 4's inputs at (M, K, N): { X, W, bias, dY }. */
function c4Inputs(M, K, N) {
  const rng = new Rng(M * 7 + K * 3 + N);
  const X = rng.normalF32(M * K, 1 / Math.sqrt(K));
  const W = rng.normalF32(K * N, 1 / Math.sqrt(K));
  const bias = rng.normalF32(N, Math.sqrt(0.1));
  const dY = rng.normalF32(M * N, 1);
  return { X, W, bias, dY };
}

/** Config 4's forward and gradient graphs for `act` ('relu' | 'tanh') at (M, K, N). */
function c4Graphs(act, M, K, N) {
  const g = new Graph();
  const xi = g.input('X', [M, K]), wi = g.input('W', [K, N]), bi = g.input('bias', [N]);
  const y = g[act](g.add(g.matmul(xi, wi), bi));
  const G = grad(g, [y], [xi, wi, bi]);
  return {
    forward: { graph: g, keep: [y] },
    gradient: { graph: G.graph, keep: [y].concat(G.grads), grads: G.grads },
  };
}

module.exports = { C3_SHAPE, C4_SHAPES, c3Inputs, c3Graphs, c4Inputs, c4Graphs };
