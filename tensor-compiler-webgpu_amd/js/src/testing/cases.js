'use strict';
// The hand-built graphs of the reference's exported cases (softmax and
// logSoftmax composites, a two-layer MLP with NLL loss, single-head attention,
// non-involutive transposes), built here with this host's builder so that a
// test can require their JSON to equal the reference's golden/cases.json
// entries node for node (src/testing/cases.js:54-112 in
// abho7/tensor-compiler-webgpu lists them).

const { Graph } = require('../ir/graph');

function builderCases() {
  const out = [];
  const composites = [
    ['softmax', [5], 0, 3], ['softmax', [3, 4], 1, 3], ['softmax', [3, 4], 0, 3], ['softmax', [2, 3, 4], 1, 3],
    ['logSoftmax', [5], 0, 3], ['logSoftmax', [3, 4], 1, 3], ['logSoftmax', [2, 3, 4], 2, 3],
    ['softmax', [2, 6], 1, 800], ['logSoftmax', [2, 6], 1, 800],
  ];
  for (const [fn, shape, axis, scale] of composites) {
    const g = new Graph();
    const x = g.input('x', shape);
    const y = g[fn](x, axis);
    out.push({ name: `${fn}-${shape.join('x')}-axis${axis}${scale === 800 ? '-large' : ''}`, graph: g.toJSON(), outputs: [y] });
  }
  {
    const g = new Graph();
    const x = g.input('x', [4, 3]);
    const w1 = g.input('w1', [3, 5]);
    const b1 = g.input('b1', [5]);
    const w2 = g.input('w2', [5, 3]);
    const b2 = g.input('b2', [3]);
    const onehot = g.const([1, 0, 0, 0, 0, 1, 0, 1, 0, 1, 0, 0], [4, 3]);
    const h = g.relu(g.add(g.matmul(x, w1), b1));
    const logp = g.logSoftmax(g.add(g.matmul(h, w2), b2), 1);
    const loss = g.div(g.neg(g.sum(g.sum(g.mul(onehot, logp), 1), 0)), g.const(4));
    out.push({ name: 'mlp-nll', graph: g.toJSON(), outputs: [loss] });
  }
  {
    const g = new Graph();
    const q = g.input('q', [2, 4, 3]);
    const k = g.input('k', [2, 4, 3]);
    const v = g.input('v', [2, 4, 3]);
    const scores = g.mul(g.matmul(q, g.transposeLast2(k)), g.const(1 / Math.sqrt(3)));
    const o = g.matmul(g.softmax(scores, -1), v);
    out.push({ name: 'attention', graph: g.toJSON(), outputs: [o] });
  }
  {
    const g = new Graph();
    const x = g.input('x', [2, 3, 4]);
    const w = g.input('w', [2, 4, 3]);
    const t = g.tanh(g.transpose(x, [2, 0, 1]));
    const back = g.transpose(t, [1, 2, 0]);
    const o = g.matmul(back, w);
    out.push({ name: 'transpose-cycles', graph: g.toJSON(), outputs: [o] });
  }
  return out;
}

module.exports = { builderCases };
