'use strict';
// Reverse-mode differentiation as a graph-to-graph transform.
//
// The backward graph extends a copy of the forward graph (forward ids keep their
// meaning). Each requested output gets an `input` node carrying its cotangent,
// named <prefix><k> in output order. The forward nodes are then visited from the
// last to the first; a visited node's accumulated adjoint is pushed through its
// op's adjoint rule, and each operand's share is added into that operand's
// adjoint (the first share is taken as is, later ones are summed with `add`).
// Only values that depend on a differentiated input take part. The interface
// and the rules are those of the reference's src/autodiff.js (grad :87-127, rule
// table :25-76 in abho7/tensor-compiler-webgpu); the rules build their terms with
// the ordinary builder in a fixed order, because the node sequence of a backward
// graph is what the fusion pass partitions and what the reference's recorded
// fusion counts pin.

const { Graph } = require('./ir/graph');
const { sameShape } = require('./ir/shapes');

class GradientError extends Error {
  constructor(message) { super(message); this.name = 'GradientError'; }
}

/** The permutation that undoes `perm`. */
function inversePermutation(perm) {
  const inv = new Array(perm.length);
  for (let i = 0; i < perm.length; i++) inv[perm[i]] = i;
  return inv;
}

/**
 * Sum an adjoint of broadcast shape `to` back to the operand's shape `from`: the
 * leading axes the broadcast added are summed away one by one (each time axis 0),
 * then every axis stretched from 1 is summed keeping its axis, and the result is
 * reshaped to `from`.
 */
function unbroadcast(B, g, from, to) {
  const added = to.length - from.length;
  let acc = g;
  for (let k = 0; k < added; k++) acc = B.sum(acc, 0, false);
  for (let axis = 0; axis < from.length; axis++) {
    if (from[axis] === 1 && to[added + axis] !== 1) acc = B.sum(acc, axis, true);
  }
  return B.reshape(acc, from);
}

/**
 * Adjoint rules: rule(B, node, g) returns, per operand of the forward `node`, the id
 * of its share of the adjoint `g` (built into B), or null where there is none. The
 * order of the builder calls inside each rule is part of the contract (see above).
 */
const RULES = {
  add: (B, n, g) => [g, g],
  sub: (B, n, g) => [g, B.neg(g)],
  mul: (B, n, g) => {
    const [x, y] = n.inputs;
    const dx = B.mul(g, y);
    return [dx, B.mul(g, x)];
  },
  div: (B, n, g) => {
    const [x, y] = n.inputs;
    const dx = B.div(g, y);
    const num = B.mul(g, x);
    const den = B.mul(y, y);
    return [dx, B.neg(B.div(num, den))];
  },
  neg: (B, n, g) => [B.neg(g)],
  // d exp(x) = exp(x) dx, read from the node's own value.
  exp: (B, n, g) => [B.mul(g, n.id)],
  log: (B, n, g) => [B.div(g, n.inputs[0])],
  relu: (B, n, g) => [B.mul(g, B.step(n.inputs[0]))],
  // d tanh(x) = (1 - y^2) dx with y the node's value.
  tanh: (B, n, g) => {
    const one = B.const(1);
    const ySquared = B.mul(n.id, n.id);
    return [B.mul(g, B.sub(one, ySquared))];
  },
  // d sqrt(x) = dx / (2 y) with y the node's value.
  sqrt: (B, n, g) => {
    const two = B.const(2);
    return [B.div(g, B.mul(two, n.id))];
  },
  // C = A·B: dA = dC·Bᵀ, dB = Aᵀ·dC (transposes of the last two axes).
  matmul: (B, n, g) => {
    const [a, b] = n.inputs;
    const bt = B.transposeLast2(b);
    const da = B.matmul(g, bt);
    const at = B.transposeLast2(a);
    return [da, B.matmul(at, g)];
  },
  // A reduction's adjoint comes back along the reduced axis.
  sum: (B, n, g) => {
    const inShape = B.shape(n.inputs[0]);
    const withAxis = inShape.map((d, i) => (i === n.attrs.axis ? 1 : d));
    return [B.broadcast(B.reshape(g, withAxis), inShape)];
  },
  broadcast: (B, n, g) => [unbroadcast(B, g, B.shape(n.inputs[0]), n.shape)],
  reshape: (B, n, g) => [B.reshape(g, B.shape(n.inputs[0]))],
  transpose: (B, n, g) => [B.transpose(g, inversePermutation(n.attrs.perm))],
  step: () => [null],
  stopGradient: () => [null],
  max: () => {
    throw new GradientError('max is not differentiable here: put it under stopGradient where its gradient vanishes (the softmax shift does)');
  },
};

/** 1 for every node whose value depends on one of `wrt` (the nodes themselves included). */
function dependents(graph, wrt) {
  const mark = new Uint8Array(graph.nodes.length);
  for (const id of wrt) mark[id] = 1;
  for (const node of graph.nodes) {
    if (!mark[node.id] && node.inputs.some((i) => mark[i])) mark[node.id] = 1;
  }
  return mark;
}

/**
 * The gradient graph of `graph` for `outputs` with respect to `wrt` (node ids).
 * Options: rules (a replacement rule table), prefix (of the cotangent inputs, 'd').
 * Returns { graph, cotangents, grads }: the extended graph, the name of the input
 * that feeds each output's cotangent, and the id of each gradient in `wrt` order (a
 * constant zero of the node's shape where no output depends on it).
 */
function grad(graph, outputs, wrt, options) {
  const o = options || {};
  const rules = o.rules || RULES;
  const prefix = o.prefix === undefined ? 'd' : o.prefix;
  const B = graph.clone();
  const live = dependents(graph, wrt);
  const adjoint = new Array(graph.nodes.length).fill(null);
  const addShare = (id, share) => {
    const want = graph.nodes[id].shape;
    const got = B.shape(share);
    if (!sameShape(got, want)) {
      throw new GradientError(`adjoint of node ${id}: a share of shape [${got}] for a value of shape [${want}]`);
    }
    adjoint[id] = adjoint[id] === null ? share : B.add(adjoint[id], share);
  };
  const cotangents = outputs.map((id, k) => {
    const name = `${prefix}${k}`;
    addShare(id, B.input(name, graph.nodes[id].shape));
    return name;
  });
  for (let id = graph.nodes.length - 1; id >= 0; id--) {
    const node = graph.nodes[id];
    if (adjoint[id] === null || !live[id] || !node.inputs.some((i) => live[i])) continue;
    const rule = rules[node.op];
    if (!rule) throw new GradientError(`no adjoint rule for op '${node.op}'`);
    const shares = rule(B, node, adjoint[id]);
    node.inputs.forEach((operand, k) => {
      if (shares[k] !== null && live[operand]) addShare(operand, shares[k]);
    });
  }
  const grads = wrt.map((id) => (adjoint[id] !== null ? adjoint[id] : B.const(0, graph.nodes[id].shape.slice())));
  return { graph: B, cotangents, grads };
}

module.exports = { grad, RULES, GradientError, Graph };
