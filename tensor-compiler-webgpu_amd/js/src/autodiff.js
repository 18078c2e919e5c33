'use strict';
// Reverse-mode differentiation as a graph-to-graph transform.
//
// grad() copies the forward graph, adds one `input` per output for its
// cotangent (named d0, d1, ...), then walks the forward nodes from last to
// first, applying each op's rule to the cotangent accumulated so far and
// summing contributions with `add`. This is the construction of
// src/autodiff.js in abho7/tensor-compiler-webgpu (RULES :25-76, grad :87-127),
// kept node for node because the backward graphs it emits (transposed matmul
// operands, row sums for broadcasts, step masks) are what the MI355X lowering
// is asked to run, and their node order fixes what the fusion pass groups.

const { Graph } = require('./ir/graph');
const { sameShape } = require('./ir/shapes');

class GradientError extends Error {
  constructor(message) { super(message); this.name = 'GradientError'; }
}

/** Per-op rules: (G, node, gy) -> one contribution id (or null) per input. */
const RULES = {
  add: (G, n, gy) => [gy, gy],
  sub: (G, n, gy) => [gy, G.neg(gy)],
  mul: (G, n, gy) => {
    const a = n.inputs[0], b = n.inputs[1];
    return [G.mul(gy, b), G.mul(gy, a)];
  },
  div: (G, n, gy) => {
    const a = n.inputs[0], b = n.inputs[1];
    const first = G.div(gy, b);
    return [first, G.neg(G.div(G.mul(gy, a), G.mul(b, b)))];
  },
  neg: (G, n, gy) => [G.neg(gy)],
  exp: (G, n, gy) => [G.mul(gy, n.id)],
  log: (G, n, gy) => [G.div(gy, n.inputs[0])],
  relu: (G, n, gy) => [G.mul(gy, G.step(n.inputs[0]))],
  tanh: (G, n, gy) => {
    const one = G.const(1);
    return [G.mul(gy, G.sub(one, G.mul(n.id, n.id)))];
  },
  sqrt: (G, n, gy) => {
    const two = G.const(2);
    return [G.div(gy, G.mul(two, n.id))];
  },
  matmul: (G, n, gy) => {
    const a = n.inputs[0], b = n.inputs[1];
    const da = G.matmul(gy, G.transposeLast2(b));
    const db = G.matmul(G.transposeLast2(a), gy);
    return [da, db];
  },
  sum: (G, n, gy) => {
    const xs = G.shape(n.inputs[0]);
    const kept = xs.map((d, i) => (i === n.attrs.axis ? 1 : d));
    return [G.broadcast(G.reshape(gy, kept), xs)];
  },
  broadcast: (G, n, gy) => {
    const xs = G.shape(n.inputs[0]);
    const lead = n.shape.length - xs.length;
    let g = gy;
    for (let i = 0; i < lead; i++) g = G.sum(g, 0, false);
    xs.forEach((d, i) => {
      if (d === 1 && n.shape[lead + i] !== 1) g = G.sum(g, i, true);
    });
    return [G.reshape(g, xs)];
  },
  reshape: (G, n, gy) => [G.reshape(gy, G.shape(n.inputs[0]))],
  transpose: (G, n, gy) => {
    const inverse = [];
    n.attrs.perm.forEach((p, i) => { inverse[p] = i; });
    return [G.transpose(gy, inverse)];
  },
  step: () => [null],
  stopGradient: () => [null],
  max: () => {
    throw new GradientError('max has no gradient; wrap it in stopGradient where its gradient is zero (as softmax does)');
  },
};

/**
 * The gradient graph of `graph` for `outputs` with respect to `wrt` (node ids).
 * Returns { graph, cotangents, grads }: forward ids are kept, `cotangents`
 * names the input fed each output's cotangent, `grads` is the id of each
 * gradient in `wrt` order (a constant zero where no output depends on it).
 */
function grad(graph, outputs, wrt, options) {
  const rules = (options && options.rules) || RULES;
  const prefix = (options && options.prefix) || 'd';
  const G = graph.clone();
  const forwardCount = graph.nodes.length;
  const dependsOnWrt = new Array(forwardCount).fill(false);
  for (const id of wrt) dependsOnWrt[id] = true;
  for (const node of graph.nodes) {
    if (node.inputs.some((i) => dependsOnWrt[i])) dependsOnWrt[node.id] = true;
  }
  const cot = new Array(forwardCount).fill(null);
  const accumulate = (id, contribution) => {
    if (!sameShape(G.shape(contribution), graph.nodes[id].shape)) {
      throw new GradientError(`gradient for node ${id} has shape [${G.shape(contribution)}], value has [${graph.nodes[id].shape}]`);
    }
    cot[id] = cot[id] === null ? contribution : G.add(cot[id], contribution);
  };
  const cotangents = outputs.map((id, i) => {
    const name = `${prefix}${i}`;
    accumulate(id, G.input(name, graph.nodes[id].shape));
    return name;
  });
  for (let id = forwardCount - 1; id >= 0; id--) {
    const node = graph.nodes[id];
    if (cot[id] === null || !dependsOnWrt[id] || node.inputs.length === 0) continue;
    if (!node.inputs.some((i) => dependsOnWrt[i])) continue;
    const rule = rules[node.op];
    if (!rule) throw new GradientError(`no gradient rule for '${node.op}'`);
    const contributions = rule(G, node, cot[id]);
    node.inputs.forEach((input, k) => {
      if (contributions[k] !== null && dependsOnWrt[input]) accumulate(input, contributions[k]);
    });
  }
  const grads = wrt.map((id) => (cot[id] !== null ? cot[id] : G.const(0, graph.nodes[id].shape.slice())));
  return { graph: G, cotangents, grads };
}

module.exports = { grad, RULES, GradientError, Graph };
