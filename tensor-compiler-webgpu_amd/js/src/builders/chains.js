'use strict';
// Benchmark config 2: seeded random elementwise programs of 8–16 ops over
// [R, C] fp32 tensors (R 8192, C 1024 at full size), drawn from add, sub, mul,
// div, neg, exp, log, relu, tanh, step and the broadcast of a [C] row vector.
// Inputs are N(0, 1). log and div operands are made positive the way the
// config says — through exp(·) or |·| + 1, with |v| built from IR ops as
// relu(v) + relu(-v) — and an interval of every value is tracked so that exp
// only sees arguments below 20: every program stays finite. A value downstream
// of `step` is marked coarse — where step's input lies within its own float32
// error of zero the budget lets the output flip between 0 and 1 — and log is
// never taken of a coarse value (its argument could then lie within its error
// of zero, an unbounded error), so every element of every program is
// judgeable. Each program is also differentiated (autodiff's gradient graph
// with respect to every input, cotangent N(0, 1)).
//
// The reference's own chains are fixed cycles (src/fusion/direct-cases-m4.js:38-44,
// workloads.js:60-65) and its random generator caps tensors at 96 elements;
// this generator is this backend's own.

const { Graph } = require('../ir/graph');
const { grad } = require('../autodiff');
const { Rng } = require('../testing/rng');

const OPS = ['add', 'sub', 'mul', 'div', 'neg', 'exp', 'log', 'relu', 'tanh', 'step', 'broadcast'];

/** One program: { graph, output, inputs: names, ops (the drawn op sequence) }. */
function chainProgram(seed, R, C) {
  const rng = new Rng((seed * 2654435761 + 7) >>> 0);
  const g = new Graph();
  const x0 = g.input('x0', [R, C]);
  const x1 = g.input('x1', [R, C]);
  const r = g.input('r', [C]);
  // Each value carries an interval [lo, hi] of what it can hold (inputs N(0,1): |x| < 6 is
  // the interval used; a draw beyond it only makes exp smaller than allowed, never larger).
  let v = { id: x0, lo: -6, hi: 6 };
  const other = () => (rng.chance(0.5) ? { id: x1, lo: -6, hi: 6 } : { id: r, lo: -6, hi: 6, row: true });
  const absPlus1 = (w) => {
    const a = g.add(g.add(g.relu(w.id), g.relu(g.neg(w.id))), g.const(1));
    return { id: a, lo: 1, hi: 1 + Math.max(Math.abs(w.lo), Math.abs(w.hi)) };
  };
  const positive = (w) => (w.hi < 20 && rng.chance(0.5)
    ? { id: g.exp(w.id), lo: Math.exp(w.lo), hi: Math.exp(w.hi) }
    : absPlus1(w));
  const L = rng.int(8, 16);
  const ops = [];
  let count = 0;
  while (count < L) {
    const op = rng.pick(OPS);
    const before = g.nodes.length;
    const coarse = !!v.coarse;
    if (op === 'log' && coarse) v = { id: g.tanh(v.id), lo: Math.tanh(v.lo), hi: Math.tanh(v.hi) };
    else if (op === 'neg') v = { id: g.neg(v.id), lo: -v.hi, hi: -v.lo };
    else if (op === 'relu') v = { id: g.relu(v.id), lo: Math.max(0, v.lo), hi: Math.max(0, v.hi) };
    else if (op === 'tanh') v = { id: g.tanh(v.id), lo: Math.tanh(v.lo), hi: Math.tanh(v.hi) };
    else if (op === 'step') v = { id: g.step(v.id), lo: 0, hi: 1 };
    else if (op === 'exp') {
      if (v.hi >= 20) v = { id: g.tanh(v.id), lo: Math.tanh(v.lo), hi: Math.tanh(v.hi) };
      v = { id: g.exp(v.id), lo: Math.exp(v.lo), hi: Math.exp(v.hi) };
    } else if (op === 'log') {
      const p = positive(v);
      v = { id: g.log(p.id), lo: Math.log(p.lo), hi: Math.log(p.hi) };
    } else if (op === 'add' || op === 'sub' || op === 'mul' || op === 'broadcast') {
      // 'broadcast' draws the row vector as the other operand of a binary op.
      const w = op === 'broadcast' ? { id: r, lo: -6, hi: 6 } : other();
      const bop = op === 'broadcast' ? rng.pick(['add', 'sub', 'mul']) : op;
      const id = g[bop](v.id, w.id);
      const c = bop === 'add' ? [v.lo + w.lo, v.hi + w.hi] : bop === 'sub' ? [v.lo - w.hi, v.hi - w.lo]
        : [v.lo * w.lo, v.lo * w.hi, v.hi * w.lo, v.hi * w.hi];
      v = { id, lo: Math.min.apply(null, c), hi: Math.max.apply(null, c) };
    } else if (op === 'div') {
      const d = positive(other());
      const c = [v.lo / d.lo, v.lo / d.hi, v.hi / d.lo, v.hi / d.hi];
      v = { id: g.div(v.id, d.id), lo: Math.min.apply(null, c), hi: Math.max.apply(null, c) };
    }
    v.coarse = coarse || op === 'step';
    // Keep magnitudes moderate: squash when the interval grows large.
    if (Math.max(Math.abs(v.lo), Math.abs(v.hi)) > 1e3) v = { id: g.tanh(v.id), lo: Math.tanh(v.lo), hi: Math.tanh(v.hi), coarse: v.coarse };
    ops.push(op);
    count++;
    if (g.nodes.length === before) throw new Error('chain generator made no node');
  }
  return { graph: g, output: v.id, inputs: ['x0', 'x1', 'r'], ops };
}

/** Forward and gradient graphs of program `seed`, with the ids to keep. */
function chainWorkload(seed, R, C) {
  const p = chainProgram(seed, R, C);
  const ids = p.graph.inputs().map((n) => n.id);
  const G = grad(p.graph, [p.output], ids);
  return {
    seed, ops: p.ops,
    forward: { graph: p.graph, keep: [p.output], outputs: [p.output] },
    gradient: { graph: G.graph, keep: [p.output].concat(G.grads), outputs: [p.output].concat(G.grads), cotangent: G.cotangents[0] },
  };
}

/** Inputs for program graphs: x0, x1 [R, C], r [C] ~ N(0,1), and the cotangent d0 ~ N(0,1). */
function chainInputs(seed, R, C) {
  const rng = new Rng((seed * 40503 + 11) >>> 0);
  return { x0: rng.normalF32(R * C, 1), x1: rng.normalF32(R * C, 1), r: rng.normalF32(C, 1), d0: rng.normalF32(R * C, 1) };
}

module.exports = { chainProgram, chainWorkload, chainInputs, OPS };
