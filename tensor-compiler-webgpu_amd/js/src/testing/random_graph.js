'use strict';
// Seeded random well-typed programs: the fuzzing corpus of the reference
// (src/testing/random-graph.js, "version 2", in abho7/tensor-compiler-webgpu).
//
// The corpus has to be the reference's program for program, because its
// recorded counts — golden/cases.json's 40 v2 graphs, and the fusion pass's
// results over corpus programs 1..2000 in golden/measurements.json m4 — pin this
// backend's builder, autodiff and fusion pass. So the construction follows the
// reference's steps and draws from the same generator (mulberry32, ../rng) in
// the same order: every value carries an interval sound for inputs in [-2, 2];
// log, div and exp are emitted only where the interval proves them safe (the
// operand wrapped as x*x + c, exp of something bounded, or tanh otherwise); an
// op whose result could exceed BOUND in magnitude is discarded with every node
// it emitted; programs are either general (weighted op choices over a pool that
// favours recent values) or targeted at one op (matmul, transpose, reshape,
// broadcast, sum); every computed value nothing consumes is an output.

const { Graph } = require('../ir/graph');
const { broadcastShapes, size } = require('../ir/shapes');
const { Rng } = require('./rng');

const MAX_SIZE = 96;
const BOUND = 1e3;
const INPUT_RANGE = [-2, 2];

/** Relative weights of the general generator's ops (random-graph.js:38-41). */
const GENERATED = {
  add: 3, sub: 3, mul: 3, div: 3, neg: 1, exp: 2, log: 2, relu: 3, tanh: 2,
  matmul: 4, sum: 3, broadcast: 2, reshape: 3, transpose: 3, softmax: 2, logSoftmax: 2,
};

/** Ops with a targeted generator (random-graph.js:44). */
const TARGETS = ['matmul', 'transpose', 'reshape', 'broadcast', 'sum'];

const last = (a) => a[a.length - 1];

function mulIv(x, y) {
  const p = [x[0] * y[0], x[0] * y[1], x[1] * y[0], x[1] * y[1]];
  return [Math.min(p[0], p[1], p[2], p[3]), Math.max(p[0], p[1], p[2], p[3])];
}

const magnitude = (iv) => Math.max(Math.abs(iv[0]), Math.abs(iv[1]));

/** The interval of node `id` from its inputs' intervals (sound, not tight). */
function interval(g, id, iv, squareAware) {
  const n = g.nodes[id];
  const a = n.inputs.length > 0 ? iv.get(n.inputs[0]) : undefined;
  const b = n.inputs.length > 1 ? iv.get(n.inputs[1]) : undefined;
  switch (n.op) {
    case 'input': return INPUT_RANGE.slice();
    case 'const': {
      const v = n.attrs.value;
      if (typeof v === 'number') return [v, v];
      let lo = Infinity, hi = -Infinity;
      for (const x of v) { if (x < lo) lo = x; if (x > hi) hi = x; }
      return [lo, hi];
    }
    case 'add': return [a[0] + b[0], a[1] + b[1]];
    case 'sub': return [a[0] - b[1], a[1] - b[0]];
    case 'mul':
      if (squareAware && n.inputs[0] === n.inputs[1]) {
        const m = magnitude(a);
        const lo = a[0] <= 0 && a[1] >= 0 ? 0 : Math.min(a[0] * a[0], a[1] * a[1]);
        return [lo, m * m];
      }
      return mulIv(a, b);
    case 'div':
      if (b[0] <= 0 && b[1] >= 0) return [-Infinity, Infinity];
      return mulIv(a, [1 / b[1], 1 / b[0]]);
    case 'neg': return [-a[1], -a[0]];
    case 'exp': return [Math.exp(a[0]), Math.exp(a[1])];
    case 'log': return a[0] > 0 ? [Math.log(a[0]), Math.log(a[1])] : [-Infinity, Infinity];
    case 'relu': return [Math.max(0, a[0]), Math.max(0, a[1])];
    case 'step': return [0, 1];
    case 'tanh': return [Math.tanh(a[0]), Math.tanh(a[1])];
    case 'sqrt': return a[0] >= 0 ? [Math.sqrt(a[0]), Math.sqrt(a[1])] : [-Infinity, Infinity];
    case 'matmul': {
      const k = last(g.shape(n.inputs[0]));
      const p = mulIv(a, b);
      return [k * p[0], k * p[1]];
    }
    case 'sum': {
      const len = g.shape(n.inputs[0])[n.attrs.axis];
      return [len * a[0], len * a[1]];
    }
    case 'max': case 'stopGradient': case 'broadcast': case 'reshape': case 'transpose':
      return a.slice();
    default: throw new Error(`no interval rule for ${n.op}`);
  }
}

const round1024 = (v) => Math.round(v * 1024) / 1024;

/** Every ordered factorisation of n into `rank` factors, smallest first factor first. */
function factorizations(n, rank) {
  if (rank === 1) return [[n]];
  const out = [];
  for (let d = 1; d <= n; d++) {
    if (n % d) continue;
    for (const rest of factorizations(n / d, rank - 1)) out.push([d].concat(rest));
  }
  return out;
}

const isInvolution = (perm) => perm.every((p, i) => perm[p] === i);
const sameShape = (a, b) => a.length === b.length && a.every((d, i) => d === b[i]);

class ProgramBuilder {
  constructor(rng) {
    this.rng = rng;
    this.g = new Graph();
    this.iv = new Map();
    this.pool = [];
    this.leaves = 0;
    this.strict = false;        // targeted programs: no size-1 dims, matmul's B always an input
    this.f32 = false;           // float32 guards (exp arguments kept above -40)
    this.squareAware = false;
    this.operand = undefined;
  }

  /** Give every node up to `id` its interval (helpers may have emitted nodes in between). */
  track(id) {
    if (!this.iv.has(id)) {
      for (let i = 0; i <= id; i++) if (!this.iv.has(i)) this.iv.set(i, interval(this.g, i, this.iv, this.squareAware));
    }
    return id;
  }

  ok(id) { return magnitude(this.iv.get(this.track(id))) <= BOUND; }

  dim() {
    if (this.strict) return this.rng.int(2, 5);
    return this.rng.chance(0.2) ? 1 : this.rng.int(2, 6);
  }

  shape(minRank, maxRank) {
    const lo = minRank === undefined ? 0 : minRank, hi = maxRank === undefined ? 4 : maxRank;
    for (;;) {
      const rank = this.rng.int(lo, hi);
      const s = [];
      for (let i = 0; i < rank; i++) s.push(this.dim());
      if (size(s) <= MAX_SIZE) return s;
    }
  }

  input(shape) { return this.push(this.g.input(`x${this.leaves++}`, shape)); }

  leaf(shape) {
    if (this.rng.chance(0.7)) return this.input(shape);
    return this.push(this.g.const(this.rng.array(size(shape), -2, 2).map(round1024), shape));
  }

  push(id) { this.track(id); this.pool.push(id); return id; }

  /** A pool value passing `filter`, favouring recent ones (r² skews toward the end). */
  choose(filter) {
    const f = filter || (() => true);
    const c = this.pool.filter((id) => f(this.g.shape(id), id));
    if (c.length === 0) return undefined;
    const r = this.rng.next();
    return c[c.length - 1 - Math.floor(r * r * c.length)];
  }

  /** The op's first operand: the forced one when given (if it passes `filter`), else chosen. */
  first(filter) {
    const f = filter || (() => true);
    if (this.operand === undefined) return this.choose(f);
    return f(this.g.shape(this.operand), this.operand) ? this.operand : undefined;
  }

  scalarConst(lo, hi) { return this.track(this.g.const(round1024(this.rng.uniform(lo, hi)))); }

  safeDenominator(x) {
    const [lo, hi] = this.iv.get(x);
    if (lo >= 0.1 || hi <= -0.1) return x;
    const r = this.rng.next();
    const g = this.g;
    if (r < 0.4) return this.track(g.add(g.mul(x, x), this.scalarConst(0.2, 1)));
    if (r < 0.6) return this.track(g.neg(g.add(g.mul(x, x), this.scalarConst(0.2, 1))));
    return this.track(g.exp(this.boundedForExp(x)));
  }

  boundedForExp(x) {
    const [lo, hi] = this.iv.get(x);
    return hi <= 4 && (!this.f32 || lo >= -40) ? x : this.track(this.g.tanh(x));
  }

  safeSqrtArgument(x) {
    if (this.iv.get(x)[0] >= 0.1) return x;
    return this.track(this.g.add(this.g.exp(this.boundedForExp(x)), this.scalarConst(0.2, 1)));
  }

  safeLogArgument(x) {
    if (this.iv.get(x)[0] >= 0.1) return x;
    const g = this.g;
    return this.rng.chance(0.6)
      ? this.track(g.add(g.mul(x, x), this.scalarConst(0.2, 1)))
      : this.track(g.exp(this.boundedForExp(x)));
  }

  /** A partner for a binary op with x: an existing broadcast-compatible value, or a new leaf. */
  partner(x) {
    const xs = this.g.shape(x);
    const b = this.rng.chance(0.5)
      ? this.choose((s) => { const o = broadcastShapes(xs, s); return !!o && size(o) <= MAX_SIZE; })
      : undefined;
    if (b !== undefined) return b;
    const drop = this.rng.chance(0.3) ? this.rng.int(0, xs.length) : 0;
    return this.leaf(xs.slice(drop).map((d) => (this.rng.chance(0.3) ? 1 : d)));
  }

  apply(op, operand) {
    const { g, rng } = this;
    this.operand = operand;
    switch (op) {
      case 'add': case 'sub': case 'mul': {
        const a = this.first();
        return g[op](a, this.partner(a));
      }
      case 'div': {
        const a = this.first();
        return g.div(a, this.safeDenominator(this.partner(a)));
      }
      case 'log': return g.log(this.safeLogArgument(this.first()));
      case 'exp': return g.exp(this.boundedForExp(this.first()));
      case 'sqrt': return g.sqrt(this.safeSqrtArgument(this.first()));
      case 'neg': case 'relu': case 'tanh': return g[op](this.first());
      case 'matmul': return this.matmul(this.first());
      case 'sum': {
        const x = this.first((s) => s.length >= 1);
        return x === undefined ? undefined : g.sum(x, rng.int(0, g.shape(x).length - 1), rng.chance(0.4));
      }
      case 'softmax': case 'logSoftmax': {
        const x = this.first((s) => s.length >= 1);
        return x === undefined ? undefined : g[op](x, rng.int(0, g.shape(x).length - 1));
      }
      case 'broadcast': return this.broadcast(this.first());
      case 'reshape': return this.reshape(this.first());
      case 'transpose': {
        const x = this.first((s) => s.length >= 2);
        return x === undefined ? undefined : this.transpose(x);
      }
      default: throw new Error(`generator has no case for '${op}'`);
    }
  }

  matmul(a0) {
    const { g, rng } = this;
    let a = a0;
    let as = g.shape(a);
    if (as.length < 2) {
      const options = factorizations(size(as), 2);
      const square = options.filter(([m, k]) => m > 1 && k > 1);
      a = this.track(g.reshape(a, rng.pick(square.length && rng.chance(0.8) ? square : options)));
      as = g.shape(a);
    }
    const batch = as.slice(0, -2);
    const k = last(as), m = as[as.length - 2];
    const n = this.dim();
    if (size(batch.concat([m, n])) > MAX_SIZE || size(batch.concat([k, n])) > MAX_SIZE) return undefined;
    const fits = (s) => s.length === as.length && s[s.length - 2] === k && batch.every((d, i) => d === s[i]) &&
      size(batch.concat([m, last(s)])) <= MAX_SIZE;
    let b;
    if (this.strict) b = this.input(batch.concat([k, n]));
    else {
      b = rng.chance(0.3) ? this.choose(fits) : undefined;
      if (b === undefined) b = this.leaf(batch.concat([k, n]));
    }
    return g.matmul(a, b);
  }

  broadcast(x) {
    const { g, rng } = this;
    const xs = g.shape(x);
    const lead = [];
    if (rng.chance(0.5)) for (let i = rng.int(1, 2); i > 0; i--) lead.push(rng.int(2, 4));
    const to = lead.concat(xs.map((d) => (d === 1 && rng.chance(0.7) ? rng.int(2, 5) : d)));
    if (to.length > 4 || size(to) > MAX_SIZE || sameShape(to, xs)) return undefined;
    return g.broadcast(x, to);
  }

  reshape(x) {
    const { g, rng } = this;
    const n = size(g.shape(x));
    const all = factorizations(n, rng.int(1, 4)).filter((s) => s.length <= 4);
    const wide = all.filter((s) => s.length >= 2 && last(s) > 1 && s[s.length - 2] > 1);
    const shape = rng.pick(wide.length && rng.chance(this.strict ? 0.9 : 0.7) ? wide : all);
    const id = g.reshape(x, shape);
    return id === x ? undefined : id;
  }

  transpose(x) {
    const { g, rng } = this;
    const rank = g.shape(x).length;
    let perm;
    for (let t = 0; t < 10; t++) {
      perm = rng.shuffle(Array.from({ length: rank }, (_, i) => i));
      if (!perm.every((p, i) => p === i) && (!isInvolution(perm) || rng.chance(this.strict ? 0.1 : 0.3))) break;
    }
    const id = g.transpose(x, perm);
    return id === x ? undefined : id;
  }

  /** x weighted elementwise by a new input of its shape, so its cotangent is not uniform. */
  weigh(x) { return this.g.mul(x, this.input(this.g.shape(x))); }
}

/** Programs built around one op, placed on a path to the output and weighted after it. */
const TARGETED = {
  matmul(b) {
    const rank = b.rng.chance(0.6) ? 2 : 3;
    const batch = rank === 3 ? [b.rng.int(2, 3)] : [];
    const m = b.rng.int(2, 5), k = b.rng.int(2, 5);
    let x = b.input(batch.concat([m, k]));
    for (let i = b.rng.int(1, 2); i > 0; i--) {
      if (b.rng.chance(0.5)) x = b.push(b.g.tanh(x));
      const y = b.matmul(x);
      if (y === undefined || !b.ok(y)) break;
      x = b.push(y);
    }
    return x;
  },
  transpose(b) {
    const x0 = b.input(b.shape(3, 4));
    const t0 = b.transpose(x0);
    let x = b.push(t0 === undefined ? x0 : t0);
    x = b.push(b.weigh(b.g.tanh(x)));
    if (b.rng.chance(0.5)) { const t1 = b.transpose(x); x = b.push(t1 === undefined ? x : t1); }
    return x;
  },
  reshape(b) {
    for (let t = 0; t < 10; t++) {
      const x0 = b.input(b.shape(2, 4));
      let x = b.push(b.g.tanh(x0));
      const r = b.reshape(x);
      if (r === undefined) continue;
      x = b.push(r);
      x = b.push(b.weigh(x));
      if (b.rng.chance(0.4)) { const r2 = b.reshape(x); if (r2 !== undefined) x = b.push(r2); }
      return x;
    }
    throw new Error('no reshape in 10 tries');
  },
  broadcast(b) {
    for (let t = 0; t < 10; t++) {
      const x0 = b.input(b.shape(1, 3).map((d) => (b.rng.chance(0.5) ? 1 : d)));
      const y = b.broadcast(b.push(b.g.tanh(x0)));
      if (y === undefined) continue;
      return b.push(b.weigh(b.push(y)));
    }
    throw new Error('no broadcast in 10 tries');
  },
  sum(b) {
    const x0 = b.input(b.shape(2, 4));
    const x = b.push(b.g.tanh(x0));
    const axis = b.rng.int(0, b.g.shape(x).length - 1);
    return b.push(b.weigh(b.push(b.g.sum(x, axis, b.rng.chance(0.4)))));
  },
};

/** Apply an op, keeping it only if its result is provably within BOUND (else unwind it). */
function tryOp(b, op, operand) {
  const before = b.g.nodes.length;
  const id = b.apply(op, operand);
  if (id === undefined) return undefined;
  if (!b.ok(id)) {
    b.g.nodes.length = before;
    for (const k of Array.from(b.iv.keys())) if (k >= before) b.iv.delete(k);
    b.pool = b.pool.filter((p) => p < before);
    return undefined;
  }
  return b.push(id);
}

/**
 * A random program { seed, focus, graph, outputs, inputs, bounds }: general, or
 * built around `focus` (one of TARGETS); `f32` turns on the float32 guards.
 */
function randomProgram(seed, options) {
  const o = options || {};
  const focus = o.focus;
  const rng = new Rng(focus ? (seed * 31 + TARGETS.indexOf(focus) + 1) >>> 0 : seed);
  const b = new ProgramBuilder(rng);
  b.f32 = !!o.f32;
  b.squareAware = !!o.squareAware;
  if (focus) {
    b.strict = true;
    let lastId = TARGETED[focus](b);
    b.strict = false;
    for (let i = rng.int(0, 2); i > 0; i--) {
      const id = tryOp(b, rng.pick(['add', 'mul', 'tanh', 'exp', 'log', 'div', 'relu', 'sum', 'softmax']), lastId);
      if (id !== undefined) lastId = id;
    }
  } else {
    for (let i = rng.int(1, 3); i > 0; i--) b.input(b.shape());
    const weights = o.withSqrt ? Object.assign({}, GENERATED, { sqrt: 3 }) : GENERATED;
    const ops = [];
    for (const op of Object.keys(weights)) for (let w = 0; w < weights[op]; w++) ops.push(op);
    const steps = rng.int(2, 10);
    let made = 0;
    for (let attempt = 0; made < steps && attempt < steps * 20; attempt++) {
      if (tryOp(b, rng.pick(ops)) !== undefined) made++;
    }
  }
  const consumed = new Set();
  for (const n of b.g.nodes) for (const i of n.inputs) consumed.add(i);
  let outputs = b.g.nodes.filter((n) => n.op !== 'input' && n.op !== 'const' && !consumed.has(n.id)).map((n) => n.id);
  if (outputs.length === 0) outputs = [last(b.pool)];
  return {
    seed, focus: focus || null, graph: b.g, outputs, inputs: b.g.inputs().map((n) => n.attrs.name),
    bounds: b.g.nodes.map((n) => (b.iv.has(n.id) ? b.iv.get(n.id) : interval(b.g, n.id, b.iv, b.squareAware))),
  };
}

/** Corpus program i: general for odd i, targeted (cycling through TARGETS) for even i. */
function corpusProgram(i, options) {
  const o = options || {};
  if (i % 2 === 1) return randomProgram(i, o);
  return randomProgram(i, Object.assign({}, o, { focus: TARGETS[(i / 2) % TARGETS.length] }));
}

/**
 * The two graphs of corpus program i as the reference's fusion checks and GPU
 * fuzzer run them (src/fusion/measure-m4.js:27-40, src/gpu/harness-m4.js:126-142):
 * the program (float32 guards on) and its gradient graph, with inputs uniform in
 * [-2, 2] and cotangents uniform in [-1, 1] drawn from Rng(i * 7919 + 17), and
 * the ids each keeps (the outputs; the outputs and every gradient).
 */
function corpusGraphs(i) {
  const { grad } = require('../autodiff');
  const p = corpusProgram(i, { f32: true });
  const rng = new Rng((i * 7919 + 17) >>> 0);
  const inputs = {};
  for (const n of p.graph.inputs()) inputs[n.attrs.name] = rng.array(size(n.shape), -2, 2);
  const G = grad(p.graph, p.outputs, p.graph.inputs().map((n) => n.id));
  const gradInputs = Object.assign({}, inputs);
  G.cotangents.forEach((name, k) => { gradInputs[name] = rng.array(size(p.graph.nodes[p.outputs[k]].shape), -1, 1); });
  return [
    { label: 'forward', graph: p.graph, inputs, keep: p.outputs },
    { label: 'gradient', graph: G.graph, inputs: gradInputs, keep: p.outputs.concat(G.grads) },
  ];
}

module.exports = { randomProgram, corpusProgram, corpusGraphs, interval, factorizations, MAX_SIZE, BOUND, GENERATED, TARGETS };
