'use strict';
// Seeded random well-typed programs: the fuzzing corpus of the reference
// (src/testing/random-graph.js, its "version 2", in abho7/tensor-compiler-webgpu).
//
// The corpus must be the reference's program for program: its recorded counts —
// golden/cases.json's 40 v2 graphs, and the fusion pass's results over corpus
// programs 1..2000 in golden/measurements.json m4 — pin this backend's builder,
// autodiff and fusion pass. So every random decision below is drawn from the same
// generator (mulberry32, ./rng) at the same point of the construction as there; the
// construction itself is this file's own. Its rules:
//   - every value carries an interval that is sound for inputs in [-2, 2]; an op
//     whose result could exceed BOUND in magnitude is undone with every node it
//     emitted (the input counter is not rewound);
//   - log, div, sqrt and exp only see operands their interval proves safe: the
//     operand is replaced by x·x + c, -(x·x + c), exp(x) or tanh(x) where needed;
//   - tensors hold at most MAX_SIZE elements;
//   - a general program draws weighted ops over a pool of values that favours the
//     recent ones; a targeted program is built around one op (matmul, transpose,
//     reshape, broadcast, sum), with no size-1 dims and fresh inputs, then takes a
//     few more ops;
//   - every computed value nothing consumes is an output.

const { Graph } = require('../ir/graph');
const { broadcastShapes, size } = require('../ir/shapes');
const { Rng } = require('./rng');

const MAX_SIZE = 96;
const BOUND = 1e3;
const INPUT_LO = -2, INPUT_HI = 2;

/** Relative weights of the general programs' ops (in this key order). */
const GENERATED = {
  add: 3, sub: 3, mul: 3, div: 3, neg: 1, exp: 2, log: 2, relu: 3, tanh: 2,
  matmul: 4, sum: 3, broadcast: 2, reshape: 3, transpose: 3, softmax: 2, logSoftmax: 2,
};

/** Ops with a program built around them, in this order. */
const TARGETS = ['matmul', 'transpose', 'reshape', 'broadcast', 'sum'];

/** The ops a targeted program may take after its target. */
const FOLLOW_UPS = ['add', 'mul', 'tanh', 'exp', 'log', 'div', 'relu', 'sum', 'softmax'];

const lastOf = (a) => a[a.length - 1];
const absMax = ([lo, hi]) => Math.max(Math.abs(lo), Math.abs(hi));
const sameDims = (a, b) => a.length === b.length && a.every((d, i) => d === b[i]);
const snap = (v) => Math.round(v * 1024) / 1024;   // to a multiple of 2^-10

/** The interval of a product of two intervals. */
function product([a0, a1], [b0, b1]) {
  const c = [a0 * b0, a0 * b1, a1 * b0, a1 * b1];
  return [Math.min.apply(null, c), Math.max.apply(null, c)];
}

const WHOLE_LINE = [-Infinity, Infinity];

/**
 * Interval rules, op -> (a, b, node, graph, squares) with a, b the operands' intervals.
 * `squares`: x·x is known non-negative (the generator's square-aware mode).
 */
const RANGE = {
  input: () => [INPUT_LO, INPUT_HI],
  const: (a, b, n) => {
    const v = n.attrs.value;
    if (typeof v === 'number') return [v, v];
    return [Math.min.apply(null, v), Math.max.apply(null, v)];
  },
  add: (a, b) => [a[0] + b[0], a[1] + b[1]],
  sub: (a, b) => [a[0] - b[1], a[1] - b[0]],
  mul: (a, b, n, g, squares) => {
    if (!(squares && n.inputs[0] === n.inputs[1])) return product(a, b);
    const m = absMax(a);
    return [a[0] <= 0 && a[1] >= 0 ? 0 : Math.min(a[0] * a[0], a[1] * a[1]), m * m];
  },
  div: (a, b) => (b[0] <= 0 && b[1] >= 0 ? WHOLE_LINE.slice() : product(a, [1 / b[1], 1 / b[0]])),
  neg: (a) => [-a[1], -a[0]],
  exp: (a) => [Math.exp(a[0]), Math.exp(a[1])],
  log: (a) => (a[0] > 0 ? [Math.log(a[0]), Math.log(a[1])] : WHOLE_LINE.slice()),
  relu: (a) => [Math.max(0, a[0]), Math.max(0, a[1])],
  step: () => [0, 1],
  tanh: (a) => [Math.tanh(a[0]), Math.tanh(a[1])],
  sqrt: (a) => (a[0] >= 0 ? [Math.sqrt(a[0]), Math.sqrt(a[1])] : WHOLE_LINE.slice()),
  // A sum of K products, K the contracted length.
  matmul: (a, b, n, g) => product(a, b).map((x) => x * lastOf(g.shape(n.inputs[0]))),
  // A sum of `len` values.
  sum: (a, b, n, g) => a.map((x) => x * g.shape(n.inputs[0])[n.attrs.axis]),
  max: (a) => a.slice(),
  stopGradient: (a) => a.slice(),
  broadcast: (a) => a.slice(),
  reshape: (a) => a.slice(),
  transpose: (a) => a.slice(),
};

/** The interval of node `id` from its operands' intervals in `known` (sound, not tight). */
function interval(g, id, known, squares) {
  const n = g.nodes[id];
  const rule = RANGE[n.op];
  if (!rule) throw new Error(`no interval rule for ${n.op}`);
  const ranges = n.inputs.map((i) => known.get(i));
  return rule(ranges[0], ranges[1], n, g, squares);
}

/** Every ordered factorisation of n into `rank` factors, by increasing first factor. */
function factorizations(n, rank) {
  if (rank === 1) return [[n]];
  const out = [];
  for (let d = 1; d <= n; d++) {
    if (n % d !== 0) continue;
    for (const tail of factorizations(n / d, rank - 1)) out.push([d].concat(tail));
  }
  return out;
}

const identity = (perm) => perm.every((p, i) => p === i);
const selfInverse = (perm) => perm.every((p, i) => perm[p] === i);

/** The state of one program under construction, and the draws that shape it. */
class Generator {
  constructor(rng, o) {
    this.rng = rng;
    this.g = new Graph();
    this.known = new Map();      // node id -> interval
    this.pool = [];              // values later ops may take, oldest first
    this.inputs = 0;             // inputs made so far (names x0, x1, ...)
    this.strict = false;         // targeted construction: no size-1 dims, matmul's B a fresh input
    this.f32 = !!o.f32;          // float32 guard: exp arguments kept above -40
    this.squares = !!o.squareAware;
    this.forced = undefined;     // the operand an op must take, if any
  }

  // ---- intervals -------------------------------------------------------------------

  /** Give every node up to `id` its interval (guards may have emitted nodes in between). */
  settle(id) {
    if (this.known.has(id)) return id;
    for (let i = 0; i <= id; i++) if (!this.known.has(i)) this.known.set(i, interval(this.g, i, this.known, this.squares));
    return id;
  }

  bounded(id) { return absMax(this.known.get(this.settle(id))) <= BOUND; }

  /** A mark to rewind to: nodes, intervals and pool entries after it are dropped. */
  mark() { return this.g.nodes.length; }

  rewind(at) {
    this.g.nodes.length = at;
    for (const k of Array.from(this.known.keys())) if (k >= at) this.known.delete(k);
    this.pool = this.pool.filter((id) => id < at);
  }

  // ---- shapes ----------------------------------------------------------------------

  dimension() {
    if (this.strict) return this.rng.int(2, 5);
    return this.rng.chance(0.2) ? 1 : this.rng.int(2, 6);
  }

  /** A shape of rank in [lo, hi] (default [0, 4]) holding at most MAX_SIZE elements. */
  randomShape(lo, hi) {
    const minRank = lo === undefined ? 0 : lo, maxRank = hi === undefined ? 4 : hi;
    for (;;) {
      const rank = this.rng.int(minRank, maxRank);
      const dims = [];
      for (let i = 0; i < rank; i++) dims.push(this.dimension());
      if (size(dims) <= MAX_SIZE) return dims;
    }
  }

  // ---- values ----------------------------------------------------------------------

  /** A value later ops may take. */
  offer(id) { this.settle(id); this.pool.push(id); return id; }

  freshInput(shape) { return this.offer(this.g.input(`x${this.inputs++}`, shape)); }

  /** A new input (70 %) or constant tensor of `shape`. */
  freshLeaf(shape) {
    if (this.rng.chance(0.7)) return this.freshInput(shape);
    const values = this.rng.array(size(shape), -2, 2).map(snap);
    return this.offer(this.g.const(values, shape));
  }

  /** A pool value passing `keep(shape, id)`, recent ones favoured (index skewed by r²). */
  pickValue(keep) {
    const fits = this.pool.filter((id) => !keep || keep(this.g.shape(id), id));
    if (fits.length === 0) return undefined;
    const r = this.rng.next();
    return fits[fits.length - 1 - Math.floor(r * r * fits.length)];
  }

  /** An op's first operand: the forced one if there is one (and it passes), else picked. */
  firstOperand(keep) {
    if (this.forced === undefined) return this.pickValue(keep);
    return !keep || keep(this.g.shape(this.forced), this.forced) ? this.forced : undefined;
  }

  /** A second operand for a binary op with x: a broadcast-compatible pool value, or a new leaf. */
  secondOperand(x) {
    const xs = this.g.shape(x);
    const compatible = (s) => { const out = broadcastShapes(xs, s); return !!out && size(out) <= MAX_SIZE; };
    const found = this.rng.chance(0.5) ? this.pickValue(compatible) : undefined;
    if (found !== undefined) return found;
    const drop = this.rng.chance(0.3) ? this.rng.int(0, xs.length) : 0;
    return this.freshLeaf(xs.slice(drop).map((d) => (this.rng.chance(0.3) ? 1 : d)));
  }

  literal(lo, hi) { return this.settle(this.g.const(snap(this.rng.uniform(lo, hi)))); }

  // ---- guards: operands an op can take safely ----------------------------------------

  /** x·x + c, c in [0.2, 1]: positive. */
  squarePlus(x) { const sq = this.g.mul(x, x); return this.g.add(sq, this.literal(0.2, 1)); }

  /** x if exp(x) stays bounded (and, with the float32 guard, normal), else tanh(x). */
  expSafe(x) {
    const [lo, hi] = this.known.get(x);
    return hi <= 4 && (!this.f32 || lo >= -40) ? x : this.settle(this.g.tanh(x));
  }

  /** x if it is at least 0.1 away from zero, else a value that is. */
  awayFromZero(x) {
    const [lo, hi] = this.known.get(x);
    if (lo >= 0.1 || hi <= -0.1) return x;
    const r = this.rng.next();
    if (r < 0.4) return this.settle(this.squarePlus(x));
    if (r < 0.6) return this.settle(this.g.neg(this.squarePlus(x)));
    return this.settle(this.g.exp(this.expSafe(x)));
  }

  /** x if it is at least 0.1, else exp(x) + c. */
  sqrtSafe(x) {
    if (this.known.get(x)[0] >= 0.1) return x;
    const e = this.g.exp(this.expSafe(x));
    return this.settle(this.g.add(e, this.literal(0.2, 1)));
  }

  /** x if it is at least 0.1, else x·x + c (60 %) or exp(x). */
  logSafe(x) {
    if (this.known.get(x)[0] >= 0.1) return x;
    return this.rng.chance(0.6) ? this.settle(this.squarePlus(x)) : this.settle(this.g.exp(this.expSafe(x)));
  }

  // ---- structural ops ----------------------------------------------------------------

  matmulWith(first) {
    const { g, rng } = this;
    let a = first;
    let as = g.shape(a);
    if (as.length < 2) {
      // A vector or scalar is first reshaped into a matrix, square-ish (80 %) where possible.
      const all = factorizations(size(as), 2);
      const square = all.filter(([m, k]) => m > 1 && k > 1);
      const choice = square.length && rng.chance(0.8) ? square : all;
      a = this.settle(g.reshape(a, rng.pick(choice)));
      as = g.shape(a);
    }
    const batch = as.slice(0, -2), m = as[as.length - 2], k = lastOf(as);
    const n = this.dimension();
    if (size(batch.concat([m, n])) > MAX_SIZE || size(batch.concat([k, n])) > MAX_SIZE) return undefined;
    const fitsB = (s) => s.length === as.length && s[s.length - 2] === k && batch.every((d, i) => d === s[i])
      && size(batch.concat([m, lastOf(s)])) <= MAX_SIZE;
    let b;
    if (this.strict) {
      b = this.freshInput(batch.concat([k, n]));
    } else {
      if (rng.chance(0.3)) b = this.pickValue(fitsB);
      if (b === undefined) b = this.freshLeaf(batch.concat([k, n]));
    }
    return g.matmul(a, b);
  }

  broadcastOf(x) {
    const { g, rng } = this;
    const xs = g.shape(x);
    const lead = [];
    if (rng.chance(0.5)) for (let count = rng.int(1, 2); count > 0; count--) lead.push(rng.int(2, 4));
    const stretched = xs.map((d) => (d === 1 && rng.chance(0.7) ? rng.int(2, 5) : d));
    const to = lead.concat(stretched);
    if (to.length > 4 || size(to) > MAX_SIZE || sameDims(to, xs)) return undefined;
    return g.broadcast(x, to);
  }

  reshapeOf(x) {
    const { g, rng } = this;
    const rank = rng.int(1, 4);
    const all = factorizations(size(g.shape(x)), rank).filter((s) => s.length <= 4);
    const wide = all.filter((s) => s.length >= 2 && lastOf(s) > 1 && s[s.length - 2] > 1);
    const choice = wide.length && rng.chance(this.strict ? 0.9 : 0.7) ? wide : all;
    const id = g.reshape(x, rng.pick(choice));
    return id === x ? undefined : id;
  }

  transposeOf(x) {
    const { g, rng } = this;
    const axes = Array.from({ length: g.shape(x).length }, (_, i) => i);
    // Up to ten shuffles for a permutation that moves something; one that is its own
    // inverse is taken only sometimes.
    let perm = axes;
    for (let tries = 0; tries < 10; tries++) {
      perm = rng.shuffle(axes);
      if (identity(perm)) continue;
      if (!selfInverse(perm) || rng.chance(this.strict ? 0.1 : 0.3)) break;
    }
    const id = g.transpose(x, perm);
    return id === x ? undefined : id;
  }

  /** x times a new input of its shape, so the cotangent reaching x is not uniform. */
  weighted(x) { return this.g.mul(x, this.freshInput(this.g.shape(x))); }
}

/** How each op is emitted, given the generator (its first operand forced or picked). */
const EMIT = {
  add: (s) => { const a = s.firstOperand(); return s.g.add(a, s.secondOperand(a)); },
  sub: (s) => { const a = s.firstOperand(); return s.g.sub(a, s.secondOperand(a)); },
  mul: (s) => { const a = s.firstOperand(); return s.g.mul(a, s.secondOperand(a)); },
  div: (s) => { const a = s.firstOperand(); return s.g.div(a, s.awayFromZero(s.secondOperand(a))); },
  log: (s) => s.g.log(s.logSafe(s.firstOperand())),
  exp: (s) => s.g.exp(s.expSafe(s.firstOperand())),
  sqrt: (s) => s.g.sqrt(s.sqrtSafe(s.firstOperand())),
  neg: (s) => s.g.neg(s.firstOperand()),
  relu: (s) => s.g.relu(s.firstOperand()),
  tanh: (s) => s.g.tanh(s.firstOperand()),
  matmul: (s) => s.matmulWith(s.firstOperand()),
  sum: (s) => {
    const x = s.firstOperand((sh) => sh.length >= 1);
    if (x === undefined) return undefined;
    const axis = s.rng.int(0, s.g.shape(x).length - 1);
    return s.g.sum(x, axis, s.rng.chance(0.4));
  },
  softmax: (s) => {
    const x = s.firstOperand((sh) => sh.length >= 1);
    return x === undefined ? undefined : s.g.softmax(x, s.rng.int(0, s.g.shape(x).length - 1));
  },
  logSoftmax: (s) => {
    const x = s.firstOperand((sh) => sh.length >= 1);
    return x === undefined ? undefined : s.g.logSoftmax(x, s.rng.int(0, s.g.shape(x).length - 1));
  },
  broadcast: (s) => s.broadcastOf(s.firstOperand()),
  reshape: (s) => s.reshapeOf(s.firstOperand()),
  transpose: (s) => {
    const x = s.firstOperand((sh) => sh.length >= 2);
    return x === undefined ? undefined : s.transposeOf(x);
  },
};

/**
 * Emit `op` (its first operand `forced` when given) and keep it only if its result is
 * provably within BOUND; otherwise undo everything it emitted. Returns the new value or
 * undefined.
 */
function attempt(s, op, forced) {
  const at = s.mark();
  s.forced = forced;
  const emit = EMIT[op];
  if (!emit) throw new Error(`no emitter for '${op}'`);
  const id = emit(s);
  if (id === undefined) return undefined;
  if (!s.bounded(id)) { s.rewind(at); return undefined; }
  return s.offer(id);
}

/** Programs built around one op: the op on a path to the result, weighted after it. */
const AROUND = {
  matmul(s) {
    const rank = s.rng.chance(0.6) ? 2 : 3;
    const batch = rank === 3 ? [s.rng.int(2, 3)] : [];
    const m = s.rng.int(2, 5), k = s.rng.int(2, 5);
    let x = s.freshInput(batch.concat([m, k]));
    for (let times = s.rng.int(1, 2); times > 0; times--) {
      if (s.rng.chance(0.5)) x = s.offer(s.g.tanh(x));
      const y = s.matmulWith(x);
      if (y === undefined || !s.bounded(y)) break;
      x = s.offer(y);
    }
    return x;
  },
  transpose(s) {
    const x0 = s.freshInput(s.randomShape(3, 4));
    const t0 = s.transposeOf(x0);
    let x = s.offer(t0 === undefined ? x0 : t0);
    x = s.offer(s.weighted(s.g.tanh(x)));
    if (s.rng.chance(0.5)) {
      const t1 = s.transposeOf(x);
      x = s.offer(t1 === undefined ? x : t1);
    }
    return x;
  },
  reshape(s) {
    for (let tries = 0; tries < 10; tries++) {
      const x0 = s.freshInput(s.randomShape(2, 4));
      let x = s.offer(s.g.tanh(x0));
      const r = s.reshapeOf(x);
      if (r === undefined) continue;
      x = s.offer(s.weighted(s.offer(r)));
      if (s.rng.chance(0.4)) {
        const r2 = s.reshapeOf(x);
        if (r2 !== undefined) x = s.offer(r2);
      }
      return x;
    }
    throw new Error('no reshape in 10 tries');
  },
  broadcast(s) {
    for (let tries = 0; tries < 10; tries++) {
      const dims = s.randomShape(1, 3).map((d) => (s.rng.chance(0.5) ? 1 : d));
      const y = s.broadcastOf(s.offer(s.g.tanh(s.freshInput(dims))));
      if (y === undefined) continue;
      return s.offer(s.weighted(s.offer(y)));
    }
    throw new Error('no broadcast in 10 tries');
  },
  sum(s) {
    const x = s.offer(s.g.tanh(s.freshInput(s.randomShape(2, 4))));
    const axis = s.rng.int(0, s.g.shape(x).length - 1);
    return s.offer(s.weighted(s.offer(s.g.sum(x, axis, s.rng.chance(0.4)))));
  },
};

/**
 * A random program { seed, focus, graph, outputs, inputs, bounds }: general, or built
 * around `focus` (one of TARGETS). Options: f32 (the float32 guard), squareAware,
 * withSqrt (sqrt among the general ops).
 */
function randomProgram(seed, options) {
  const o = options || {};
  const focus = o.focus;
  const rng = new Rng(focus ? (seed * 31 + TARGETS.indexOf(focus) + 1) >>> 0 : seed);
  const s = new Generator(rng, o);
  if (focus) {
    s.strict = true;
    let result = AROUND[focus](s);
    s.strict = false;
    for (let more = rng.int(0, 2); more > 0; more--) {
      const id = attempt(s, rng.pick(FOLLOW_UPS), result);
      if (id !== undefined) result = id;
    }
  } else {
    for (let count = rng.int(1, 3); count > 0; count--) s.freshInput(s.randomShape());
    const weights = o.withSqrt ? Object.assign({}, GENERATED, { sqrt: 3 }) : GENERATED;
    const bag = [];
    for (const op of Object.keys(weights)) for (let w = 0; w < weights[op]; w++) bag.push(op);
    const want = rng.int(2, 10);
    let made = 0;
    for (let tries = 0; made < want && tries < want * 20; tries++) {
      if (attempt(s, rng.pick(bag)) !== undefined) made++;
    }
  }
  const read = new Set();
  for (const n of s.g.nodes) for (const i of n.inputs) read.add(i);
  let outputs = s.g.nodes.filter((n) => n.op !== 'input' && n.op !== 'const' && !read.has(n.id)).map((n) => n.id);
  if (outputs.length === 0) outputs = [lastOf(s.pool)];
  return {
    seed, focus: focus || null, graph: s.g, outputs, inputs: s.g.inputs().map((n) => n.attrs.name),
    bounds: s.g.nodes.map((n) => (s.known.has(n.id) ? s.known.get(n.id) : interval(s.g, n.id, s.known, s.squares))),
  };
}

/** Corpus program i: general for odd i, targeted (TARGETS in turn) for even i. */
function corpusProgram(i, options) {
  const o = options || {};
  if (i % 2 === 1) return randomProgram(i, o);
  return randomProgram(i, Object.assign({}, o, { focus: TARGETS[(i / 2) % TARGETS.length] }));
}

/**
 * The two graphs of corpus program i as the reference's fusion checks and GPU fuzzer
 * run them (src/fusion/measure-m4.js:27-40, src/gpu/harness-m4.js:126-142): the program
 * (float32 guard on) and its gradient graph, inputs uniform in [-2, 2] and cotangents
 * uniform in [-1, 1] drawn from Rng(i·7919 + 17), with the ids each keeps (the outputs;
 * the outputs and every gradient).
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
