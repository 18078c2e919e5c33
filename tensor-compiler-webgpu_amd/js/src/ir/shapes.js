'use strict';
// Static shapes of the IR: every op's result shape, computed once when the node
// is created, so a graph that exists is shape-consistent.
//
// The op set and shape rules are the reference's (src/ir/shapes.js of
// abho7/tensor-compiler-webgpu: OPS :51, inferShape :55-116, broadcastShapes
// :29-39), since graphs must be interchangeable with its builder's; the reference's
// module needs Node >= 24, so the host side of this backend carries its own.

class ShapeError extends Error {
  constructor(message) { super(message); this.name = 'ShapeError'; }
}

function size(shape) {
  let n = 1;
  for (const d of shape) n *= d;
  return n;
}

function sameShape(a, b) {
  if (a.length !== b.length) return false;
  for (let i = 0; i < a.length; i++) if (a[i] !== b[i]) return false;
  return true;
}

const fmt = (shape) => `[${shape.join(',')}]`;

function checkShape(shape, what) {
  const ok = Array.isArray(shape) && shape.every((d) => Number.isInteger(d) && d >= 1);
  if (!ok) throw new ShapeError(`${what}: a shape is a list of positive integers, not ${JSON.stringify(shape)}`);
}

/** A possibly negative axis resolved against `rank` (shapes.js:20-27). */
function normAxis(axis, rank, op) {
  const a = axis < 0 ? axis + rank : axis;
  if (!Number.isInteger(a) || a < 0 || a >= rank) throw new ShapeError(`${op}: no axis ${axis} in a rank-${rank} value`);
  return a;
}

/** NumPy broadcasting of two shapes; null when they do not broadcast (shapes.js:29-39). */
function broadcastShapes(a, b) {
  const rank = Math.max(a.length, b.length);
  const out = new Array(rank);
  for (let i = 0; i < rank; i++) {
    const ia = a.length - rank + i, ib = b.length - rank + i;
    const da = ia >= 0 ? a[ia] : 1;
    const db = ib >= 0 ? b[ib] : 1;
    if (da !== db && da !== 1 && db !== 1) return null;
    out[i] = Math.max(da, db);
  }
  return out;
}

/** True when `from` broadcasts to exactly `to` (shapes.js:42-46). */
function broadcastsTo(from, to) {
  if (from.length > to.length) return false;
  const lead = to.length - from.length;
  for (let i = 0; i < from.length; i++) if (from[i] !== 1 && from[i] !== to[lead + i]) return false;
  return true;
}

const UNARY = new Set(['neg', 'exp', 'log', 'relu', 'tanh', 'step', 'stopGradient', 'sqrt']);
const BINARY = new Set(['add', 'sub', 'mul', 'div']);
const REDUCE = new Set(['sum', 'max']);
const OPS = ['input', 'const', 'add', 'sub', 'mul', 'div', 'neg', 'exp', 'log', 'relu', 'tanh', 'step',
  'stopGradient', 'sqrt', 'matmul', 'sum', 'max', 'broadcast', 'reshape', 'transpose'];

/** Is `p` a permutation of 0 .. rank-1? */
function isPermutation(p, rank) {
  if (!Array.isArray(p) || p.length !== rank) return false;
  const seen = new Array(rank).fill(false);
  for (const v of p) {
    if (!Number.isInteger(v) || v < 0 || v >= rank || seen[v]) return false;
    seen[v] = true;
  }
  return true;
}

/** A leaf's declared shape (and a constant's value, one number or one per element). */
function leafShape(op, attrs) {
  checkShape(attrs.shape, op);
  if (op === 'const') {
    const v = attrs.value;
    if (!(typeof v === 'number' || (Array.isArray(v) && v.length === size(attrs.shape)))) {
      throw new ShapeError(`const of shape ${fmt(attrs.shape)}: expected one number or ${size(attrs.shape)} of them`);
    }
  }
  return attrs.shape.slice();
}

/**
 * Shape rules: op -> { arity, rule(shapes, attrs, op) } (the result shape, or a thrown
 * ShapeError). Binary ops take equal shapes only: the builder inserts broadcasts.
 */
const SHAPE_RULES = {
  input: { arity: 0, rule: (s, attrs, op) => leafShape(op, attrs) },
  const: { arity: 0, rule: (s, attrs, op) => leafShape(op, attrs) },
  matmul: {
    arity: 2,
    rule([a, b]) {
      if (a.length < 2 || b.length < 2) throw new ShapeError(`matmul of ${fmt(a)} by ${fmt(b)}: both operands need two or more axes`);
      if (a.length !== b.length || !sameShape(a.slice(0, -2), b.slice(0, -2))) {
        throw new ShapeError(`matmul of ${fmt(a)} by ${fmt(b)}: the leading (batch) axes must agree`);
      }
      const k = a[a.length - 1];
      if (k !== b[b.length - 2]) throw new ShapeError(`matmul of ${fmt(a)} by ${fmt(b)}: contracted lengths ${k} and ${b[b.length - 2]}`);
      return a.slice(0, -1).concat([b[b.length - 1]]);
    },
  },
  broadcast: {
    arity: 1,
    rule([x], attrs, op) {
      checkShape(attrs.shape, op);
      if (!broadcastsTo(x, attrs.shape)) throw new ShapeError(`broadcast: cannot stretch ${fmt(x)} to ${fmt(attrs.shape)}`);
      return attrs.shape.slice();
    },
  },
  reshape: {
    arity: 1,
    rule([x], attrs, op) {
      checkShape(attrs.shape, op);
      if (size(attrs.shape) !== size(x)) {
        throw new ShapeError(`reshape: ${fmt(x)} (${size(x)} elements) cannot become ${fmt(attrs.shape)} (${size(attrs.shape)})`);
      }
      return attrs.shape.slice();
    },
  },
  transpose: {
    arity: 1,
    rule([x], attrs) {
      if (!isPermutation(attrs.perm, x.length)) {
        throw new ShapeError(`transpose of ${fmt(x)}: ${JSON.stringify(attrs.perm)} is not a permutation of its ${x.length} axes`);
      }
      return attrs.perm.map((i) => x[i]);
    },
  },
};
for (const op of BINARY) {
  SHAPE_RULES[op] = {
    arity: 2,
    rule([a, b]) {
      if (!sameShape(a, b)) throw new ShapeError(`${op} of ${fmt(a)} and ${fmt(b)}: operands must have one shape (insert a broadcast)`);
      return a.slice();
    },
  };
}
for (const op of UNARY) SHAPE_RULES[op] = { arity: 1, rule: ([x]) => x.slice() };
for (const op of REDUCE) {
  SHAPE_RULES[op] = {
    arity: 1,
    rule([x], attrs) {
      const axis = normAxis(attrs.axis, x.length, op);
      if (attrs.axis !== axis) throw new ShapeError(`${op}: store the axis as ${axis}, not ${attrs.axis}`);
      const out = [];
      for (let i = 0; i < x.length; i++) {
        if (i !== axis) out.push(x[i]);
        else if (attrs.keepDims) out.push(1);
      }
      return out;
    },
  };
}

/** The result shape of `op` on inputs of `shapes`, or a thrown ShapeError (the rules of shapes.js:55-116). */
function inferShape(op, shapes, attrs) {
  const r = SHAPE_RULES[op];
  if (!r) throw new ShapeError(`'${op}' is not an op of this IR`);
  if (shapes.length !== r.arity) throw new ShapeError(`${op} takes ${r.arity} operand(s), was given ${shapes.length}`);
  return r.rule(shapes, attrs || {}, op);
}

/** Row-major strides of `shape` (interp.js:10-15). */
function strides(shape) {
  const s = new Array(shape.length);
  let acc = 1;
  for (let i = shape.length - 1; i >= 0; i--) { s[i] = acc; acc *= shape[i]; }
  return s;
}

module.exports = { ShapeError, size, sameShape, fmt, normAxis, broadcastShapes, broadcastsTo, inferShape, strides,
  OPS, UNARY, BINARY, REDUCE };
