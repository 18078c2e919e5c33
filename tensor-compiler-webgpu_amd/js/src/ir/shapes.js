'use strict';
// Static shapes of the IR: every op's result shape, computed once when the node
// is created, so a graph that exists is shape-consistent.
//
// Same rules and op set as src/ir/shapes.js of abho7/tensor-compiler-webgpu
// (OPS :51, inferShape :55-116, broadcastShapes :29-39); the reference's own
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
  if (!ok) throw new ShapeError(`${what}: shape must be a list of positive integers, got ${JSON.stringify(shape)}`);
}

/** A possibly negative axis resolved against `rank` (shapes.js:20-27). */
function normAxis(axis, rank, op) {
  const a = axis < 0 ? axis + rank : axis;
  if (!Number.isInteger(a) || a < 0 || a >= rank) throw new ShapeError(`${op}: axis ${axis} out of range for rank ${rank}`);
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
const OP_SET = new Set(OPS);

function arityOf(op) {
  if (op === 'input' || op === 'const') return 0;
  if (op === 'matmul' || BINARY.has(op)) return 2;
  return 1;
}

/** The result shape of `op` on inputs of `shapes`, or a thrown ShapeError (shapes.js:55-116). */
function inferShape(op, shapes, attrs) {
  if (!OP_SET.has(op)) throw new ShapeError(`unknown op '${op}'`);
  const want = arityOf(op);
  if (shapes.length !== want) throw new ShapeError(`${op}: takes ${want} inputs, got ${shapes.length}`);
  if (op === 'input' || op === 'const') {
    checkShape(attrs.shape, op);
    if (op === 'const') {
      const v = attrs.value;
      const ok = typeof v === 'number' || (Array.isArray(v) && v.length === size(attrs.shape));
      if (!ok) throw new ShapeError(`const: value must be a number or ${size(attrs.shape)} numbers`);
    }
    return attrs.shape.slice();
  }
  if (BINARY.has(op)) {
    if (!sameShape(shapes[0], shapes[1])) {
      throw new ShapeError(`${op}: shapes ${fmt(shapes[0])} and ${fmt(shapes[1])} differ; broadcast explicitly`);
    }
    return shapes[0].slice();
  }
  if (UNARY.has(op)) return shapes[0].slice();
  if (op === 'matmul') {
    const a = shapes[0], b = shapes[1];
    if (a.length < 2 || b.length < 2) throw new ShapeError(`matmul: needs rank >= 2, got ${fmt(a)} and ${fmt(b)}`);
    if (a.length !== b.length || !sameShape(a.slice(0, -2), b.slice(0, -2))) {
      throw new ShapeError(`matmul: batch dims of ${fmt(a)} and ${fmt(b)} differ`);
    }
    if (a[a.length - 1] !== b[b.length - 2]) throw new ShapeError(`matmul: inner dims of ${fmt(a)} and ${fmt(b)} differ`);
    return a.slice(0, -1).concat([b[b.length - 1]]);
  }
  if (REDUCE.has(op)) {
    const x = shapes[0];
    const axis = normAxis(attrs.axis, x.length, op);
    if (attrs.axis !== axis) throw new ShapeError(`${op}: axis must be stored normalised`);
    return attrs.keepDims ? x.map((d, i) => (i === axis ? 1 : d)) : x.filter((_, i) => i !== axis);
  }
  if (op === 'broadcast') {
    checkShape(attrs.shape, op);
    if (!broadcastsTo(shapes[0], attrs.shape)) {
      throw new ShapeError(`broadcast: ${fmt(shapes[0])} does not broadcast to ${fmt(attrs.shape)}`);
    }
    return attrs.shape.slice();
  }
  if (op === 'reshape') {
    checkShape(attrs.shape, op);
    if (size(attrs.shape) !== size(shapes[0])) {
      throw new ShapeError(`reshape: ${fmt(shapes[0])} has ${size(shapes[0])} elements, ${fmt(attrs.shape)} has ${size(attrs.shape)}`);
    }
    return attrs.shape.slice();
  }
  if (op === 'transpose') {
    const x = shapes[0], p = attrs.perm;
    let isPerm = Array.isArray(p) && p.length === x.length;
    if (isPerm) {
      const sorted = p.slice().sort((u, v) => u - v);
      isPerm = sorted.every((v, i) => v === i);
    }
    if (!isPerm) throw new ShapeError(`transpose: ${JSON.stringify(p)} is not a permutation of rank ${x.length}`);
    return p.map((i) => x[i]);
  }
  throw new ShapeError(`no shape rule for '${op}'`);
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
