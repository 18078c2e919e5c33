'use strict';
// The tensor IR: nodes in SSA form, ids are list positions (so the list is in
// topological order), shapes inferred at creation. The builder makes NumPy
// broadcasting explicit with `broadcast` nodes.
//
// Node for node the construction of src/ir/graph.js in
// abho7/tensor-compiler-webgpu (emit :21-31, builder :66-128, softmax and
// logSoftmax composites :133-146): graphs built here serialise to the same JSON
// as the reference's (pinned against its golden/cases.json), so the reference's
// own graphs and this host's are interchangeable at the backend's boundary.

const { inferShape, broadcastShapes, normAxis, sameShape, size, fmt, ShapeError } = require('./shapes');

/** Deep copy of plain attribute data (numbers, strings, booleans, arrays, objects). */
function cloneAttrs(v) {
  if (Array.isArray(v)) return v.map(cloneAttrs);
  if (v !== null && typeof v === 'object') {
    const o = {};
    for (const k of Object.keys(v)) o[k] = cloneAttrs(v[k]);
    return o;
  }
  return v;
}

class Graph {
  constructor() { this.nodes = []; }

  /** Append a node; returns its id (graph.js:21-31). */
  emit(op, inputs, attrs) {
    inputs = inputs || [];
    attrs = attrs || {};
    for (const id of inputs) {
      if (!Number.isInteger(id) || id < 0 || id >= this.nodes.length) {
        throw new ShapeError(`${op}: operand ${id} does not name a node of this graph`);
      }
    }
    const shape = inferShape(op, inputs.map((id) => this.nodes[id].shape), attrs);
    const id = this.nodes.length;
    this.nodes.push({ id, op, inputs: inputs.slice(), attrs: cloneAttrs(attrs), shape });
    return id;
  }

  shape(id) { return this.nodes[id].shape; }

  inputId(name) {
    for (const n of this.nodes) if (n.op === 'input' && n.attrs.name === name) return n.id;
    return undefined;
  }

  inputs() { return this.nodes.filter((n) => n.op === 'input'); }

  clone() {
    const g = new Graph();
    g.nodes = this.nodes.map((n) => ({ id: n.id, op: n.op, inputs: n.inputs.slice(), attrs: cloneAttrs(n.attrs), shape: n.shape.slice() }));
    return g;
  }

  toJSON() {
    return { nodes: this.nodes.map((n) => ({ op: n.op, inputs: n.inputs, attrs: n.attrs, shape: n.shape })) };
  }

  /** Rebuild from toJSON() output, re-checking every shape (graph.js:53-62). */
  static fromJSON(json) {
    const g = new Graph();
    for (const n of json.nodes) {
      const id = g.emit(n.op, n.inputs, n.attrs);
      if (!sameShape(g.shape(id), n.shape)) {
        throw new ShapeError(`node ${id} (${n.op}): recorded as ${fmt(n.shape)}, its rule gives ${fmt(g.shape(id))}`);
      }
    }
    return g;
  }

  // ---- builder ---------------------------------------------------------------

  input(name, shape) {
    if (this.inputId(name) !== undefined) throw new Error(`the graph has an input named '${name}' already`);
    return this.emit('input', [], { name, shape });
  }

  const(value, shape) { return this.emit('const', [], { shape: shape || [], value }); }

  broadcast(x, shape) {
    return sameShape(this.shape(x), shape) ? x : this.emit('broadcast', [x], { shape: shape.slice() });
  }

  binary(op, a, b) {
    const shape = broadcastShapes(this.shape(a), this.shape(b));
    if (!shape) throw new ShapeError(`${op}: no common broadcast shape for ${fmt(this.shape(a))} and ${fmt(this.shape(b))}`);
    const ba = this.broadcast(a, shape);
    const bb = this.broadcast(b, shape);
    return this.emit(op, [ba, bb]);
  }

  add(a, b) { return this.binary('add', a, b); }
  sub(a, b) { return this.binary('sub', a, b); }
  mul(a, b) { return this.binary('mul', a, b); }
  div(a, b) { return this.binary('div', a, b); }

  neg(x) { return this.emit('neg', [x]); }
  exp(x) { return this.emit('exp', [x]); }
  log(x) { return this.emit('log', [x]); }
  relu(x) { return this.emit('relu', [x]); }
  tanh(x) { return this.emit('tanh', [x]); }
  sqrt(x) { return this.emit('sqrt', [x]); }
  step(x) { return this.emit('step', [x]); }
  stopGradient(x) { return this.emit('stopGradient', [x]); }
  matmul(a, b) { return this.emit('matmul', [a, b]); }

  sum(x, axis, keepDims) {
    return this.emit('sum', [x], { axis: normAxis(axis, this.shape(x).length, 'sum'), keepDims: !!keepDims });
  }

  max(x, axis, keepDims) {
    return this.emit('max', [x], { axis: normAxis(axis, this.shape(x).length, 'max'), keepDims: !!keepDims });
  }

  reshape(x, shape) {
    return sameShape(this.shape(x), shape) ? x : this.emit('reshape', [x], { shape: shape.slice() });
  }

  /** Permute axes; no `perm` reverses them; the identity is no node. */
  transpose(x, perm) {
    const rank = this.shape(x).length;
    if (perm === undefined || perm === null) {
      perm = [];
      for (let i = rank - 1; i >= 0; i--) perm.push(i);
    }
    return perm.every((p, i) => p === i) ? x : this.emit('transpose', [x], { perm: perm.slice() });
  }

  transposeLast2(x) {
    const rank = this.shape(x).length;
    const perm = [];
    for (let i = 0; i < rank; i++) perm.push(i);
    perm[rank - 2] = rank - 1;
    perm[rank - 1] = rank - 2;
    return this.transpose(x, perm);
  }

  // ---- composites ---------------------------------------------------------------

  /** x minus its gradient-free maximum along `axis` (graph.js:133-136). */
  shifted(x, axis) {
    const m = this.stopGradient(this.max(x, axis, true));
    return this.sub(x, m);
  }

  softmax(x, axis) {
    if (axis === undefined) axis = -1;
    const z = this.exp(this.shifted(x, axis));
    return this.div(z, this.sum(z, axis, true));
  }

  logSoftmax(x, axis) {
    if (axis === undefined) axis = -1;
    const z = this.shifted(x, axis);
    return this.sub(z, this.log(this.sum(this.exp(z), axis, true)));
  }
}

module.exports = { Graph, size, cloneAttrs };
