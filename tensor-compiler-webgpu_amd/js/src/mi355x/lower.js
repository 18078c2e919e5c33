'use strict';
// Lowering a (possibly fused) graph to MI355X launches.
//
// Same contract as the reference's lowerFused / lower
// (src/fusion/lower-fused.js:32-45, src/gpu/lower.js:68-114 in
// abho7/tensor-compiler-webgpu): one launch per node that is neither an input
// nor a constant, in graph order, each naming its node, its input node ids, its
// u32 parameters and its grid. `code` is a kernel name; the HIP text is in
// `kernels[k].source`, compiled by the runner (one module per launch list).
//
// A plain node lowers as a one-op body through the same skeletons a fused
// node uses (elementwise, rowwise, column reduction, matmul), so an unfused
// graph is the fused graph's chain of kernels, each op rounded by the same
// tcmi::op_* helper. Kinds:
//   fused-elementwise | fused-rowwise | fused-epilogue   a fused node
//   elementwise | gather | rowreduce | colreduce | matmul  a plain node
// Every record also carries `bytes` — each unique operand read once at its own
// size plus the output, the reference's byte count (workloads.js:171-172) —
// and `flops` (2·batch·M·N·K) for matmuls.

const { Graph } = require('../ir/graph');
const { size } = require('../ir/shapes');
const { bodyOf } = require('../fusion/fuse');
const cg = require('./codegen');

const ELEMENTWISE_OPS = new Set(['add', 'sub', 'mul', 'div', 'neg', 'exp', 'log', 'relu', 'tanh', 'sqrt', 'step', 'stopGradient']);
const GATHERS = new Set(['broadcast', 'transpose', 'reshape']);

/** A one-op body graph for `node` of `graph`: inputs a0.., then the op. */
function oneOpBody(graph, node, inputShapes, attrs) {
  const g = new Graph();
  const shapes = inputShapes || node.inputs.map((id) => graph.nodes[id].shape);
  const ins = shapes.map((s, k) => g.input(`a${k}`, s));
  const out = g.emit(node.op, ins, attrs || node.attrs);
  return { body: g, output: out };
}

function algorithmicBytes(graph, node) {
  let bytes = size(node.shape) * 4;
  for (const id of new Set(node.inputs)) bytes += size(graph.nodes[id].shape) * 4;
  return bytes;
}

function single(k) {
  const kernels = k.kernels || [{ name: k.name, source: k.source, grid: k.grid, block: k.block, lds: k.lds }];
  return { kernels, params: k.params, workspace: k.workspace || 0, flops: k.flops || 0 };
}

/** Kernels for one node. */
function lowerNode(graph, node, opts) {
  if (node.op === 'fused') {
    const b = bodyOf(node);
    const out = node.attrs.output;
    const kind = node.attrs.kind;
    const tuning = opts.tuning || {};
    const sab = { sabotage: opts.sabotage, pattern: node.attrs.pattern };
    if (kind === 'elementwise') {
      return Object.assign({ kind: 'fused-elementwise' }, single(cg.elementwiseKernel(b, out, node.shape, Object.assign({ tuning: tuning.ew }, sab))));
    }
    if (kind === 'rowwise') return Object.assign({ kind: 'fused-rowwise' }, single(cg.rowwiseKernel(b, out, sab)));
    if (kind === 'epilogue') return Object.assign({ kind: 'fused-epilogue' }, single(cg.gemmKernel(b, out, Object.assign({ tuning: tuning.gemm }, sab))));
    throw new Error(`no MI355X kernel for fused kind '${kind}'`);
  }
  if (ELEMENTWISE_OPS.has(node.op) || GATHERS.has(node.op)) {
    const { body, output } = oneOpBody(graph, node);
    const kind = GATHERS.has(node.op) ? 'gather' : 'elementwise';
    return Object.assign({ kind }, single(cg.elementwiseKernel(body, output, node.shape, { tuning: (opts.tuning || {}).ew })));
  }
  if (node.op === 'sum' || node.op === 'max') {
    const inShape = graph.nodes[node.inputs[0]].shape;
    const axis = node.attrs.axis;
    const outer = size(inShape.slice(0, axis)), n = inShape[axis], inner = size(inShape.slice(axis + 1));
    if (inner === 1) {
      // A reduction over the last non-trivial axis: the rowwise kernel on [outer, n].
      const { body, output } = oneOpBody(graph, node, [[outer, n]], { axis: 1, keepDims: true });
      return Object.assign({ kind: 'rowreduce' }, single(cg.rowwiseKernel(body, output, {})));
    }
    const c = cg.colreduceKernels(node.op, outer, n, inner, (opts.tuning || {}).colreduce);
    return { kind: 'colreduce', kernels: c.launches, params: c.params, workspace: c.workspace, flops: 0 };
  }
  if (node.op === 'matmul') {
    const { body, output } = oneOpBody(graph, node);
    return Object.assign({ kind: 'matmul' }, single(cg.gemmKernel(body, output, { tuning: (opts.tuning || {}).gemm })));
  }
  throw new Error(`no MI355X lowering for '${node.op}'`);
}

/**
 * Lower `graph` for the MI355X runner. Options: sabotage (one of the
 * reference's fused-kernel sabotages: 'epilogue-before-bias',
 * 'layernorm-tree-short', 'softmax-no-max', 'fused-bounds-off-by-one'),
 * applied to fused kernels only; tuning ({ ew: { unroll, nt, blocks }, colreduce: { blocks } })
 * overrides the kernels' launch-shape defaults (used by sweeps).
 * Returns { launches, workspace } (workspace: bytes of scratch the largest launch needs).
 */
function lowerMI355X(graph, options) {
  const opts = options || {};
  const cache = new Map();
  const launches = [];
  let workspace = 0;
  for (const node of graph.nodes) {
    if (node.op === 'input' || node.op === 'const') continue;
    // Kernels depend on structure and shapes only: reuse across identical nodes.
    const key = JSON.stringify([node.op, node.inputs.map((id) => graph.nodes[id].shape), node.attrs, node.shape,
      node.op === 'fused' ? opts.sabotage : null, opts.tuning || null]);
    let k = cache.get(key);
    if (!k) { k = lowerNode(graph, node, opts); cache.set(key, k); }
    workspace = Math.max(workspace, k.workspace);
    launches.push({
      node: node.id, op: node.op, kind: k.kind, pattern: node.op === 'fused' ? node.attrs.pattern : undefined,
      inputs: node.inputs.slice(), params: k.params, grid: k.kernels[0].grid, code: k.kernels[0].name,
      kernels: k.kernels, workspace: k.workspace, bytes: algorithmicBytes(graph, node), flops: k.flops,
    });
  }
  return { launches, workspace };
}

/** Every distinct kernel source of a launch list, in first-use order. */
function kernelSources(lowered) {
  const seen = new Map();
  for (const l of lowered.launches) for (const k of l.kernels) if (!seen.has(k.name)) seen.set(k.name, k.source);
  return seen;
}

module.exports = { lowerMI355X, kernelSources, lowerNode, oneOpBody, algorithmicBytes };
