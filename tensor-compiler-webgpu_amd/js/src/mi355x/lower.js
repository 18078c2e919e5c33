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
//
// With `perf` (the trainer's and the bench's lowering; results are bit for bit
// those of the plain lowering, only fewer bytes move):
//   - a reshape launches nothing: its node shares its input's buffer (a
//     row-major reshape is the same bytes), listed in `aliases`;
//   - a transpose whose every consumer is a matmul operand (directly, through
//     further such transposes, or as an epilogue group's operand that only its
//     matmul reads) launches nothing either (`folded`): the matmuls read its
//     source in place through a strided view (tcmi_gemm.h). The records of
//     those matmuls name the source as their input. Reshapes on the way are
//     passed through where the readers are plain or epilogue products: their
//     view then maps a row or column index over several strides (a mapped view,
//     chainMap below; attention's heads merged back into rows).
//   - a relu whose every reader takes it as such a matmul operand launches
//     nothing: the matmuls apply relu to the relu's operand as they load it
//     (operandLoadOps below).
//   - a broadcast whose every consumer reads it in an elementwise, rowwise or
//     epilogue body (not as a matmul operand, not through a reduction or another
//     gather) launches nothing: each consumer's kernel reads the broadcast's
//     source through the broadcast's index map instead of a materialised copy.
//   - launches of one kernel text with no data path between them (the three
//     projections of an attention layer and their weight gradients, the
//     per-tensor parameter updates) are placed together and listed in
//     `batches`: the runner issues each batch as one dispatch per kernel of the
//     kernels' batched forms (batchPlan below).
// Nodes in `keep` are never folded, so their values stay readable.

const { Graph } = require('../ir/graph');
const { size } = require('../ir/shapes');
const { bodyOf } = require('../fusion/fuse');
const cg = require('./codegen');

const isReduce = (n) => n.op === 'sum' || n.op === 'max';
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

/** Each unique operand buffer read once at its own size, plus the output (workloads.js:171-172). */
function algorithmicBytes(graph, node, inputs) {
  let bytes = size(node.shape) * 4;
  for (const id of new Set(inputs || node.inputs)) bytes += size(graph.nodes[id].shape) * 4;
  return bytes;
}

function single(k) {
  const kernels = k.kernels || [{ name: k.name, source: k.source, grid: k.grid, block: k.block, lds: k.lds, needsPad: !!k.needsPad }];
  return { kernels, params: k.params, workspace: k.workspace || 0, flops: k.flops || 0 };
}

/**
 * `body` with the inputs at positions `folds` (pos -> {from, to} shapes) taking
 * the broadcast's source shape `from`, each followed by a broadcast to `to` that
 * stands for the input in the rest of the body. Returns { body, output }.
 */
function widenInputs(body, output, folds) {
  if (!folds || folds.size === 0) return { body, output };
  const g = new Graph();
  const map = new Map();
  for (const n of body.nodes) {
    if (n.op === 'input') {
      const pos = Number(n.attrs.name.slice(1));
      const f = folds.get(pos);
      const id = g.input(n.attrs.name, f ? f.from : n.shape);
      map.set(n.id, f ? g.broadcast(id, f.to) : id);
    } else {
      map.set(n.id, g.emit(n.op, n.inputs.map((i) => map.get(i)), n.attrs));
    }
  }
  return { body: g, output: map.get(output) };
}

/**
 * The body of a row-statistics chain `node` with its reductions folded in (`rowFold`, the
 * plan's records): inputs a{k} at the chain's launch positions, the reductions formed from
 * their operands (or their producers' bodies), then the chain. Returns { body, output }.
 */
function rowFoldBody(graph, node, rowFold) {
  const folds = rowFold.map((f) => {
    const fold = { pos: f.pos, op: graph.nodes[f.red].op, attrs: graph.nodes[f.red].attrs,
      shape: graph.nodes[f.red].shape, inShape: graph.nodes[graph.nodes[f.red].inputs[0]].shape };
    if (f.prod !== undefined) {
      // The producer's body, its inputs at the launch positions `ppos`.
      const p = graph.nodes[f.prod];
      const one = p.op === 'fused' ? { body: bodyOf(p), output: p.attrs.output } : oneOpBody(graph, p);
      fold.producer = Object.assign(widenInputs(one.body, one.output, f.prodFolds), { ppos: f.ppos });
    }
    return fold;
  });
  const chain = node.op === 'fused' ? { body: bodyOf(node), output: node.attrs.output } : oneOpBody(graph, node);
  return foldReductions(chain.body, chain.output, folds);
}

/**
 * The body a launch of `node` runs in the perf lowering before it forms any value it reads
 * (lowerNode's elementwise, gather, rowwise, row-statistics-chain and row-reduction
 * kernels), on inputs a{k} at its operand positions: a row-statistics chain with its
 * reductions folded in; a fused elementwise or rowwise body, or one elementwise op or
 * launched broadcast or transpose, with its broadcast operands widened and its absorbed
 * producers formed; a reduction over the last
 * non-trivial axis on its operand as [rows, n] rows (its producers formed), reshaped to
 * its own shape. Returns { body, output }, or null for other launches.
 */
function launchBase(graph, node, folds, rowFold, absorbs) {
  if (rowFold) return rowFoldBody(graph, node, rowFold);
  if (node.op === 'fused') {
    if (node.attrs.kind !== 'elementwise' && node.attrs.kind !== 'rowwise') return null;
    return absorbProducers(graph, widenInputs(bodyOf(node), node.attrs.output, folds), absorbs);
  }
  if (ELEMENTWISE_OPS.has(node.op) || node.op === 'broadcast' || node.op === 'transpose') {
    const one = oneOpBody(graph, node);
    return absorbProducers(graph, widenInputs(one.body, one.output, folds), absorbs);
  }
  if (node.op === 'sum' || node.op === 'max') {
    const inShape = graph.nodes[node.inputs[0]].shape;
    const axis = node.attrs.axis;
    const outer = size(inShape.slice(0, axis)), n = inShape[axis];
    if (size(inShape.slice(axis + 1)) !== 1 || n < 2) return null;
    const { body, output } = absorbProducers(graph, oneOpBody(graph, node, [[outer, n]], { axis: 1, keepDims: true }), absorbs);
    return { body, output: body.reshape(output, node.shape) };
  }
  return null;
}

/**
 * Whether a broadcast from `from` to `to` spreads a value of one element per row along the
 * rows' last C elements: the dims of `to` up to some point are the source's own, the rest
 * (C elements) are broadcast. The source's element for flat index e is then e / C.
 */
function rowBroadcast(from, to, C) {
  const lead = to.length - from.length;
  const src = (d) => (d < lead ? 1 : from[d - lead]);
  for (let p = 0; p <= to.length; p++) {
    if (size(to.slice(p)) !== C) continue;
    let ok = true;
    for (let d = 0; d < to.length && ok; d++) ok = d < p ? src(d) === to[d] : (src(d) === 1 || to[d] === 1);
    if (ok) return true;
  }
  return false;
}

/**
 * The rows a body reduces: { R, C } where every reduction reduces the last axis (C > 1
 * elements) of an operand of R·C elements and the output has R·C or R elements; { R: 0 }
 * for a body without reductions; null where they disagree, or where a value it computes
 * with R elements would pass for a row value without being one (no rowwise kernel runs
 * it). The rowwise kernel computes a value of R elements once per row, at the row index:
 * every reader of such a value must then be another value of R elements or a broadcast
 * spreading it along the rows (rowBroadcast) — with as many rows as their length, a
 * column vector broadcast down the rows has R elements too. And it reduces the row it is
 * on: a value depending on a reduction may reach an element only through ops at that
 * element's own index and such broadcasts, never through a transpose or another
 * broadcast, which would read it at another row's element.
 */
function rowLayout(body, output) {
  let R = 0, C = 0;
  for (const n of body.nodes) {
    if (!isReduce(n)) continue;
    const s = body.nodes[n.inputs[0]].shape;
    const c = s[s.length - 1];
    if (n.attrs.axis !== s.length - 1 || c < 2) return null;
    if (C === 0) { C = c; R = size(s) / c; } else if (c !== C || size(s) !== R * C) return null;
  }
  if (C === 0) return { R: 0 };
  const o = size(body.nodes[output].shape);
  if (o !== R * C && o !== R) return null;
  const rowDep = new Set();
  for (const n of body.nodes) {
    if (n.op === 'input' || n.op === 'const') continue;
    if (isReduce(n) || n.inputs.some((i) => rowDep.has(i))) rowDep.add(n.id);
    for (const i of n.inputs) {
      const src = body.nodes[i];
      const gather = n.op === 'broadcast' || n.op === 'transpose';
      if (gather && rowDep.has(i) && !(n.op === 'broadcast' && size(src.shape) === R && rowBroadcast(src.shape, n.shape, C))) return null;
      if (src.op === 'input' || src.op === 'const' || size(src.shape) !== R) continue;
      if (n.op === 'broadcast' ? !rowBroadcast(src.shape, n.shape, C) : (n.op === 'transpose' || size(n.shape) !== R)) return null;
    }
  }
  return { R, C };
}

/** Kernels for one node. */
function lowerNode(graph, node, opts, mmViews, folds, rowFold, lastReads, peers, absorbs, composed, streamOut, colFold) {
  if (colFold) {
    // The chain run as its column sum's kernel: the sum formed as in its own launch, the
    // chain's body applied to each sum (inputs at `pos`) at the store.
    const red = graph.nodes[colFold.red];
    const inShape = graph.nodes[red.inputs[0]].shape;
    const axis = red.attrs.axis;
    const chain = node.op === 'fused' ? { body: bodyOf(node), output: node.attrs.output } : oneOpBody(graph, node);
    const c = cg.colreduceKernels(red.op, size(inShape.slice(0, axis)), inShape[axis], size(inShape.slice(axis + 1)),
      (opts.tuning || {}).colreduce, null, { body: chain.body, output: chain.output, sumAt: colFold.pos });
    return { kind: 'colreduce', kernels: c.launches, params: c.params, workspace: c.workspace, flops: 0 };
  }
  if (composed) {
    // A launch forming values it reads (`composed`: its body with theirs inside, on the
    // buffers left to read): a rowwise kernel where the body reduces rows, with the
    // reductions' own tuning so the rows are reduced in their order; else elementwise.
    const t = opts.tuning || {};
    if (composed.body.nodes.some(isReduce)) {
      return Object.assign({ kind: 'fused-rowwise' },
        single(cg.rowwiseKernel(composed.body, composed.output, { tuning: t.rowreduce || t.row, lastReads, streamOut })));
    }
    return Object.assign({ kind: 'fused-elementwise' },
      single(cg.elementwiseKernel(composed.body, composed.output, node.shape, { tuning: t.ew, lastReads, streamOut })));
  }
  if (rowFold) {
    // A row-statistics chain with its reductions folded in: the rowwise kernel of the
    // reductions, with their own tuning so the rows are reduced in their order.
    const f = rowFoldBody(graph, node, rowFold);
    const t = opts.tuning || {};
    return Object.assign({ kind: 'fused-rowwise' }, single(cg.rowwiseKernel(f.body, f.output, { tuning: t.rowreduce || t.row, lastReads, streamOut })));
  }
  if (node.op === 'fused') {
    const w = absorbProducers(graph, widenInputs(bodyOf(node), node.attrs.output, folds), absorbs);
    const b = w.body;
    const out = w.output;
    const kind = node.attrs.kind;
    const tuning = opts.tuning || {};
    const sab = { sabotage: opts.sabotage, pattern: node.attrs.pattern };
    if (kind === 'elementwise') {
      return Object.assign({ kind: 'fused-elementwise' },
        single(cg.elementwiseKernel(b, out, node.shape, Object.assign({ tuning: tuning.ew, lastReads, streamOut }, sab))));
    }
    if (kind === 'rowwise') {
      return Object.assign({ kind: 'fused-rowwise' }, single(cg.rowwiseKernel(b, out, Object.assign({ tuning: tuning.row, lastReads, streamOut }, sab))));
    }
    if (kind === 'epilogue') {
      return Object.assign({ kind: 'fused-epilogue' }, single(cg.gemmKernel(b, out, Object.assign({ tuning: tuning.gemm, peers }, sab, mmViews))));
    }
    if (kind === 'attention') {
      return Object.assign({ kind: 'fused-attention' }, single(cg.attentionKernel(b, out, Object.assign({ tuning: tuning.attn }, mmViews))));
    }
    if (kind === 'attention-grad') {
      // One part of the three sharing this body; the kernel forming all three rides along
      // (batchPlan runs the three as one launch of it).
      const k = cg.attentionGradKernel(b, out, Object.assign({}, mmViews));
      const r = single(k);
      r.kernels[0].joint = k.joint;
      r.kernels[0].part = k.part;
      return Object.assign({ kind: 'fused-attention-grad' }, r);
    }
    throw new Error(`no MI355X kernel for fused kind '${kind}'`);
  }
  if (ELEMENTWISE_OPS.has(node.op) || GATHERS.has(node.op)) {
    const one = oneOpBody(graph, node);
    const { body, output } = absorbProducers(graph, widenInputs(one.body, one.output, folds), absorbs);
    const kind = GATHERS.has(node.op) ? 'gather' : 'elementwise';
    return Object.assign({ kind }, single(cg.elementwiseKernel(body, output, node.shape, { tuning: (opts.tuning || {}).ew, lastReads, streamOut })));
  }
  if (node.op === 'sum' || node.op === 'max') {
    const inShape = graph.nodes[node.inputs[0]].shape;
    const axis = node.attrs.axis;
    const outer = size(inShape.slice(0, axis)), n = inShape[axis], inner = size(inShape.slice(axis + 1));
    if (inner === 1) {
      // A reduction over the last non-trivial axis: the rowwise kernel on [outer, n] (its
      // operand formed in place where the lowering absorbed the operand's producer).
      const { body, output } = absorbProducers(graph, oneOpBody(graph, node, [[outer, n]], { axis: 1, keepDims: true }), absorbs);
      const t = opts.tuning || {};
      return Object.assign({ kind: 'rowreduce' }, single(cg.rowwiseKernel(body, output, { tuning: t.rowreduce || t.row, lastReads })));
    }
    // A column reduction whose operand's producer the lowering absorbed forms it (with what
    // it took in) on the producer's operands as it reads them.
    let prod = null;
    if (absorbs) {
      const g = new Graph();
      const a0 = g.input('a0', inShape);
      prod = absorbProducers(graph, { body: g, output: a0 }, absorbs);
    }
    const c = cg.colreduceKernels(node.op, outer, n, inner, (opts.tuning || {}).colreduce, prod);
    return { kind: 'colreduce', kernels: c.launches, params: c.params, workspace: c.workspace, flops: 0 };
  }
  if (node.op === 'matmul') {
    const { body, output } = oneOpBody(graph, node);
    return Object.assign({ kind: 'matmul' }, single(cg.gemmKernel(body, output, Object.assign({ tuning: (opts.tuning || {}).gemm, peers }, mmViews))));
  }
  throw new Error(`no MI355X lowering for '${node.op}'`);
}

/** Contiguous strides of `shape`. */
function stridesOf(shape) {
  const st = new Array(shape.length);
  let acc = 1;
  for (let d = shape.length - 1; d >= 0; d--) { st[d] = acc; acc *= shape[d]; }
  return st;
}

/** Consumers of every node: id -> [consumer ids] (with repeats per operand slot). */
function consumersOf(graph) {
  const c = graph.nodes.map(() => []);
  for (const n of graph.nodes) for (const i of n.inputs) c[i].push(n.id);
  return c;
}

/**
 * The matmul operand slots of node `n`: [[slot, operand position in n.inputs]]
 * for the operands only its matmuls read — 'a' and 'b' of a matmul or an
 * epilogue group's matmul; 'q', 'k' and 'v' of a fused attention (Q and Kt of
 * the scores, V of the output product).
 */
function matmulSlots(n) {
  if (n.op === 'matmul') return [['a', 0], ['b', 1]];
  // An attention gradient reads Q, K, V and dO (a0..a3) in its products alone.
  if (n.op === 'fused' && n.attrs.kind === 'attention-grad') return [['q', 0], ['k', 1], ['v', 2], ['o', 3]];
  if (n.op === 'fused' && n.attrs.kind === 'attention') {
    const b = n.attrs.body;
    const m2 = b.nodes[n.attrs.output];
    const m1 = b.nodes.find((x, i) => x.op === 'matmul' && i !== n.attrs.output);
    const only = (bodyId, user) => b.nodes.every((x, i) => i === user || !x.inputs.includes(bodyId));
    const slots = [];
    const m1Id = b.nodes.indexOf(m1);
    if (m1.inputs[0] !== m1.inputs[1]) {
      if (only(m1.inputs[0], m1Id)) slots.push(['q', Number(b.nodes[m1.inputs[0]].attrs.name.slice(1))]);
      if (only(m1.inputs[1], m1Id)) slots.push(['k', Number(b.nodes[m1.inputs[1]].attrs.name.slice(1))]);
    }
    if (only(m2.inputs[1], n.attrs.output)) slots.push(['v', Number(b.nodes[m2.inputs[1]].attrs.name.slice(1))]);
    return slots;
  }
  if (n.op !== 'fused' || n.attrs.kind !== 'epilogue') return [];
  const b = n.attrs.body;
  const root = b.nodes.find((x) => x.op === 'matmul');
  const slots = [];
  root.inputs.forEach((bodyId, k) => {
    const users = b.nodes.filter((x) => x.inputs.includes(bodyId));
    if (users.length === 1 && users[0].id === root.id && root.inputs[0] !== root.inputs[1]) {
      slots.push([k === 0 ? 'a' : 'b', Number(b.nodes[bodyId].attrs.name.slice(1))]);
    }
  });
  return slots;
}

/**
 * Perf-mode plan: { aliases: id -> source, folded: Set, views: id -> {slot: { source, view }},
 * broadcasts, dead: Set }. `dead`: nodes whose values nothing kept depends on (autodiff leaves
 * such sinks, e.g. the gradient flowing into the max shift's stopGradient, or the dX of a
 * one-hot input): no launch, no buffer. Inputs and constants are never dead.
 */
function perfPlan(graph, keep, rowFolding, absorbing, loadOps, noAbsorb) {
  const cons = consumersOf(graph);
  const live = new Set();
  for (let id = graph.nodes.length - 1; id >= 0; id--) {
    const n = graph.nodes[id];
    if (keep.has(id) || n.op === 'input' || n.op === 'const' || cons[id].some((c) => live.has(c))) live.add(id);
  }
  const dead = new Set(graph.nodes.filter((n) => !live.has(n.id)).map((n) => n.id));
  const aliases = new Map();
  for (const n of graph.nodes) {
    if (n.op === 'reshape' && !keep.has(n.id)) {
      const src = n.inputs[0];
      aliases.set(n.id, aliases.has(src) ? aliases.get(src) : src);
    }
  }
  // Which (consumer, operand position) pairs are matmul-only operand slots.
  const slotOf = new Map();
  for (const n of graph.nodes) for (const [slot, pos] of matmulSlots(n)) slotOf.set(`${n.id}:${pos}`, slot);
  const { folded, views } = inPlaceTransposes(graph, keep, cons, slotOf, dead);
  // Broadcasts read in place by every consumer's body (never through a matmul
  // operand slot, a plain reduction or another gather).
  const bodyReader = (c, pos) => {
    const n = graph.nodes[c];
    if (ELEMENTWISE_OPS.has(n.op)) return true;
    if (n.op !== 'fused') return false;
    return !slotOf.has(`${c}:${pos}`);
  };
  const broadcasts = new Map();   // consumer id -> Map(pos -> { source, from, to })
  for (const n of graph.nodes) {
    if (n.op !== 'broadcast' || keep.has(n.id) || cons[n.id].length === 0) continue;
    const ok = cons[n.id].every((c) => graph.nodes[c].inputs.every((i, pos) => i !== n.id || bodyReader(c, pos)));
    if (!ok) continue;
    folded.add(n.id);
    const src = n.inputs[0];
    for (const c of new Set(cons[n.id])) {
      graph.nodes[c].inputs.forEach((i, pos) => {
        if (i !== n.id) return;
        if (!broadcasts.has(c)) broadcasts.set(c, new Map());
        broadcasts.get(c).set(pos, { source: src, from: graph.nodes[src].shape, to: n.shape });
      });
    }
  }
  // Row statistics folded into their reduction: a plain sum or max over the last
  // non-trivial axis whose consumers (one or two) are all elementwise chains of its own
  // size, fused or a single op (LayerNorm's mean and deviation scale, softmax's row
  // scale, the backward pass's chains over the same statistics, the loss's log-sum and
  // mean), every operand of each chain a value of that
  // size (read at the row index), launches nothing: each chain runs as a rowwise kernel
  // that forms the reduction itself from the reduction's operand, its body on the row's
  // reduced value in registers — the same reduction order and the same ops in the same
  // order, so the same bits as the separate launches. The reductions a chain takes in
  // must share one operand shape (one rowwise kernel walks one row length).
  const rowFolds = new Map();   // chain id -> [{ red: reduction id, pos: its operand positions }]
  const isChain = (c, rows) => ((c.op === 'fused' && c.attrs.kind === 'elementwise') || ELEMENTWISE_OPS.has(c.op))
    && size(c.shape) === rows && c.inputs.every((i) => size(graph.nodes[i].shape) === rows && !folded.has(i));
  const cand = new Set();
  for (const n of rowFolding ? graph.nodes : []) {
    if ((n.op !== 'sum' && n.op !== 'max') || keep.has(n.id) || dead.has(n.id) || cons[n.id].length === 0) continue;
    const inShape = graph.nodes[n.inputs[0]].shape;
    if (size(inShape.slice(n.attrs.axis + 1)) !== 1 || inShape[n.attrs.axis] === 1) continue;
    const users = Array.from(new Set(cons[n.id]));
    if (users.length <= 2 && users.every((u) => isChain(graph.nodes[u], size(n.shape)))) cand.add(n.id);
  }
  const inShapeOf = (r) => graph.nodes[graph.nodes[r].inputs[0]].shape.join('x');
  for (const c of graph.nodes) {
    const reds = Array.from(new Set(c.inputs.filter((i) => cand.has(i))));
    for (const r of reds) if (inShapeOf(r) !== inShapeOf(reds[0])) cand.delete(r);
  }
  for (const r of cand) {
    folded.add(r);
    for (const u of new Set(cons[r])) {
      if (!rowFolds.has(u)) rowFolds.set(u, []);
      rowFolds.get(u).push({ red: r, pos: graph.nodes[u].inputs.map((i, k) => (i === r ? k : -1)).filter((k) => k >= 0) });
    }
  }
  // A folded reduction's producer folded in with it: an elementwise node (one op or a
  // fused chain) of the reduction's [rows, n] operand shape that only the reduction reads
  // and nothing keeps launches nothing either. The rowwise kernel forms the producer's
  // value per element from the producer's own operands, in registers, with the same ops
  // in the same order, then reduces it: the same bits, without writing the operand and
  // reading it back. Its operands join the chain's (the first in the reduction's slot,
  // the rest after the chain's own), all within one argument block. A fused producer's
  // body must hold full-size values only, besides its operands and constants and their
  // broadcasts: the rowwise kernel tells a row's value from an element's by size, so a
  // computed vector of the row length would be read at the row index where the rows are
  // as many as their length.
  const fullBody = (p) => {
    if (p.op !== 'fused') return true;
    const b = p.attrs.body.nodes;
    const n = size(p.shape);
    return b.every((x) => x.op === 'input' || x.op === 'const' || (ELEMENTWISE_OPS.has(x.op) && size(x.shape) === n)
      || (x.op === 'broadcast' && (b[x.inputs[0]].op === 'input' || b[x.inputs[0]].op === 'const')));
  };
  const producer = (r) => {
    const red = graph.nodes[r];
    const p = graph.nodes[red.inputs[0]];
    if (keep.has(p.id) || folded.has(p.id) || aliases.has(p.id) || p.shape.length !== 2 || red.attrs.axis !== 1) return null;
    if (!ELEMENTWISE_OPS.has(p.op) && !(p.op === 'fused' && p.attrs.kind === 'elementwise' && fullBody(p))) return null;
    if (new Set(cons[p.id]).size !== 1) return null;
    const own = broadcasts.get(p.id);
    if (!p.inputs.every((i, pos) => !folded.has(i) || (own && own.has(pos)))) return null;
    return p;
  };
  const producers = new Map();   // reduction id -> producer node
  for (const r of cand) { const p = producer(r); if (p) producers.set(r, p); }
  const operandsWith = (u) => rowFolds.get(u).reduce((n, f) => n + (producers.has(f.red) ? producers.get(f.red).inputs.length - 1 : 0),
    graph.nodes[u].inputs.length);
  for (let again = true; again;) {
    again = false;
    for (const u of rowFolds.keys()) {
      if (operandsWith(u) <= cg.MAX_IN) continue;
      for (const f of rowFolds.get(u)) again = producers.delete(f.red) || again;
    }
  }
  for (const [u, fs] of rowFolds) {
    let next = graph.nodes[u].inputs.length;
    for (const f of fs) {
      const p = producers.get(f.red);
      if (!p) continue;
      folded.add(p.id);
      f.prod = p.id;
      f.prodFolds = broadcasts.get(p.id) || null;
      f.ppos = p.inputs.map((_, j) => (j === 0 ? f.pos[0] : next++));
    }
  }
  // Producers absorbed into their one reader (with `absorb`: the trainer's lowering). An
  // elementwise node (one op or a fused chain) that nothing keeps and whose only live
  // reader is another elementwise node runs inside that reader's kernel: the reader's body
  // forms the producer's value from the producer's own operands, with the producer's ops
  // in their order, where it would have loaded it — the same bits, without writing the
  // value and reading it back. Autodiff leaves such pairs where the producer's other
  // consumer is dead (a stopGradient branch) and the fusion contract, which keeps every
  // node, could not join them. A producer read through a broadcast inside the reader's
  // body is formed at the broadcast's source index. A producer may have absorbed its own
  // producers (taken along), row-statistics chains take no part, and every operand fits
  // one argument block.
  // A row reduction over the last axis of a 2-D operand (a rowwise kernel) absorbs its
  // operand's producer too, where the producer's body, and those of the producers it
  // brings along, hold full-size values only (the rule of producer folds); so does a
  // column reduction (below).
  let absorbed = new Map();   // reader id -> [{ prod, pos: [reader positions], ppos, prodFolds, nested }]
  let operands = new Map();   // reader id -> its kernel's operand count with what it absorbed
  const isElementwise = (n) => ELEMENTWISE_OPS.has(n.op) || (n.op === 'fused' && n.attrs.kind === 'elementwise');
  const isRowReduction = (n) => (n.op === 'sum' || n.op === 'max') && n.attrs.axis === 1
    && graph.nodes[n.inputs[0]].shape.length === 2;
  const fullTree = (id, n) => size(graph.nodes[id].shape) === n && fullBody(graph.nodes[id])
    && (absorbed.get(id) || []).every((a) => fullTree(a.prod, n));
  // A column reduction (a sum or max over an axis other than the last non-trivial one: the
  // column-reduction kernels) absorbs its operand's producer too: the kernel forms it at
  // each element's flat index, broadcast operands through their index maps (LayerNorm's
  // dγ = Σ dy·x̂ over rows, x̂ formed from the centred rows and the row deviation).
  const isColReduction = (n) => (n.op === 'sum' || n.op === 'max') && !dead.has(n.id)
    && size(graph.nodes[n.inputs[0]].shape.slice(n.attrs.axis + 1)) > 1
    && size(graph.nodes[n.inputs[0]].shape) < 2 ** 32;
  const readersOf = (pid) => Array.from(new Set(cons[pid].filter((c) => !dead.has(c))));
  // The full-size operands a producer's kernel reads (its folded broadcasts' sources and
  // its operands of other sizes aside; those of the producers it absorbed included).
  const fullReads = (pid) => {
    const p = graph.nodes[pid];
    const pf = broadcasts.get(pid);
    const took = new Map((absorbed.get(pid) || []).map((a) => [a.prod, a]));
    const out = new Set();
    p.inputs.forEach((i, j) => {
      if (pf && pf.has(j)) return;
      if (took.has(i)) for (const x of fullReads(i)) out.add(x);
      else if (size(graph.nodes[i].shape) === size(p.shape)) out.add(i);
    });
    return out;
  };
  // A producer with several live readers is formed by each of them where all of them can
  // take it in and that moves no more bytes than its own launch would: r readers reading its
  // f full-size operands instead of its value (r·f) against the launch reading them and
  // writing its value (f + 1) and the readers reading that (r). LayerNorm's centred rows,
  // normalised rows and scaled gradient (read by two to five chains each) are such. Passes
  // repeat with the producers some reader could not take in left out, until every producer
  // allowed is taken in by all its readers (those launch nothing).
  let allowed = null;
  const before = new Set(folded);
  for (;;) {
    absorbed = new Map();
    operands = new Map();
    for (const id of Array.from(folded)) if (!before.has(id)) folded.delete(id);
    const shared = new Map();   // producer with several readers -> readers that took it in
    for (const e of absorbing ? graph.nodes : []) {
      const reduction = isRowReduction(e);
      const columns = isColReduction(e);
      if (!(isElementwise(e) || reduction || columns) || folded.has(e.id) || dead.has(e.id) || aliases.has(e.id) || rowFolds.has(e.id)) continue;
      if (noAbsorb && noAbsorb.has(e.id)) continue;
      const own = broadcasts.get(e.id);
      let next = e.inputs.length;
      const list = [];
      for (const pid of new Set(e.inputs)) {
        const p = graph.nodes[pid];
        const at = e.inputs.map((i, pos) => (i === pid ? pos : -1)).filter((pos) => pos >= 0);
        if (!isElementwise(p) || keep.has(pid) || folded.has(pid) || dead.has(pid) || aliases.has(pid) || rowFolds.has(pid)) continue;
        if (at.some((pos) => own && own.has(pos))) continue;
        const r = readersOf(pid).length;
        if (r !== 1) {
          if (allowed ? !allowed.has(pid) : r * fullReads(pid).size > fullReads(pid).size + 1 + r) continue;
        }
        if (reduction && !fullTree(pid, size(p.shape))) continue;
          const pf = broadcasts.get(pid);
        if (!p.inputs.every((i, j) => !folded.has(i) || (pf && pf.has(j)) || (absorbed.get(pid) || []).some((a) => a.prod === i))) continue;
        const m = operands.get(pid) || p.inputs.length;
        // A producer of constants alone has no operand to take the reader's slot.
        if (m === 0 || next + m - 1 > cg.MAX_IN) continue;
        const ppos = [];
        for (let j = 0; j < m; j++) ppos.push(j === 0 ? at[0] : next + j - 1);
        list.push({ prod: pid, pos: at, ppos, prodFolds: pf || null, nested: absorbed.get(pid) || null });
        next += m - 1;
        if (r !== 1) { if (!shared.has(pid)) shared.set(pid, new Set()); shared.get(pid).add(e.id); }
      }
      if (!list.length) continue;
      absorbed.set(e.id, list);
      operands.set(e.id, next);
      for (const a of list) if (!shared.has(a.prod)) folded.add(a.prod);
    }
    const whole = new Set(Array.from(shared).filter(([pid, by]) => by.size === readersOf(pid).length).map(([pid]) => pid));
    if (allowed && whole.size === allowed.size) {
      for (const pid of whole) folded.add(pid);
      break;
    }
    allowed = whole;
  }
  if (loadOps) operandLoadOps(graph, keep, cons, slotOf, dead, folded, views);
  // Column sums folded into their one reader: a sum over a non-last axis (a column sum,
  // such as a bias gradient) that nothing keeps and whose only reader is a kept
  // elementwise chain of its own size (the bias's update), every operand of which is a
  // value of that size, launches nothing: the chain runs as the column-sum kernel, which
  // forms each sum in the order of the sum's own launch and applies the chain's ops to
  // it at the store, so the same bits as the two launches. Only sums that run in one pass
  // (up to COLRED_ONE_PASS elements: config 1's biases): a larger one runs a second kernel
  // combining its row chunks, and its update already shares a dispatch with the others
  // (config 5's 31), so the fold would save no dispatch. Not where the sum forms its
  // operand's producer, or the chain reads a broadcast, a view or an absorbed producer.
  const colFolds = new Map();   // chain id -> { red: the sum's id, pos: its operand positions }
  for (const r of rowFolding ? graph.nodes : []) {
    if (r.op !== 'sum' || keep.has(r.id) || dead.has(r.id) || folded.has(r.id) || aliases.has(r.id) || absorbed.has(r.id)) continue;
    if (size(graph.nodes[r.inputs[0]].shape.slice(r.attrs.axis + 1)) === 1) continue;
    if (size(graph.nodes[r.inputs[0]].shape) > cg.COLRED_ONE_PASS) continue;
    const users = Array.from(new Set(cons[r.id]));
    if (users.length !== 1) continue;
    const u = graph.nodes[users[0]];
    if (!keep.has(u.id) || !isChain(u, size(r.shape)) || folded.has(u.id) || dead.has(u.id) || aliases.has(u.id)) continue;
    // Elementwise ops of one size only (constants and their broadcasts aside, which the
    // kernel writes as literals): every operand read at the element stored.
    const bodyNodes = u.op === 'fused' ? u.attrs.body.nodes : [];
    if (!bodyNodes.every((x) => x.op === 'const' || (x.op === 'broadcast' && bodyNodes[x.inputs[0]].op === 'const')
      || ((x.op === 'input' || ELEMENTWISE_OPS.has(x.op)) && size(x.shape) === size(r.shape)))) continue;
    if (rowFolds.has(u.id) || colFolds.has(u.id) || absorbed.has(u.id) || broadcasts.has(u.id) || views.has(u.id)) continue;
    folded.add(r.id);
    colFolds.set(u.id, { red: r.id, pos: u.inputs.map((i, k) => (i === r.id ? k : -1)).filter((k) => k >= 0) });
  }
  return { aliases, folded, views, broadcasts, dead, rowFolds, absorbed, colFolds };
}

/** The dense row-major view of an operand of `shape` ([..batch, R, C]). */
function denseView(shape) {
  const st = stridesOf(shape);
  const r = shape.length;
  return { batch: shape.slice(0, r - 2).map((e, d) => [e, st[d]]), sr: st[r - 2], sc: st[r - 1] };
}

/**
 * Relu applied as matmul operands load (perf lowering): a relu whose every live reader
 * takes it as a matmul operand (slot a or b), directly or through transposes and reshapes
 * read in place, launches nothing. Each such matmul reads the relu's own operand through
 * the same view, with `op: 'relu'` on it, and applies relu to every element it loads
 * (tcmi::op_relu, the op the relu kernel would run, so the same bits; a zero-filled tile
 * edge stays 0). Config 5's relu(h·W1 + b1) is one: read by h·W2 and, transposed, by the
 * weight gradient of W2, while the backward pass reads the pre-activation. Updates
 * `folded` and `views` (consumer id -> { slot: { pos, source, view, size } }).
 */
function operandLoadOps(graph, keep, cons, slotOf, dead, folded, views) {
  for (const n of graph.nodes) {
    if (n.op !== 'relu' || keep.has(n.id) || dead.has(n.id) || folded.has(n.id) || n.shape.length < 2) continue;
    const src = n.inputs[0];
    if (folded.has(src) || dead.has(src)) continue;
    const users = cons[n.id].filter((c) => !dead.has(c));
    const direct = [];
    const ok = users.length > 0 && users.every((c) => {
      if (folded.has(c) && graph.nodes[c].op === 'transpose') return true;
      return graph.nodes[c].inputs.every((i, pos) => {
        if (i !== n.id) return true;
        const slot = slotOf.get(`${c}:${pos}`);
        if (slot !== 'a' && slot !== 'b') return false;
        direct.push([c, slot, pos]);
        return true;
      });
    });
    if (!ok) continue;
    const viewed = [];
    for (const slots of views.values()) for (const [slot, v] of Object.entries(slots)) if (v.source === n.id) viewed.push([slot, v]);
    if (viewed.some(([slot]) => slot !== 'a' && slot !== 'b')) continue;
    folded.add(n.id);
    const size_ = size(graph.nodes[src].shape);
    for (const [, v] of viewed) Object.assign(v, { source: src, view: Object.assign({}, v.view, { op: 'relu' }), size: size_, opNode: n.id });
    for (const [c, slot, pos] of direct) {
      if (!views.has(c)) views.set(c, {});
      views.get(c)[slot] = { pos, source: src, view: Object.assign(denseView(n.shape), { op: 'relu' }), size: size_, opNode: n.id };
    }
  }
}

/**
 * The index map of a value read from a source buffer through a chain of transposes and
 * reshapes (`chain`: node ids from the source's reader to the value): per dimension of the
 * value, its factors [[extent, stride], ...] outer to inner, so that index x of the
 * dimension addresses Σ_f ((x / inner_f) % extent_f) · stride_f (inner_f: the product of
 * the extents inside f). A transpose permutes the dimensions; a reshape regroups the
 * factors of the row-major order, splitting one where a new dimension ends inside it.
 * null where a reshape cuts a factor at a point that divides neither way (no such map).
 */
function chainMap(graph, source, chain) {
  const shape = graph.nodes[source].shape;
  const st = stridesOf(shape);
  let dims = shape.map((e, d) => [[e, st[d]]]);
  for (const id of chain) {
    const n = graph.nodes[id];
    if (n.op === 'transpose') {
      dims = n.attrs.perm.map((p) => dims[p]);
      continue;
    }
    const flat = [].concat(...dims).filter(([e]) => e > 1);
    const out = new Array(n.shape.length);
    for (let d = n.shape.length - 1; d >= 0; d--) {
      let E = n.shape[d];
      const fs = [];
      while (E > 1) {
        if (!flat.length) return null;
        const [e, s] = flat.pop();
        if (E % e === 0) { fs.unshift([e, s]); E /= e; } else if (e % E === 0) { fs.unshift([E, s]); flat.push([e / E, s * E]); E = 1; } else return null;
      }
      out[d] = fs;
    }
    if (flat.length) return null;
    dims = out;
  }
  // Adjacent factors that step as one (outer stride = inner extent · inner stride) merge.
  return dims.map((fs) => {
    const m = [];
    for (const [e, s] of fs) {
      const last = m[m.length - 1];
      if (last && last[1] === e * s) m[m.length - 1] = [last[0] * e, s];
      else m.push([e, s]);
    }
    return m.length ? m : [[1, 0]];
  });
}

/**
 * Transposes read in place by matmuls, and the operand views through which they are read.
 * A transpose launches nothing when every consumer reads it as a matmul operand (or is such
 * a transpose itself): the matmul reads the transpose's source through a strided view. A
 * reshape between them (the heads of an attention merged back into rows, transpose(o)
 * reshaped to [B·T, d], and the gradients of q, k and v on their way back) is passed
 * through as well where the readers are plain or epilogue products (operand slots a and
 * b); their view then maps a row or column index over several strides (chainMap). A chain
 * whose reshape no such map expresses keeps its transposes launched. Dead readers (nodes no
 * kept value depends on) launch nothing and do not count.
 * Returns { folded: Set of transposes, views: consumer id -> { slot: { pos, source, view, size } } }.
 */
function inPlaceTransposes(graph, keep, cons, slotOf, dead) {
  const refused = new Set();
  const bySlot = (c, id, ab) => graph.nodes[c].inputs.every((i, pos) => {
    if (i !== id) return true;
    const s = slotOf.get(`${c}:${pos}`);
    return s !== undefined && (!ab || s === 'a' || s === 'b');
  });
  // Whether transpose or reshape `id` is read only through matmul operand slots, directly or
  // through further transposes and reshapes (`via`: a reshape lies on the way).
  const inPlace = (id, via) => {
    const users = cons[id].filter((c) => !dead.has(c));
    if (keep.has(id) || users.length === 0) return false;
    return users.every((c) => {
      const n = graph.nodes[c];
      if (n.op === 'transpose') return !refused.has(c) && inPlace(c, via);
      if (n.op === 'reshape') return inPlace(c, true);
      return bySlot(c, id, via);
    });
  };
  for (;;) {
    const folded = new Set();
    for (const n of graph.nodes) if (n.op === 'transpose' && !refused.has(n.id) && inPlace(n.id, false)) folded.add(n.id);
    const views = new Map();
    let bad = null;
    for (const n of graph.nodes) {
      for (const [slot, pos] of matmulSlots(n)) {
        let cur = n.inputs[pos];
        const chain = [];
        while (folded.has(cur) || (graph.nodes[cur].op === 'reshape' && !keep.has(cur))) {
          chain.push(cur);
          cur = graph.nodes[cur].inputs[0];
        }
        // Reshapes at the source's end read the source's layout as it is: the view starts there.
        while (chain.length && !folded.has(chain[chain.length - 1])) cur = chain.pop();
        if (!chain.length) continue;
        const shape = graph.nodes[n.inputs[pos]].shape;
        const r = shape.length;
        let view;
        if (chain.every((id) => graph.nodes[id].op === 'transpose')) {
          let perm = shape.map((_, d) => d);
          for (const id of chain) perm = perm.map((d) => graph.nodes[id].attrs.perm[d]);
          const st = stridesOf(graph.nodes[cur].shape);
          const s = perm.map((d) => st[d]);
          view = { batch: shape.slice(0, r - 2).map((e, d) => [e, s[d]]), sr: s[r - 2], sc: s[r - 1] };
        } else {
          const dims = chainMap(graph, cur, chain.slice().reverse());
          if (!dims) { bad = chain.filter((id) => folded.has(id)); break; }
          const batch = [].concat(...dims.slice(0, r - 2)).filter(([e]) => e > 1);
          const [rf, cf] = [dims[r - 2], dims[r - 1]];
          view = rf.length === 1 && cf.length === 1 ? { batch, sr: rf[0][1], sc: cf[0][1] } : { batch, sr: null, sc: null, r: rf, c: cf };
        }
        if (!views.has(n.id)) views.set(n.id, {});
        views.get(n.id)[slot] = { pos, source: cur, view, size: size(graph.nodes[cur].shape) };
      }
      if (bad) break;
    }
    if (!bad) return { folded, views };
    for (const id of bad) refused.add(id);
  }
}

/**
 * `w.body` with the input at the positions of each absorbed producer replaced by that
 * producer's body on the producer's own operands (inputs a{ppos[j]}, broadcasts it reads
 * in place widened as for any body, and what it absorbed formed the same way): the
 * reader's kernel forms the producer's value where it would have loaded it. Returns
 * { body, output }.
 */
function absorbProducers(graph, w, absorbs) {
  if (!absorbs) return w;
  const g = new Graph();
  const map = new Map();
  const at = new Map();
  for (const a of absorbs) for (const pos of a.pos) at.set(pos, a);
  const formed = new Map();
  for (const n of w.body.nodes) {
    const a = n.op === 'input' ? at.get(Number(n.attrs.name.slice(1))) : undefined;
    if (a) {
      if (!formed.has(a)) {
        const p = graph.nodes[a.prod];
        const one = p.op === 'fused' ? { body: bodyOf(p), output: p.attrs.output } : oneOpBody(graph, p);
        const pw = absorbProducers(graph, widenInputs(one.body, one.output, a.prodFolds), a.nested);
        const pm = new Map();
        for (const pn of pw.body.nodes) {
          pm.set(pn.id, pn.op === 'input' ? g.input(`a${a.ppos[Number(pn.attrs.name.slice(1))]}`, pn.shape)
            : g.emit(pn.op, pn.inputs.map((i) => pm.get(i)), pn.attrs));
        }
        formed.set(a, pm.get(pw.output));
      }
      map.set(n.id, formed.get(a));
    } else if (n.op === 'input') {
      map.set(n.id, g.input(n.attrs.name, n.shape));
    } else {
      map.set(n.id, g.emit(n.op, n.inputs.map((i) => map.get(i)), n.attrs));
    }
  }
  return { body: g, output: map.get(w.output) };
}

/**
 * `body` with each input at the positions of a fold (a row reduction's value) replaced by
 * that reduction of a new input, in the first of those positions: the reduction's operand
 * read as [outer, n] rows (its reduced axis is the last non-trivial one) and reduced along
 * them, as the plain lowering reduces it, then reshaped to the reduction's own shape — the
 * body of a chain with its reductions folded in.
 */
function foldReductions(body, output, folds) {
  const g = new Graph();
  const map = new Map();
  const at = new Map();
  for (const f of folds) for (const p of f.pos) at.set(p, f);
  const reduced = new Map();
  for (const n of body.nodes) {
    const f = n.op === 'input' ? at.get(Number(n.attrs.name.slice(1))) : undefined;
    if (f) {
      if (!reduced.has(f)) {
        const outer = size(f.inShape.slice(0, f.attrs.axis)), len = f.inShape[f.attrs.axis];
        let src;
        if (f.producer) {
          // The reduction's operand formed in place by its producer's body ([outer, len]).
          const pm = new Map();
          for (const pn of f.producer.body.nodes) {
            pm.set(pn.id, pn.op === 'input' ? g.input(`a${f.producer.ppos[Number(pn.attrs.name.slice(1))]}`, pn.shape)
              : g.emit(pn.op, pn.inputs.map((i) => pm.get(i)), pn.attrs));
          }
          src = pm.get(f.producer.output);
        } else {
          src = g.input(`a${f.pos[0]}`, [outer, len]);
        }
        const r = g.emit(f.op, [src], { axis: 1, keepDims: true });
        reduced.set(f, g.reshape(r, f.shape));
      }
      map.set(n.id, reduced.get(f));
    } else if (n.op === 'input') {
      map.set(n.id, g.input(n.attrs.name, n.shape));
    } else {
      map.set(n.id, g.emit(n.op, n.inputs.map((i) => map.get(i)), n.attrs));
    }
  }
  return { body: g, output: map.get(output) };
}

/**
 * Lower `graph` for the MI355X runner. Options: sabotage (one of the
 * reference's fused-kernel sabotages: 'epilogue-before-bias',
 * 'layernorm-tree-short', 'softmax-no-max', 'fused-bounds-off-by-one'),
 * applied to fused kernels only; tuning ({ ew: { unroll, nt, blocks }, colreduce: { blocks } })
 * overrides the kernels' launch-shape defaults (used by sweeps); perf and
 * keep (node ids) as described at the top of this file; batch: false keeps the
 * perf lowering's launches one dispatch each, in graph order; rowFolds: false keeps
 * every reduction and its producer a launch of their own (an unfused graph measured
 * against its fused form, where a fold would be fusion by another name).
 * Returns { launches, workspace, aliases, folded, dead, batches } (workspace: bytes of
 * scratch the largest launch needs; aliases: [[node, source]]; folded and dead: node
 * ids with neither a launch nor a buffer; batches, perf only: [{ start, count, kernels, wsStride }]).
 */
/** A matmul's shape (batch, M, K, N) as a key — of a plain matmul node or of an epilogue group's matmul — or null. */
function productKey(graph, node) {
  let a, b;
  if (node.op === 'matmul') [a, b] = node.inputs.map((i) => graph.nodes[i].shape);
  else if (node.op === 'fused' && node.attrs.kind === 'epilogue') {
    const body = node.attrs.body;
    const mm = body.nodes.find((n) => n.op === 'matmul');
    [a, b] = mm.inputs.map((i) => body.nodes[i].shape);
  } else return null;
  return `${size(a.slice(0, -2))}x${a[a.length - 2]}x${a[a.length - 1]}x${b[b.length - 1]}`;
}

/** Launch records of folded reductions and absorbed producers (for node-local checks). */
const foldRecords = (rowFold) => rowFold.map((f) => (f.prod === undefined ? { reduction: f.red, pos: f.pos }
  : { reduction: f.red, pos: f.pos, producer: f.prod, producerPos: f.ppos }));
const absorbRecord = (a) => Object.assign({ producer: a.prod, pos: a.pos, producerPos: a.ppos },
  a.nested ? { absorbed: a.nested.map(absorbRecord) } : {});

/** Bytes from which a last read is streamed (non-temporal loads): 1 MiB. */
const STREAM_FROM = 1 << 20;
/** Full rows a launch forming values may hold in registers (its cached operands). */
const FORM_CACHED = 6;
/**
 * The estimate by which the perf lowering forms values (MI355X): a launch takes its bytes
 * at EST_BW, plus its vector work at EST_ALU, plus EST_LAUNCH — added, not overlapped: a
 * config-2 gradient kernel repeating two exp and two tanh per element measured 28.3 us,
 * its bytes alone 16.8 us and its arithmetic 10.9 us by this count. EST_BW lies
 * between the measured copy and read ceilings (5.7 and 6.4 TB/s); EST_ALU is 256 CUs of
 * 4 SIMDs of 16 lanes at 2.4 GHz (a wavefront's instruction over 4 cycles); EST_LAUNCH is
 * about what a launch adds to a replayed step of small kernels.
 */
const EST_BW = 6.0e12;
const EST_ALU = 256 * 4 * 16 * 2.4e9;
const EST_LAUNCH = 2e-6;
/**
 * Vector instructions per element of each op's tcmi:: form: exp, log and the reciprocal
 * behind div and tanh run on the transcendental unit at a quarter of the rate; tanh
 * also clamps, takes |x| and restores the sign. Shape-only ops cost nothing here.
 */
const OP_COST = { exp: 5, log: 10, tanh: 18, div: 5, sqrt: 5, relu: 2, step: 2, neg: 1, add: 1, sub: 1, mul: 1,
  stopGradient: 0, copy: 0, reshape: 0, broadcast: 0, transpose: 0, input: 0, const: 0 };

/**
 * Estimated seconds of one launch running `body` (output `output`) over buffers `ins`
 * (graph `graph` for their sizes). Elementwise bodies compute every node at every
 * output element (a broadcast's source again at each element it is spread to); rowwise
 * bodies compute the elements under each reduction and under the output once per element
 * of the rows, a row value once per row (not counted), and accumulate each reduction once
 * per element.
 */
function launchEstimate(graph, body, output, ins) {
  const lay = rowLayout(body, output);
  const rowwise = !!(lay && lay.R);
  const full = rowwise ? lay.R * lay.C : size(body.nodes[output].shape);
  const rowTier = (n) => rowwise && size(n.shape) === lay.R && lay.R !== full;
  const roots = [output];
  let ops = 0;
  if (rowwise) for (const n of body.nodes) if (isReduce(n)) { roots.push(n.inputs[0]); ops += full; }
  for (const root of roots) {
    const seen = new Set();
    const walk = (id) => {
      const n = body.nodes[id];
      if (seen.has(id) || isReduce(n) || (rowTier(n) && n.op !== 'input')) return;
      seen.add(id);
      ops += (OP_COST[n.op] === undefined ? 1 : OP_COST[n.op]) * full;
      for (const i of n.inputs) walk(i);
    };
    walk(root);
  }
  const bytes = 4 * (ins.reduce((acc, x) => acc + size(graph.nodes[x].shape), 0) + size(body.nodes[output].shape));
  return bytes / EST_BW + ops / EST_ALU + EST_LAUNCH;
}

function lowerMI355X(graph, options) {
  const opts = options || {};
  if (opts.perf && !opts.keep) throw new Error('the perf lowering needs `keep`: the nodes whose values are read');
  // A launch that takes producers in, with their index maps, may need more parameter words
  // than its argument block holds: its reader then takes none in, and the plan is made again.
  // So may a launch forming values: those values are then launched, and the plan is made again.
  const noAbsorb = new Set();
  const noForm = new Set();
  for (;;) {
    try {
      return lowerOnce(graph, opts, noAbsorb, noForm);
    } catch (e) {
      if (e instanceof cg.ParamOverflow && e.formed && e.formed.some((v) => !noForm.has(v))) {
        for (const v of e.formed) noForm.add(v);
        continue;
      }
      if (!(e instanceof cg.ParamOverflow) || e.reader === undefined || noAbsorb.has(e.reader)) throw e;
      noAbsorb.add(e.reader);
    }
  }
}

function lowerOnce(graph, opts, noAbsorb, noForm) {
  const plan = opts.perf ? perfPlan(graph, new Set(opts.keep), opts.rowFolds !== false, opts.absorb === true && opts.rowFolds !== false,
    opts.loadOps !== false, noAbsorb)
    : { aliases: new Map(), folded: new Set(), views: new Map(), broadcasts: new Map(), dead: new Set(), rowFolds: new Map(), absorbed: new Map(),
      colFolds: new Map() };
  const cache = new Map();
  const launches = [];
  let workspace = 0;
  const launched = (node) => node.op !== 'input' && node.op !== 'const' && !plan.aliases.has(node.id)
    && !plan.folded.has(node.id) && !plan.dead.has(node.id);
  const resolve = (id) => (plan.aliases.has(id) ? plan.aliases.get(id) : id);
  // The buffers a launch reads before it forms any value, operand by operand: a reshape's
  // buffer is its source's, and an operand read through a view, a folded broadcast or a
  // folded reduction is read from the node it stands for.
  const baseInputsOf = (node) => {
    const inputs = node.inputs.map(resolve);
    const v = plan.views.get(node.id);
    if (v) for (const s of Object.values(v)) inputs[s.pos] = resolve(s.source);
    const folds = plan.broadcasts.get(node.id);
    if (folds) for (const [pos, f] of folds) inputs[pos] = resolve(f.source);
    const rowFold = plan.rowFolds.get(node.id);
    if (rowFold) {
      for (const f of rowFold) {
        if (f.prod === undefined) {
          for (const pos of f.pos) inputs[pos] = resolve(graph.nodes[f.red].inputs[0]);
          continue;
        }
        // The producer's operands (a broadcast it reads in place: the broadcast's source).
        const p = graph.nodes[f.prod];
        const pins = p.inputs.map((i, j) => resolve(f.prodFolds && f.prodFolds.has(j) ? f.prodFolds.get(j).source : i));
        for (const pos of f.pos) inputs[pos] = pins[0];
        f.ppos.forEach((pos, j) => { inputs[pos] = pins[j]; });
      }
    }
    const colFold = plan.colFolds.get(node.id);
    if (colFold) for (const pos of colFold.pos) inputs[pos] = resolve(graph.nodes[colFold.red].inputs[0]);
    for (const a of plan.absorbed.get(node.id) || []) {
      // An absorbed producer's operands (its own, with what it absorbed), in its positions.
      const pins = baseInputsOf(graph.nodes[a.prod]);
      for (const pos of a.pos) inputs[pos] = pins[0];
      a.ppos.forEach((pos, j) => { inputs[pos] = pins[j]; });
    }
    return inputs;
  };
  // Values formed by their readers (perf lowering, with row folds). A value — full-size or
  // a row value — computed by an elementwise, rowwise or row-statistics launch or a
  // last-axis reduction, kept by nobody, launches nothing where every launch reading it can
  // compute it instead: each such reader forms it inside its own kernel from what the value's
  // launch would have read (its body inlined there, the values that body reads formed in
  // turn), so the value is never written or read back. A reader so formed runs a rowwise
  // kernel where its body then reduces rows (all over rows of one length, its output of
  // full or row size: rowLayout), else an elementwise one; the reductions run with the
  // same lanes and order as in the value's own launch (the rowwise kernel's layout depends
  // on the row length and tuning alone), so every bit is the plain lowering's. A value is
  // formed where that takes no longer by launchEstimate: its own launch and its readers as
  // they are, against the readers forming it. Bytes the readers save (the value's write
  // and read-backs) weigh against the operands they read instead and the arithmetic they
  // repeat, priced by op (LayerNorm's centred rows and statistics, softmax's exponentials
  // and row sums: the backward of a row function then reads x and dy alone; a chain of
  // transcendental ops shared by several readers stays a launch). Values are taken in
  // graph order, so a value's own operands are settled before it.
  // Not under a sabotage (the planted kernel runs alone) or with rowwise and row-reduction
  // tunings that differ (the reductions' lanes would).
  const formedSet = new Set();
  const baseOf = new Map();
  const baseBody = (id) => {
    if (!baseOf.has(id)) {
      const node = graph.nodes[id];
      baseOf.set(id, plan.views.has(id) || plan.colFolds.has(id) ? null : launchBase(graph, node, plan.broadcasts.get(id) || null,
        plan.rowFolds.get(id) || null, plan.absorbed.get(id) || null));
    }
    return baseOf.get(id);
  };
  // Launch `id`'s body with every value of `set` it reads formed inside it (each once: its
  // base body on what it reads), on the buffers left to read: { body, output, ins, values }.
  const compose = (id, set) => {
    const g = new Graph();
    const ins = [];
    const leafAt = new Map();
    const made = new Map();
    let inline;
    const valueOf = (buf) => {
      if (set.has(buf)) {
        if (!made.has(buf)) made.set(buf, inline(buf));
        return made.get(buf);
      }
      if (!leafAt.has(buf)) {
        leafAt.set(buf, g.input(`a${ins.length}`, graph.nodes[buf].shape));
        ins.push(buf);
      }
      return leafAt.get(buf);
    };
    inline = (nid) => {
      const base = baseBody(nid);
      const bins = baseInputsOf(graph.nodes[nid]);
      const map = new Map();
      for (const n of base.body.nodes) {
        map.set(n.id, n.op === 'input' ? g.reshape(valueOf(bins[Number(n.attrs.name.slice(1))]), n.shape)
          : g.emit(n.op, n.inputs.map((i) => map.get(i)), n.attrs));
      }
      return map.get(base.output);
    };
    const output = inline(id);
    return { body: g, output, ins, values: Array.from(made.keys()), made };
  };
  const tune = opts.tuning || {};
  const rowTuningsAlike = !tune.rowreduce || JSON.stringify(tune.rowreduce) === JSON.stringify(tune.row);
  if (opts.perf && opts.rowFolds !== false && opts.formRows !== false && !opts.sabotage && rowTuningsAlike) {
    const keepBufs = new Set(opts.keep.map(resolve));
    const sz = (id) => size(graph.nodes[id].shape);
    const order = graph.nodes.filter(launched);
    // What each launch reads, kept up to date as values are formed.
    const reads = new Map(order.map((n) => [n.id, new Set(baseInputsOf(n))]));
    for (const u of order) {
      if (keepBufs.has(u.id) || noForm.has(u.id) || !baseBody(u.id)) continue;
      const readers = order.filter((r) => r !== u && !formedSet.has(r.id) && reads.get(r.id).has(u.id));
      if (!readers.length || !readers.every((r) => baseBody(r.id))) continue;
      const own = compose(u.id, formedSet);
      if (!rowLayout(own.body, own.output)) continue;
      const est = (c) => launchEstimate(graph, c.body, c.output, c.ins);
      const trial = new Set(formedSet).add(u.id);
      let ok = true, after = 0, before = est(own);
      for (const r of readers) {
        const c = compose(r.id, trial);
        const lay = rowLayout(c.body, c.output);
        // Within the argument block, and at most FORM_CACHED full rows held in registers.
        if (!lay || c.ins.length > cg.MAX_IN || (lay.R && c.ins.filter((x) => sz(x) === lay.R * lay.C).length > FORM_CACHED)) {
          ok = false;
          break;
        }
        after += est(c);
        before += est(compose(r.id, formedSet));
      }
      if (!ok || after > before) continue;
      formedSet.add(u.id);
      for (const r of readers) {
        const set = reads.get(r.id);
        set.delete(u.id);
        for (const x of own.ins) set.add(x);
      }
    }
    for (const id of formedSet) plan.folded.add(id);
  }
  // The launches that form values, and what every launch reads.
  const composed = new Map();
  for (const node of graph.nodes) {
    if (launched(node) && formedSet.size && baseInputsOf(node).some((id) => formedSet.has(id))) composed.set(node.id, compose(node.id, formedSet));
  }
  const inputsOf = (node) => (composed.has(node.id) ? composed.get(node.id).ins : baseInputsOf(node));
  // Last reads (perf lowering): an elementwise or rowwise kernel loads a full-size operand of
  // STREAM_FROM bytes or more non-temporally where no later launch of the list reads
  // that buffer, so data read for the last time streams past the caches instead of
  // displacing data still to be read. A hint only: the values loaded are the same.
  // Smaller buffers stay cached: streaming them saves nothing, and a repeated launch
  // of a small kernel would miss where it hits.
  // Products that may share one dispatch: those whose value no node reads (a trainer's
  // weight gradients with their update epilogues), counted per shape, launched or not.
  // Nothing waits on them, so the perf lowering can issue all of them together; a
  // product that another node reads runs where its readers need it, alone as far as
  // this count can tell (1). The K split of a product depends on its shape and on this
  // count alone, so the plain and the perf lowering of a graph split every product alike.
  const readers = new Set();
  for (const node of graph.nodes) for (const id of node.inputs) readers.add(id);
  const productPeers = new Map();
  for (const node of graph.nodes) {
    const pk = readers.has(node.id) ? null : productKey(graph, node);
    if (pk !== null) productPeers.set(pk, (productPeers.get(pk) || 0) + 1);
  }
  const peersOf = (node) => (readers.has(node.id) ? 1 : productPeers.get(productKey(graph, node)) || 1);
  const lastRead = new Map();
  if (opts.perf) for (const node of graph.nodes) if (launched(node)) for (const id of inputsOf(node)) lastRead.set(id, node.id);
  // Output stores (perf lowering), a hint like the last reads: an output the next launch of
  // the list reads is stored through the caches, where that launch finds it (false); one of
  // STREAM_FROM bytes or more that the next launch does not read is stored non-temporally,
  // so it does not displace what that launch reads (true). The last launch's output is
  // stored non-temporally where the launch streams two or more such operands, and left to
  // the kernel otherwise: measured on the rowwise programs of config 3, the gradients'
  // last launch (reading x and dy) is 11 % faster with non-temporal stores and the
  // forwards' one launch (reading x) 8 % slower. Elementwise kernels store non-temporally
  // unless false, rowwise kernels only if true.
  const streamOut = new Map();
  if (opts.perf) {
    const big = (id) => size(graph.nodes[id].shape) * 4 >= STREAM_FROM;
    const order = graph.nodes.filter(launched);
    order.forEach((node, i) => {
      const next = order[i + 1];
      if (next && inputsOf(next).includes(node.id)) streamOut.set(node.id, false);
      else if (big(node.id) && (next || new Set(inputsOf(node).filter(big)).size >= 2)) streamOut.set(node.id, true);
    });
  }
  for (const node of graph.nodes) {
    if (!launched(node)) continue;
    const v = plan.views.get(node.id);
    let mmViews = null;
    if (v) {
      mmViews = { views: {}, sizes: {} };
      for (const slot of Object.keys(v)) { mmViews.views[slot] = v[slot].view; mmViews.sizes[slot] = v[slot].size; }
    }
    const folds = plan.broadcasts.get(node.id) || null;
    const foldKey = folds ? Array.from(folds.entries()).map(([pos, f]) => [pos, f.from, f.to]) : null;
    const rowFold = plan.rowFolds.get(node.id) || null;
    const prodKey = (f) => {
      if (f.prod === undefined) return null;
      const p = graph.nodes[f.prod];
      return [f.ppos, p.op, p.attrs, p.inputs.map((i) => graph.nodes[i].shape),
        f.prodFolds ? Array.from(f.prodFolds.entries()).map(([pos, b]) => [pos, b.from, b.to]) : null];
    };
    const rowKey = rowFold ? rowFold.map((f) => [f.pos, graph.nodes[f.red].op, graph.nodes[f.red].attrs,
      graph.nodes[graph.nodes[f.red].inputs[0]].shape, prodKey(f)]) : null;
    const colFold = plan.colFolds.get(node.id) || null;
    const colKey = colFold ? [colFold.pos, graph.nodes[colFold.red].attrs, graph.nodes[graph.nodes[colFold.red].inputs[0]].shape] : null;
    const absorbs = plan.absorbed.get(node.id) || null;
    const absorbSig = (a) => [a.pos, prodKey({ prod: a.prod, ppos: a.ppos, prodFolds: a.prodFolds }),
      a.nested ? a.nested.map(absorbSig) : null];
    const absorbKey = absorbs ? absorbs.map(absorbSig) : null;
    // A launch forming values is keyed by the body it runs.
    const comp = composed.get(node.id) || null;
    const formKey = comp ? [comp.body.nodes.map((n) => [n.op, n.inputs, n.attrs, n.shape]), comp.output] : null;
    const inputs = inputsOf(node);
    const lastReads = [];
    inputs.forEach((id, pos) => {
      if (lastRead.get(id) === node.id && size(graph.nodes[id].shape) * 4 >= STREAM_FROM) lastReads.push(pos);
    });
    // Kernels depend on structure, shapes, operand views, folded broadcasts and last
    // reads only: reuse across identical nodes.
    const peers = peersOf(node);
    const key = JSON.stringify([node.op, node.inputs.map((id) => graph.nodes[id].shape), node.attrs, node.shape,
      node.op === 'fused' ? opts.sabotage : null, opts.tuning || null, mmViews, foldKey, rowKey, lastReads, peers, absorbKey, formKey,
      streamOut.get(node.id), colKey]);
    let k = cache.get(key);
    if (!k) {
      try {
        k = lowerNode(graph, node, opts, mmViews, folds, rowFold, lastReads, peers, absorbs, comp, streamOut.get(node.id), colFold);
      } catch (e) {
        if (e instanceof cg.ParamOverflow && comp) e.formed = comp.values;
        else if (e instanceof cg.ParamOverflow && absorbs) e.reader = node.id;
        throw e;
      }
      cache.set(key, k);
    }
    workspace = Math.max(workspace, k.workspace);
    launches.push({
      node: node.id, op: node.op, kind: k.kind, pattern: node.op === 'fused' ? node.attrs.pattern : undefined,
      inputs, params: k.params, grid: k.kernels[0].grid, code: k.kernels[0].name,
      kernels: k.kernels, workspace: k.workspace, bytes: algorithmicBytes(graph, node, inputs), flops: k.flops,
    });
    // For node-local checks: the reductions folded into this launch, the producers it
    // forms in place of loading them, and the values it forms (each with its own folds and
    // absorbed producers, in the order the launch forms them).
    if (rowFold) launches[launches.length - 1].rowFolds = foldRecords(rowFold);
    // A column sum folded into its reader: recorded as a fold over the sum's own axis.
    if (colFold) launches[launches.length - 1].rowFolds = [{ reduction: colFold.red, pos: colFold.pos, columns: true }];
    if (absorbs) launches[launches.length - 1].absorbed = absorbs.map(absorbRecord);
    if (comp) {
      launches[launches.length - 1].formed = comp.values.map((v) => Object.assign({ value: v },
        plan.rowFolds.has(v) ? { rowFolds: foldRecords(plan.rowFolds.get(v)) } : {},
        plan.absorbed.has(v) ? { absorbed: plan.absorbed.get(v).map(absorbRecord) } : {}));
    }
    if (v) {
      // Operands read in place: for each folded slot, the node it stands for and the view of its source.
      launches[launches.length - 1].views = {};
      // A view applying an op on load (view.op) names the node of that op (opNode).
      for (const slot of Object.keys(v)) {
        launches[launches.length - 1].views[slot] = Object.assign({ pos: v[slot].pos, operand: node.inputs[v[slot].pos], source: v[slot].source,
          view: v[slot].view }, v[slot].opNode !== undefined ? { opNode: v[slot].opNode } : {});
      }
    }
  }
  const out = { launches, workspace, aliases: Array.from(plan.aliases.entries()), folded: Array.from(plan.folded), dead: Array.from(plan.dead) };
  if (opts.perf && opts.batch !== false) {
    const b = batchPlan(launches, plan.aliases);
    out.launches = b.launches;
    out.batches = b.batches;
    for (const x of b.batches) out.workspace = Math.max(out.workspace, x.count * x.wsStride);
  }
  return out;
}

/**
 * Batched launches (perf lowering): launches of one kernel family (codegen.js
 * batchFamily) over the same grids with no data path between them run as one dispatch per kernel of the
 * kernels' batched forms (codegen.js batchedKernel). Three passes over the list:
 *   1. walking it in order, a batchable launch opens a batch, and every later
 *      launch of the same kernels whose operands are all written by launches
 *      already placed joins it (up to MAX_BATCH); the members are placed
 *      together where the first one was, each moved only earlier;
 *   2. launches of one kernel still alone are grouped where their windows meet:
 *      a launch may sit anywhere after the last launch writing one of its
 *      operands and before the first launch reading its output, so launches
 *      whose windows share a point (and none of which reads another's output)
 *      are moved together to the first such point (the bias gradients of every
 *      layer, read only by the parameter updates at the end of a step);
 *   3. one-kernel launches of small kernels still alone, whatever their kernels and
 *      grids, are grouped the same way (each window tried in turn as a group's
 *      first) into ragged batches (codegen.js raggedKernel): one dispatch of their
 *      summed workgroups, each member over its own range of them.
 * Every launch thus stays after its operands' writers and before its output's
 * readers, so it reads exactly the values it read in graph order, and writes its
 * own node's buffer (a batch's members each their own workspace slice). A batch
 * runs its launches' kernels over all members in turn (all first kernels, then
 * all second kernels), member k with the workspace slice
 * [k·wsStride, (k + 1)·wsStride). Returns { launches (the new order), batches:
 * [{ start, count, kernels, wsStride, ragged?, joint? }] } with each batch's members at
 * launches[start .. start + count).
 */
function batchPlan(launches, aliases) {
  const owner = (id) => (aliases.has(id) ? aliases.get(id) : id);
  const n = launches.length;
  const writer = new Map();
  launches.forEach((l, i) => writer.set(owner(l.node), i));
  // A launch's kernels as run: a kernel's text does not always fix its grid (a
  // column sum's outer extent is its grid's z extent only).
  // Launches of one kernel family at each position (the same text up to its operand views)
  // may share a dispatch.
  const one = (l) => (l.kernels.every((k) => cg.batchable(k)) ? l.kernels.map((k) => cg.batchFamily(k)).join(' ') : null);
  const fits = (l, count) => l.kernels.every((k) => cg.batchable(k, count));
  // Pass 1: units (arrays of launches; two or more: a batch), in order.
  const placed = new Uint8Array(n);
  const ready = (l) => l.inputs.every((id) => { const w = writer.get(owner(id)); return w === undefined || placed[w] === 1; });
  let units = [];
  // An attention gradient's three parts (the same operands, none reading another) run as
  // one launch of their joint kernel, members in the order dQ, dK, dV, where the first
  // of them stood.
  const jointOf = (l) => l.kernels.length === 1 && l.kernels[0].joint ? l.kernels[0].joint.name : null;
  for (let i = 0; i < n; i++) {
    if (placed[i]) continue;
    const jn = jointOf(launches[i]);
    if (jn) {
      const parts = new Map();
      for (let j = i; j < n; j++) {
        const l = launches[j];
        if (!placed[j] && jointOf(l) === jn && l.inputs.join() === launches[i].inputs.join() && !parts.has(l.kernels[0].part)) {
          parts.set(l.kernels[0].part, j);
        }
      }
      const order = launches[i].kernels[0].joint.parts;
      if (order.every((p) => parts.has(p))) {
        const group = order.map((p) => parts.get(p));
        const unit = group.map((j) => launches[j]);
        unit.joint = launches[i].kernels[0].joint;
        for (const j of group) placed[j] = 1;
        units.push(unit);
        continue;
      }
    }
    const group = [i];
    const name = one(launches[i]);
    if (name) {
      for (let j = i + 1; j < n && group.length < cg.MAX_BATCH; j++) {
        if (!placed[j] && one(launches[j]) === name && ready(launches[j])) group.push(j);
      }
      while (group.length > 1 && !fits(launches[i], group.length)) group.pop();
    }
    for (const j of group) placed[j] = 1;
    units.push(group.map((j) => launches[j]));
  }
  // Passes 2 and 3: group the launches still alone by their windows, those of one key
  // (keyOf: null for a launch that may not join) while `admits` takes the group so far
  // and a new member; `mark` tags each new unit.
  const byWindows = (keyOf, admits, mark, everyStart) => {
    for (let changed = true; changed;) {
      changed = false;
      const unitOf = new Map();   // buffer owner -> index of the unit writing it
      units.forEach((u, x) => { for (const l of u) unitOf.set(owner(l.node), x); });
      const lo = [], hi = [];     // window: after unit lo, before unit hi
      units.forEach((u) => { lo.push(-1); hi.push(units.length); });
      units.forEach((u, x) => {
        for (const l of u) {
          for (const id of l.inputs) {
            const w = unitOf.get(owner(id));
            if (w === undefined) continue;
            lo[x] = Math.max(lo[x], w);
            hi[w] = Math.min(hi[w], x);
          }
        }
      });
      const byKey = new Map();
      units.forEach((u, x) => {
        const k = u.length === 1 ? keyOf(u[0]) : null;
        if (k) { if (!byKey.has(k)) byKey.set(k, []); byKey.get(k).push(x); }
      });
      const reads = (x, y) => units[y][0].inputs.some((id) => unitOf.get(owner(id)) === x);
      for (const xs of byKey.values()) {
        if (xs.length < 2) continue;
        // A lone launch may follow any unit from lo (its operands' last writer) up to,
        // not including, hi (its output's first reader); grow a group from the
        // earliest-opening window (with `everyStart`, from each in turn until a group
        // forms) while the windows still share an anchor.
        const cand = xs.slice().sort((a, b) => lo[a] - lo[b] || a - b);
        for (let s0 = 0; s0 < (everyStart ? cand.length - 1 : 1) && !changed; s0++) {
          const group = [cand[s0]];
          let from = lo[cand[s0]], to = hi[cand[s0]];
          for (const x of cand.slice(s0 + 1)) {
            if (group.length >= cg.MAX_BATCH) break;
            // Anchors a (insert after unit a) with lo <= a < hi, for every member.
            const f = Math.max(from, lo[x]), t = Math.min(to, hi[x]);
            if (f >= t) continue;
            if (group.some((g) => reads(g, x) || reads(x, g))) continue;
            if (!admits(group.map((g) => units[g][0]), units[x][0])) continue;
            group.push(x);
            from = f; to = t;
          }
          while (group.length > 1 && !fits(units[group[0]][0], group.length)) group.pop();
          if (group.length < 2) continue;
          // Place the group right after unit `from` (the latest writer of any member's
          // operand): every member's readers come after it, at `to` or later.
          const members = group.slice().sort((a, b) => a - b).map((x) => units[x][0]);
          if (mark) mark(members);
          const inGroup = new Set(group);
          const next = [];
          if (from < 0) next.push(members);
          units.forEach((u, x) => {
            if (!inGroup.has(x)) next.push(u);
            if (x === from) next.push(members);
          });
          units = next;
          changed = true;
        }
        if (changed) break;
      }
    }
  };
  byWindows(one, () => true, null, false);
  // Pass 3 (ragged batches): single-kernel launches of any kernels that may share a
  // dispatch whose members' grids differ (codegen.js raggedKernel) and still stand alone.
  const raggedKey = (l) => (l.kernels.length === 1 && !l.workspace && cg.raggable(l.kernels[0]) ? `ragged@${l.kernels[0].block[0]}` : null);
  byWindows(raggedKey, (group, l) => cg.raggedFits(group.concat([l]).map((m) => m.kernels[0])), (members) => { members.ragged = true; }, true);
  const order = [], batches = [];
  for (const u of units) {
    if (u.joint) {
      const j = u.joint;
      batches.push({ start: order.length, count: u.length, kernels: [{ name: j.name, source: j.source, grid: j.grid, block: j.block, lds: j.lds }],
        wsStride: 0, joint: true });
      order.push(...u);
      continue;
    }
    if (u.length > 1 && u.ragged) {
      batches.push({ start: order.length, count: u.length, kernels: [cg.raggedKernel(u.map((m) => m.kernels[0]))], wsStride: 0, ragged: true });
    } else if (u.length > 1) {
      const l = u[0];
      batches.push({ start: order.length, count: u.length, kernels: l.kernels.map((k, j) => cg.batchedKernel(u.map((m) => m.kernels[j]), u.length)),
        wsStride: l.workspace ? Math.ceil(l.workspace / 256) * 256 : 0 });
    }
    order.push(...u);
  }
  return { launches: order, batches };
}

/** Every distinct kernel source of a launch list (its batched kernels included), in first-use order. */
function kernelSources(lowered) {
  const seen = new Map();
  for (const l of lowered.launches) for (const k of l.kernels) if (!seen.has(k.name)) seen.set(k.name, k.source);
  for (const b of lowered.batches || []) for (const k of b.kernels) if (!seen.has(k.name)) seen.set(k.name, k.source);
  return seen;
}

module.exports = { lowerMI355X, kernelSources, batchPlan, lowerNode, oneOpBody, algorithmicBytes, chainMap };
