'use strict';
// The fusion-group contract: an IR-to-IR pass that replaces groups of nodes by
// one `fused` node each. A fused node's attrs hold its body, an ordinary graph
// whose inputs a0, a1, ... are the fused node's operands; `kind` is
// 'elementwise', 'epilogue' (a matmul whose only consumer is such a group, of
// its shape) or 'rowwise' (last-axis sum/max whose row results come back
// through broadcast), and `pattern` labels it for reporting.
//
// This is the contract of src/fusion/fuse.js in abho7/tensor-compiler-webgpu
// (grow :54-169, label :172-180, body :183-199, fuse :215-292), restated so the
// MI355X backend is driven by exactly the groups the reference forms: at most
// MAX_OPERANDS = 6 operands per group (a WebGPU binding limit the contract
// keeps), no recompute unless asked, a producer joins only when every consumer
// is already in the group, epilogue operands always stored values, rowwise
// groups only for rows longer than one. The grouping order (sinks from the
// last node down, a fixpoint over members in insertion order) is kept, since
// it decides the partition. Pure JavaScript: nothing here touches a GPU.

const { Graph } = require('../ir/graph');
const { size, sameShape } = require('../ir/shapes');

const ELEMENTWISE = new Set(['add', 'sub', 'mul', 'div', 'neg', 'exp', 'log', 'relu', 'tanh', 'sqrt', 'step', 'stopGradient']);
const MOVES = new Set(['broadcast', 'reshape', 'transpose']);
const MAX_OPERANDS = 6;
const PATTERNS = ['elementwise', 'epilogue', 'rowwise'];

const fround32 = Math.fround;

/** A scalar constant: one finite float32 value, whatever its shape (fuse.js:27-34). */
function scalarConst(node) {
  if (node.op !== 'const') return false;
  const v = node.attrs.value;
  const first = typeof v === 'number' ? v : v[0];
  if (!Number.isFinite(fround32(first))) return false;
  if (typeof v === 'number') return true;
  for (const x of v) if (!Object.is(x, first)) return false;
  return true;
}

const constValue = (node) => (typeof node.attrs.value === 'number' ? node.attrs.value : node.attrs.value[0]);

function consumersOf(graph) {
  const c = graph.nodes.map(() => []);
  for (const n of graph.nodes) for (const i of new Set(n.inputs)) c[i].push(n.id);
  return c;
}

const lastAxisReduce = (graph, n) => (n.op === 'sum' || n.op === 'max') && n.attrs.keepDims
  && n.attrs.axis === graph.nodes[n.inputs[0]].shape.length - 1;

const rowShape = (s) => s.slice(0, -1).concat([1]);

/** Grow one group from `sink`; returns { members, kind, root } or null. */
function grow(graph, sink, consumers, taken, keep, opts) {
  const { patterns, recompute, maxOperands, sabotage } = opts;
  const nodes = graph.nodes;
  const S = nodes[sink].shape;
  const n = size(S);
  const members = new Set([sink]);
  let kind = 'elementwise';
  let root = null;
  const C = S[S.length - 1];
  const isRowShape = (s) => s.length === S.length && sameShape(s, rowShape(S));

  const free = (id) => !taken.has(id) || recompute;
  const allIn = (id, extra) => consumers[id].every((c) => members.has(c) || (extra !== undefined && extra.has(c)));
  const exclusive = (id, extra) => !keep.has(id) && (recompute || allIn(id, extra) || sabotage === 'fusion-absorbs-shared');

  const operandsOf = (set) => {
    const ext = new Set();
    for (const m of set) {
      const node = nodes[m];
      if (node.op === 'const') continue;
      for (const i of node.inputs) if (!set.has(i)) ext.add(i);
    }
    return ext;
  };
  const fits = (set) => operandsOf(set).size <= maxOperands;

  // The row region feeding row-broadcast `b`: row-tier elementwise ops, scalar
  // constants and last-axis reductions of element-tier values (fuse.js:83-107).
  const rowRegion = (b) => {
    const region = new Set();
    let reductions = 0;
    const stack = [nodes[b].inputs[0]];
    while (stack.length) {
      const id = stack.pop();
      if (region.has(id) || members.has(id)) continue;
      const node = nodes[id];
      if (scalarConst(node)) { region.add(id); continue; }
      if (node.op === 'broadcast' && scalarConst(nodes[node.inputs[0]])) { region.add(id); region.add(node.inputs[0]); continue; }
      if (!isRowShape(node.shape) || !free(id)) continue;
      if (lastAxisReduce(graph, node) && sameShape(nodes[node.inputs[0]].shape, S)) {
        region.add(id);
        reductions++;
        continue;
      }
      if (ELEMENTWISE.has(node.op) || node.op === 'stopGradient') {
        region.add(id);
        for (const i of node.inputs) stack.push(i);
      }
    }
    if (!reductions) return null;
    const extra = new Set(region);
    extra.add(b);
    for (const id of region) {
      if (!scalarConst(nodes[id]) && nodes[id].op !== 'broadcast' && !exclusive(id, extra)) return null;
    }
    return region;
  };

  const tryAdd = (list) => {
    const next = new Set(members);
    for (const id of list) next.add(id);
    if (!fits(next)) return false;
    for (const id of list) members.add(id);
    return true;
  };

  let changed = true;
  while (changed) {
    changed = false;
    for (const m of Array.from(members)) {
      const mNode = nodes[m];
      if (mNode.op === 'const' || m === root || mNode.op === 'broadcast' || mNode.op === 'transpose') continue;
      const rowTier = kind === 'rowwise' && !lastAxisReduce(graph, mNode) && mNode.op !== 'broadcast' && isRowShape(mNode.shape);
      for (const p of new Set(mNode.inputs)) {
        if (members.has(p)) continue;
        // A matmul epilogue's own operands are read at arbitrary indices: stored values, never members.
        if (root !== null && nodes[root].inputs.includes(p)) continue;
        const pn = nodes[p];
        if (scalarConst(pn)) { changed = tryAdd([p]) || changed; continue; }
        if (pn.op === 'broadcast' && scalarConst(nodes[pn.inputs[0]])) { changed = tryAdd([p, pn.inputs[0]]) || changed; continue; }
        if (!free(p) || !exclusive(p)) continue;
        if (ELEMENTWISE.has(pn.op) || pn.op === 'reshape') {
          changed = tryAdd([p]) || changed;
          continue;
        }
        if ((pn.op === 'broadcast' || pn.op === 'transpose') && mNode.op !== 'broadcast' && mNode.op !== 'transpose') {
          const src = nodes[pn.inputs[0]];
          if (pn.op === 'broadcast' && patterns.includes('rowwise') && root === null && !rowTier
            && sameShape(pn.shape, S) && isRowShape(src.shape) && C > 1) {
            const region = rowRegion(p);
            if (region && tryAdd([p].concat(Array.from(region)))) { kind = 'rowwise'; changed = true; continue; }
          }
          if (recompute && kind !== 'rowwise' && ELEMENTWISE.has(src.op) && free(src.id) && !keep.has(src.id)) {
            if (tryAdd([p, src.id])) { changed = true; continue; }
          }
          changed = tryAdd([p]) || changed;
          continue;
        }
        if (pn.op === 'matmul' && patterns.includes('epilogue') && kind === 'elementwise' && root === null
          && size(pn.shape) === n && !rowTier && !pn.inputs.some((i) => members.has(i))) {
          if (tryAdd([p])) { kind = 'epilogue'; root = p; changed = true; }
          continue;
        }
      }
    }
  }
  if (kind === 'elementwise' && !patterns.includes('elementwise')) return null;
  let real = 0;
  for (const id of members) if (nodes[id].op !== 'const') real++;
  if (real < 2) return null;
  return { members, kind, root };
}

/** The label a group is reported under (fuse.js:172-180). */
function label(graph, members, kind) {
  if (kind !== 'rowwise') return kind === 'epilogue' ? 'matmul-epilogue' : 'elementwise';
  const counts = {};
  for (const id of members) { const op = graph.nodes[id].op; counts[op] = (counts[op] || 0) + 1; }
  const count = (op) => counts[op] || 0;
  if (count('sum') >= 2 && count('sqrt') >= 1) return 'layernorm';
  if (count('max') >= 1 && count('exp') >= 1 && count('sum') >= 1 && count('log') >= 1) return 'log-softmax';
  if (count('max') >= 1 && count('exp') >= 1 && count('sum') >= 1 && count('div') >= 1) return 'softmax';
  return 'rowwise';
}

/** The body graph of a group: inputs a0.. for its operands, then its members in id order (fuse.js:183-199). */
function body(graph, members, sink) {
  const g = new Graph();
  const order = Array.from(members).sort((a, b) => a - b);
  const operands = [];
  const map = new Map();
  for (const id of order) {
    const node = graph.nodes[id];
    for (const i of node.inputs) {
      if (!members.has(i) && !map.has(i)) {
        map.set(i, g.input(`a${operands.length}`, graph.nodes[i].shape));
        operands.push(i);
      }
    }
    map.set(id, g.emit(node.op, node.inputs.map((i) => map.get(i)), node.attrs));
  }
  return { graph: g, operands, output: map.get(sink) };
}

const bodies = new WeakMap();
/** The body of a fused node as a Graph (cached per node object). */
function bodyOf(node) {
  let b = bodies.get(node);
  if (!b) { b = Graph.fromJSON(node.attrs.body); bodies.set(node, b); }
  return b;
}

/**
 * Fuse `graph`. Options: patterns, recompute (false), keep (ids that must
 * survive), maxOperands (6), sabotage ('fusion-absorbs-shared'), and
 * attention (false: this backend's extension, attention.js, applied after the
 * contract's own pass).
 * Returns { graph, origin, index, groups }: origin[newId] = original id, and
 * index maps each surviving original id to its new id (fuse.js:215-292).
 */
function fuse(graph, options) {
  const o = options || {};
  const fused = fuseContract(graph, o);
  if (!o.attention) return fused;
  return require('./attention').fuseAttention(fused, { keep: o.keep });
}

function fuseContract(graph, options) {
  const o = options || {};
  const patterns = o.patterns || PATTERNS;
  const recompute = !!o.recompute;
  const keep = o.keep || [];
  const maxOperands = o.maxOperands === undefined ? MAX_OPERANDS : o.maxOperands;
  const sabotage = o.sabotage;
  const nodes = graph.nodes;
  const consumers = consumersOf(graph);
  const keepSet = new Set(keep);
  const taken = new Set();
  const groups = [];
  const sinkOf = new Map();
  for (let id = nodes.length - 1; id >= 0; id--) {
    const node = nodes[id];
    if (taken.has(id) || !ELEMENTWISE.has(node.op)) continue;
    const gr = grow(graph, id, consumers, taken, keepSet, { patterns, recompute, maxOperands, sabotage });
    if (!gr) continue;
    for (const m of gr.members) {
      const mn = nodes[m];
      if (mn.op !== 'const' && !(mn.op === 'broadcast' && scalarConst(nodes[mn.inputs[0]]))) taken.add(m);
    }
    const group = { sink: id, members: gr.members, kind: gr.kind, root: gr.root, pattern: label(graph, gr.members, gr.kind) };
    groups.push(group);
    sinkOf.set(id, group);
  }

  const rewire = new Map();
  if (sabotage === 'fusion-absorbs-shared') {
    for (const gr of groups) {
      for (const m of gr.members) {
        if (m === gr.sink || nodes[m].op === 'const') continue;
        if (consumers[m].some((c) => !gr.members.has(c))) rewire.set(m, gr.sink);
      }
    }
  }
  const via = (id) => (rewire.has(id) ? rewire.get(id) : id);

  const needed = new Set();
  const built = new Map();
  for (let id = nodes.length - 1; id >= 0; id--) {
    const node = nodes[id];
    if (consumers[id].length === 0 || keepSet.has(id)) needed.add(id);
    if (!needed.has(id)) continue;
    if (sinkOf.has(id)) {
      const b = body(graph, sinkOf.get(id).members, id);
      built.set(id, b);
      for (const op of b.operands) needed.add(via(op));
    } else {
      for (const i of node.inputs) needed.add(via(i));
    }
  }

  const out = new Graph();
  const index = new Map();
  const origin = [];
  const ref = (id) => {
    const r = via(id);
    if (!index.has(r)) throw new Error(`fuse: node ${r} used before it is built`);
    return index.get(r);
  };
  for (const node of nodes) {
    if (!needed.has(node.id)) continue;
    let id;
    if (built.has(node.id)) {
      const gr = sinkOf.get(node.id);
      const b = built.get(node.id);
      id = out.nodes.length;
      out.nodes.push({ id, op: 'fused', inputs: b.operands.map(ref),
        attrs: { kind: gr.kind, pattern: gr.pattern, body: b.graph.toJSON(), output: b.output }, shape: node.shape.slice() });
    } else if (rewire.size && node.op !== 'input' && node.op !== 'const') {
      id = out.nodes.length;
      out.nodes.push({ id, op: node.op, inputs: node.inputs.map(ref), attrs: JSON.parse(JSON.stringify(node.attrs)), shape: node.shape.slice() });
    } else {
      id = out.emit(node.op, node.inputs.map(ref), node.attrs);
    }
    index.set(node.id, id);
    origin[id] = node.id;
  }
  return { graph: out, origin, index, groups };
}

/** Counts of fused nodes by pattern and the launches before and after (fuse.js:333-338). */
function fusionSummary(original, fused) {
  const launches = (g) => g.nodes.filter((n) => n.op !== 'input' && n.op !== 'const').length;
  const byPattern = {};
  for (const n of fused.graph.nodes) if (n.op === 'fused') byPattern[n.attrs.pattern] = (byPattern[n.attrs.pattern] || 0) + 1;
  return { launchesBefore: launches(original), launchesAfter: launches(fused.graph), byPattern };
}

module.exports = { fuse, bodyOf, scalarConst, constValue, fusionSummary, ELEMENTWISE, MOVES, MAX_OPERANDS, PATTERNS };
