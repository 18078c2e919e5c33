'use strict';
// The fusion-group contract: an IR-to-IR pass that replaces groups of nodes by one
// `fused` node each, whose attrs hold the group's body — an ordinary graph over
// inputs a0, a1, ... that stand for the fused node's operands — its `kind`
// ('elementwise', 'epilogue': a matmul feeding such a group, 'rowwise': last-axis
// sum/max whose row results come back through broadcasts) and a reporting `pattern`.
//
// The contract is the reference's (src/fusion/fuse.js in abho7/tensor-compiler-webgpu,
// grouping :54-169, labels :172-180, bodies :183-199, the pass :215-292), since the
// MI355X backend must be handed exactly the groups the reference forms. Its rules:
//   - groups are seeded at elementwise sinks, from the last node of the graph down;
//     a node already in a group is not seeded or taken again (unless `recompute`);
//   - a group grows to a fixpoint: each round visits the members (in the order they
//     joined, as they were at the round's start) and offers each member's distinct
//     operands in order; an offer that would give the group more than MAX_OPERANDS
//     outside operands is refused, and may succeed in a later round;
//   - a producer joins only if no kept value is it and every consumer of it is
//     already a member (both waived by `recompute`);
//   - scalar constants (and broadcasts of them) join freely; elementwise ops and
//     reshapes join; a broadcast or transpose joins as an indexed load of its
//     source, or — a row value broadcast back over [.., C > 1] rows — brings in the
//     row region that computes it (the rowwise kind), or — with `recompute` — brings
//     in an elementwise source, evaluated at the source index;
//   - a matmul of the group's size joins as the root of an epilogue group, whose
//     own operands then stay stored values; a rowwise group takes no matmul;
//   - a group of fewer than two non-constant members is no group.
// Pure JavaScript: nothing here touches a GPU.

const { Graph } = require('../ir/graph');
const { size, sameShape } = require('../ir/shapes');

const ELEMENTWISE = new Set(['add', 'sub', 'mul', 'div', 'neg', 'exp', 'log', 'relu', 'tanh', 'sqrt', 'step', 'stopGradient']);
const MOVES = new Set(['broadcast', 'reshape', 'transpose']);
const MAX_OPERANDS = 6;
const PATTERNS = ['elementwise', 'epilogue', 'rowwise'];

/** The one value of a constant node (a number, or the first of its list). */
const constValue = (node) => (typeof node.attrs.value === 'number' ? node.attrs.value : node.attrs.value[0]);

/**
 * A constant whose elements are all one finite float32 value: inlined into kernel text
 * as a literal, so it may join any group.
 */
function scalarConst(node) {
  if (node.op !== 'const') return false;
  const first = constValue(node);
  if (!Number.isFinite(Math.fround(first))) return false;
  const v = node.attrs.value;
  return typeof v === 'number' || v.every((x) => Object.is(x, first));
}

/** A broadcast of a scalar constant (built by the builder for `x op const`). */
function broadcastConst(graph, node) {
  return node.op === 'broadcast' && scalarConst(graph.nodes[node.inputs[0]]);
}

/** A sum or max over the last axis that keeps it: a row reduction. */
function isRowReduction(graph, node) {
  if (node.op !== 'sum' && node.op !== 'max') return false;
  return node.attrs.keepDims && node.attrs.axis === graph.nodes[node.inputs[0]].shape.length - 1;
}

/** One growing group, seeded at `sink`. */
class Group {
  constructor(planner, sink) {
    this.p = planner;
    this.nodes = planner.graph.nodes;
    this.sink = sink;
    this.members = new Set([sink]);
    this.kind = 'elementwise';
    this.root = null;
    const S = this.nodes[sink].shape;
    this.elems = size(S);
    this.cols = S[S.length - 1];
    this.rowShape = S.slice(0, -1).concat([1]);
    this.shape = S;
  }

  /** The row tier of a rowwise group: shape [.., 1] of the sink's rank. */
  isRowTier(shape) { return shape.length === this.shape.length && sameShape(shape, this.rowShape); }

  /** Not yet in another group (or recomputation allowed). */
  available(id) { return this.p.recompute || !this.p.claimed.has(id); }

  /** May leave the outside: not kept, and every consumer inside (or in `extra`), or recomputed. */
  absorbable(id, extra) {
    if (this.p.keep.has(id)) return false;
    if (this.p.recompute || this.p.sabotage === 'fusion-absorbs-shared') return true;
    return this.p.users[id].every((u) => this.members.has(u) || (extra !== undefined && extra.has(u)));
  }

  /** Number of distinct outside values the non-constant members of `set` read. */
  outsideOperands(set) {
    const outside = new Set();
    for (const id of set) {
      const node = this.nodes[id];
      if (node.op === 'const') continue;
      for (const i of node.inputs) if (!set.has(i)) outside.add(i);
    }
    return outside.size;
  }

  /** Add `ids` if the group then reads at most MAX_OPERANDS outside values. */
  admit(ids) {
    const next = new Set(this.members);
    for (const id of ids) next.add(id);
    if (this.outsideOperands(next) > this.p.maxOperands) return false;
    for (const id of ids) this.members.add(id);
    return true;
  }

  /**
   * The nodes that compute the row value broadcast by `b` (row tier to element tier):
   * row-tier elementwise ops, scalar constants (bare or broadcast), and row reductions
   * of element-tier values, walked depth first from b's source; anything else stays an
   * outside operand read at the row index. Null unless the region holds a reduction
   * and every op in it may leave the outside.
   */
  rowRegion(b) {
    const region = new Set();
    let reductions = 0;
    const todo = [this.nodes[b].inputs[0]];
    while (todo.length) {
      const id = todo.pop();
      if (region.has(id) || this.members.has(id)) continue;
      const node = this.nodes[id];
      if (scalarConst(node)) { region.add(id); continue; }
      if (broadcastConst(this.p.graph, node)) { region.add(id); region.add(node.inputs[0]); continue; }
      if (!this.isRowTier(node.shape) || !this.available(id)) continue;
      if (isRowReduction(this.p.graph, node) && sameShape(this.nodes[node.inputs[0]].shape, this.shape)) {
        region.add(id);
        reductions += 1;
      } else if (ELEMENTWISE.has(node.op)) {
        region.add(id);
        for (const i of node.inputs) todo.push(i);
      }
    }
    if (reductions === 0) return null;
    const inside = new Set(region).add(b);
    for (const id of region) {
      const node = this.nodes[id];
      if (scalarConst(node) || node.op === 'broadcast') continue;
      if (!this.absorbable(id, inside)) return null;
    }
    return region;
  }

  /**
   * Offer `p`, an operand of a member m; true if the group changed. `mRowTier`: m is a
   * row-tier op of a rowwise group (as the group stood when m's offers began).
   */
  offer(p, mRowTier) {
    const nodes = this.nodes;
    const pn = nodes[p];
    if (this.root !== null && nodes[this.root].inputs.includes(p)) return false;   // epilogue operands stay stored
    if (scalarConst(pn)) return this.admit([p]);
    if (broadcastConst(this.p.graph, pn)) return this.admit([p, pn.inputs[0]]);
    if (!this.available(p) || !this.absorbable(p)) return false;
    if (ELEMENTWISE.has(pn.op) || pn.op === 'reshape') return this.admit([p]);
    if (pn.op === 'broadcast' || pn.op === 'transpose') {
      const src = nodes[pn.inputs[0]];
      if (pn.op === 'broadcast' && this.p.patterns.includes('rowwise') && this.root === null && !mRowTier
        && sameShape(pn.shape, this.shape) && this.isRowTier(src.shape) && this.cols > 1) {
        const region = this.rowRegion(p);
        if (region && this.admit([p].concat(Array.from(region)))) { this.kind = 'rowwise'; return true; }
      }
      if (this.p.recompute && this.kind !== 'rowwise' && ELEMENTWISE.has(src.op) && this.available(src.id) && !this.p.keep.has(src.id)) {
        if (this.admit([p, src.id])) return true;
      }
      return this.admit([p]);
    }
    if (pn.op === 'matmul' && this.p.patterns.includes('epilogue') && this.kind === 'elementwise' && this.root === null
      && size(pn.shape) === this.elems && !mRowTier && !pn.inputs.some((i) => this.members.has(i))) {
      if (this.admit([p])) { this.kind = 'epilogue'; this.root = p; return true; }
    }
    return false;
  }

  /** Grow to a fixpoint; returns { members, kind, root } or null. */
  grow() {
    const nodes = this.nodes;
    let changed = true;
    while (changed) {
      changed = false;
      for (const m of Array.from(this.members)) {
        const mn = nodes[m];
        // Constants, the root and gathers offer nothing: a gather is a load of its source,
        // or its source joined with it.
        if (mn.op === 'const' || m === this.root || mn.op === 'broadcast' || mn.op === 'transpose') continue;
        // A row-tier member of a rowwise group reads the row tier (a reduction reads the element tier).
        const mRowTier = this.kind === 'rowwise' && !isRowReduction(this.p.graph, mn) && this.isRowTier(mn.shape);
        for (const p of new Set(mn.inputs)) {
          if (this.members.has(p)) continue;
          if (this.offer(p, mRowTier)) changed = true;
        }
      }
    }
    if (this.kind === 'elementwise' && !this.p.patterns.includes('elementwise')) return null;
    let ops = 0;
    for (const id of this.members) if (nodes[id].op !== 'const') ops += 1;
    return ops < 2 ? null : { members: this.members, kind: this.kind, root: this.root };
  }
}

/** The pattern a group is reported under: its kind, or for rowwise groups what it computes. */
function patternOf(graph, members, kind) {
  if (kind === 'epilogue') return 'matmul-epilogue';
  if (kind !== 'rowwise') return 'elementwise';
  const n = {};
  for (const id of members) { const op = graph.nodes[id].op; n[op] = (n[op] || 0) + 1; }
  const has = (op, k) => (n[op] || 0) >= (k || 1);
  if (has('sum', 2) && has('sqrt')) return 'layernorm';
  if (has('max') && has('exp') && has('sum') && has('log')) return 'log-softmax';
  if (has('max') && has('exp') && has('sum') && has('div')) return 'softmax';
  return 'rowwise';
}

/**
 * The body graph of a group: an input a<k> for each outside value in order of first
 * use (members visited in id order, operands in order), then every member in id order
 * with its own attributes. Returns { graph, operands (outside ids), output (body id of
 * the sink) }.
 */
function buildBody(graph, members, sink) {
  const g = new Graph();
  const here = new Map();
  const operands = [];
  const ordered = Array.from(members).sort((x, y) => x - y);
  for (const id of ordered) {
    const node = graph.nodes[id];
    for (const i of node.inputs) {
      if (members.has(i) || here.has(i)) continue;
      here.set(i, g.input(`a${operands.length}`, graph.nodes[i].shape));
      operands.push(i);
    }
    here.set(id, g.emit(node.op, node.inputs.map((i) => here.get(i)), node.attrs));
  }
  return { graph: g, operands, output: here.get(sink) };
}

const bodyCache = new WeakMap();
/** The body of a fused node as a Graph (cached per node object). */
function bodyOf(node) {
  let b = bodyCache.get(node);
  if (!b) {
    b = Graph.fromJSON(node.attrs.body);
    bodyCache.set(node, b);
  }
  return b;
}

/** The fusion planner over one graph: the groups, seeded from the last node down. */
class Planner {
  constructor(graph, o) {
    this.graph = graph;
    this.patterns = o.patterns || PATTERNS;
    this.recompute = !!o.recompute;
    this.keep = new Set(o.keep || []);
    this.maxOperands = o.maxOperands === undefined ? MAX_OPERANDS : o.maxOperands;
    this.sabotage = o.sabotage;
    // Consumers of each node, once per consuming node.
    this.users = graph.nodes.map(() => []);
    for (const n of graph.nodes) for (const i of new Set(n.inputs)) this.users[i].push(n.id);
    this.claimed = new Set();
  }

  plan() {
    const groups = [];
    const nodes = this.graph.nodes;
    for (let sink = nodes.length - 1; sink >= 0; sink--) {
      if (this.claimed.has(sink) || !ELEMENTWISE.has(nodes[sink].op)) continue;
      const g = new Group(this, sink).grow();
      if (!g) continue;
      // Shared scalar constants (and their broadcasts) stay free for other groups.
      for (const m of g.members) {
        const mn = nodes[m];
        if (mn.op !== 'const' && !broadcastConst(this.graph, mn)) this.claimed.add(m);
      }
      groups.push({ sink, members: g.members, kind: g.kind, root: g.root, pattern: patternOf(this.graph, g.members, g.kind) });
    }
    return groups;
  }
}

/**
 * Fuse `graph`. Options: patterns (all three), recompute (false), keep (ids that must
 * survive, e.g. a step's outputs), maxOperands (6), sabotage ('fusion-absorbs-shared':
 * the reference's planted pass error), and attention (false: this backend's extension,
 * fusion/attention.js, applied after the contract's own pass).
 * Returns { graph, origin, index, groups }: origin[new id] = original id, and index maps
 * every surviving original id to its new id.
 */
function fuse(graph, options) {
  const o = options || {};
  const fused = fuseContract(graph, o);
  if (!o.attention) return fused;
  return require('./attention').fuseAttention(fused, { keep: o.keep });
}

function fuseContract(graph, o) {
  const planner = new Planner(graph, o);
  const groups = planner.plan();
  const nodes = graph.nodes;
  const users = planner.users;
  const keep = planner.keep;
  const groupAt = new Map(groups.map((g) => [g.sink, g]));

  // The planted pass error: a member still used outside its group is treated as gone,
  // and that outside use is pointed at the group's output instead.
  const redirect = new Map();
  if (o.sabotage === 'fusion-absorbs-shared') {
    for (const g of groups) {
      for (const m of g.members) {
        if (m !== g.sink && nodes[m].op !== 'const' && users[m].some((u) => !g.members.has(u))) redirect.set(m, g.sink);
      }
    }
  }
  const target = (id) => (redirect.has(id) ? redirect.get(id) : id);

  // Survivors: the graph's results (values nobody consumes, and `keep`), and, walking
  // back, the operands of every survivor (a group's outside operands for its sink).
  const survives = new Set();
  const bodies = new Map();
  for (let id = nodes.length - 1; id >= 0; id--) {
    if (users[id].length === 0 || keep.has(id)) survives.add(id);
    if (!survives.has(id)) continue;
    const g = groupAt.get(id);
    if (g) {
      const b = buildBody(graph, g.members, id);
      bodies.set(id, b);
      for (const x of b.operands) survives.add(target(x));
    } else {
      for (const x of nodes[id].inputs) survives.add(target(x));
    }
  }

  // Emission in the original order: a fused node per surviving group sink, the other
  // survivors as they were, every operand renumbered.
  const out = new Graph();
  const index = new Map();
  const origin = [];
  const renumber = (id) => {
    const t = target(id);
    if (!index.has(t)) throw new Error(`fuse: operand ${t} is read before its node is emitted`);
    return index.get(t);
  };
  const append = (node) => { out.nodes.push(node); return node.id; };
  for (const node of nodes) {
    if (!survives.has(node.id)) continue;
    const id = out.nodes.length;
    const g = groupAt.get(node.id);
    if (g) {
      const b = bodies.get(node.id);
      append({ id, op: 'fused', inputs: b.operands.map(renumber),
        attrs: { kind: g.kind, pattern: g.pattern, body: b.graph.toJSON(), output: b.output }, shape: node.shape.slice() });
    } else if (redirect.size && node.op !== 'input' && node.op !== 'const') {
      // The sabotaged pass does not re-check shapes: a redirected operand may not fit.
      append({ id, op: node.op, inputs: node.inputs.map(renumber), attrs: JSON.parse(JSON.stringify(node.attrs)), shape: node.shape.slice() });
    } else {
      out.emit(node.op, node.inputs.map(renumber), node.attrs);
    }
    index.set(node.id, id);
    origin[id] = node.id;
  }
  return { graph: out, origin, index, groups };
}

/** Fused nodes by pattern, and the launches (non-input, non-constant nodes) before and after. */
function fusionSummary(original, fused) {
  const launches = (g) => g.nodes.reduce((c, n) => c + (n.op !== 'input' && n.op !== 'const' ? 1 : 0), 0);
  const byPattern = {};
  for (const n of fused.graph.nodes) if (n.op === 'fused') byPattern[n.attrs.pattern] = (byPattern[n.attrs.pattern] || 0) + 1;
  return { launchesBefore: launches(original), launchesAfter: launches(fused.graph), byPattern };
}

module.exports = { fuse, bodyOf, scalarConst, constValue, fusionSummary, ELEMENTWISE, MOVES, MAX_OPERANDS, PATTERNS };
