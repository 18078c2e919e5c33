'use strict';
// Attention fusion: an extension of the fusion contract, off by default. The
// reference lists fused attention as the stretch its milestone never attempted
// (DESIGN.md:1055-1056 in abho7/tensor-compiler-webgpu); the contract's three
// kinds (fuse.js:136-161) are unchanged, and so is every count pinned to it.
//
// After fuse(), a scaled-dot-product attention is three launches:
//   M1 = matmul(Q, Kt)            plain matmul, scores [..., Tq, Tk]
//   S  = fused rowwise 'softmax'  its body: whatever elementwise ops the group
//                                 grew over the scores (scale, additive mask)
//                                 and the softmax composite (graph.js softmax)
//   M2 = matmul(S, V)             plain matmul, [..., Tq, Dv]
// When M1 is read only by S, S only by M2, neither is kept, and the sizes fit
// the kernel (keys and head sizes below; both operand tiles in LDS), the three
// become one fused node of kind 'attention'. Its body is an ordinary graph —
// a0 = Q, a1 = Kt, M1, S's body with its score operand replaced by M1 and its
// other operands as a2.., then V last and M2 — so the float64 interpreter
// evaluates it like any fused node, and its value is M2's.

const { Graph } = require('../ir/graph');
const { bodyOf } = require('./fuse');

const size = (shape) => shape.reduce((p, d) => p * d, 1);
const roundUp = (x, m) => Math.ceil(x / m) * m;

/** What one fused attention kernel holds: keys, head sizes, LDS for the K and V tiles, operands. */
const ATTENTION_LIMITS = { keys: 512, head: 128, ldsBytes: 80 * 1024, operands: 8 };

/** LDS bytes of the key and value tiles for tk keys and head sizes dh, dv (rows padded to 16, row stride + 4). */
function attentionLds(tk, dh, dv) {
  const rows = roundUp(tk, 16);
  return rows * (roundUp(dh, 16) + 4) * 4 + rows * (roundUp(dv, 16) + 4) * 4;
}

/** Why the three nodes cannot be one attention kernel, or null. */
function attentionFits(q, kt, v, others) {
  const r = q.length;
  const tq = q[r - 2], dh = q[r - 1], tk = kt[r - 1], dv = v[r - 1];
  if (tk > ATTENTION_LIMITS.keys) return `${tk} keys`;
  if (dh > ATTENTION_LIMITS.head || dv > ATTENTION_LIMITS.head) return `head sizes ${dh}, ${dv}`;
  if (attentionLds(tk, dh, dv) > ATTENTION_LIMITS.ldsBytes) return 'key and value tiles exceed LDS';
  if (others + 3 > ATTENTION_LIMITS.operands) return `${others + 3} operands`;
  if (size(q.slice(0, r - 2)) > 65535) return 'batch exceeds the grid';
  if (tq < 1 || tk < 1) return 'empty';
  return null;
}

/**
 * Collapse every fusable attention of a fuse() result. `keep`: original ids that
 * must survive (as given to fuse). Returns a fuse()-shaped result { graph, origin,
 * index, groups } plus `attention`: [{ sink, members }] in original ids.
 */
function fuseAttention(fused, options) {
  const o = options || {};
  const g = fused.graph;
  const keepFused = new Set((o.keep || []).map((id) => fused.index.get(id)).filter((id) => id !== undefined));
  const cons = g.nodes.map(() => []);
  for (const n of g.nodes) for (const i of n.inputs) cons[i].push(n.id);
  const matches = new Map();   // M2 id -> { m1, s, xPos }
  const absorbed = new Set();
  for (const m2 of g.nodes) {
    if (m2.op !== 'matmul') continue;
    const s = g.nodes[m2.inputs[0]];
    if (s.op !== 'fused' || s.attrs.kind !== 'rowwise' || s.attrs.pattern !== 'softmax') continue;
    if (keepFused.has(s.id) || cons[s.id].length !== 1 || m2.inputs[1] === s.id || absorbed.has(s.id)) continue;
    const sb = bodyOf(s);
    const full = sb.nodes.filter((n) => n.op === 'input' && size(n.shape) === size(s.shape));
    if (full.length !== 1) continue;
    const xPos = Number(full[0].attrs.name.slice(1));
    const m1 = g.nodes[s.inputs[xPos]];
    if (m1.op !== 'matmul' || keepFused.has(m1.id) || cons[m1.id].length !== 1 || absorbed.has(m1.id)) continue;
    const [q, kt] = m1.inputs.map((i) => g.nodes[i].shape);
    const v = g.nodes[m2.inputs[1]].shape;
    if (q.length !== s.shape.length || v.length !== q.length) continue;
    if (attentionFits(q, kt, v, s.inputs.length - 1)) continue;
    matches.set(m2.id, { m1: m1.id, s: s.id, xPos });
    absorbed.add(m1.id);
    absorbed.add(s.id);
  }
  if (!matches.size) return Object.assign({}, fused, { attention: [] });

  const out = new Graph();
  const index = new Map();   // fused-graph id -> new id
  const origin = [];
  const attention = [];
  const groupOf = new Map(fused.groups.map((gr) => [fused.index.get(gr.sink), gr]));
  for (const n of g.nodes) {
    if (absorbed.has(n.id)) continue;
    const m = matches.get(n.id);
    let id;
    if (!m && n.op === 'fused') {
      id = out.nodes.length;
      out.nodes.push({ id, op: 'fused', inputs: n.inputs.map((i) => index.get(i)), attrs: n.attrs, shape: n.shape.slice() });
    } else if (!m) {
      id = out.emit(n.op, n.inputs.map((i) => index.get(i)), n.attrs);
    } else {
      const m1 = g.nodes[m.m1], s = g.nodes[m.s];
      const b = new Graph();
      const operands = [m1.inputs[0], m1.inputs[1]];
      const qIn = b.input('a0', g.nodes[m1.inputs[0]].shape);
      const kIn = b.input('a1', g.nodes[m1.inputs[1]].shape);
      const scores = b.emit('matmul', [qIn, kIn], {});
      const sb = bodyOf(s);
      const map = new Map();
      for (const bn of sb.nodes) {
        if (bn.op === 'input') {
          const k = Number(bn.attrs.name.slice(1));
          if (k === m.xPos) map.set(bn.id, scores);
          else {
            map.set(bn.id, b.input(`a${operands.length}`, bn.shape));
            operands.push(s.inputs[k]);
          }
        } else {
          map.set(bn.id, b.emit(bn.op, bn.inputs.map((i) => map.get(i)), bn.attrs));
        }
      }
      const vIn = b.input(`a${operands.length}`, g.nodes[n.inputs[1]].shape);
      operands.push(n.inputs[1]);
      const output = b.emit('matmul', [map.get(s.attrs.output), vIn], {});
      id = out.nodes.length;
      out.nodes.push({ id, op: 'fused', inputs: operands.map((i) => index.get(i)),
        attrs: { kind: 'attention', pattern: 'attention', body: b.toJSON(), output }, shape: n.shape.slice() });
      const sGroup = groupOf.get(s.id);
      const members = new Set(sGroup ? sGroup.members : []);
      members.add(fused.origin[m1.id]);
      members.add(fused.origin[n.id]);
      attention.push({ sink: fused.origin[n.id], members });
    }
    index.set(n.id, id);
    origin[id] = fused.origin[n.id];
  }
  const originalIndex = new Map();
  for (const [orig, fid] of fused.index) if (index.has(fid)) originalIndex.set(orig, index.get(fid));
  const sinks = new Set(Array.from(matches.values()).map((m) => fused.origin[m.s]));
  const groups = fused.groups.filter((gr) => !sinks.has(gr.sink))
    .concat(attention.map((a) => ({ sink: a.sink, members: a.members, kind: 'attention', root: a.sink, pattern: 'attention' })));
  return { graph: out, origin, index: originalIndex, groups, attention };
}

// ---- attention in a training step ---------------------------------------------------
//
// In a fused training step the softmax splits (R5): the backward pass reads the
// exponentials and their row sum, so one attention is, after fuse(),
//   M1 = matmul(Q, Kt)   R1 = fused rowwise (scale, mask, max shift, exp)
//   Sm = sum(R1)   P = div(R1, broadcast(Sm))   O = matmul(P, V)
// and its gradient
//   dP = matmul(dO, transpose(V))   dV = matmul(transpose(P), dO)
//   Z  = fused rowwise (the softmax backward on dP, R1, Sm)   dS = Z's elementwise chain (the scale)
//   dQ = matmul(dS, K)   dK = matmul(transpose(dS), Q)
// eleven launches, five of them [.., T, T] score tensors written and read back.
// With the gradient recomputing P from Q and K (as the forward extension forms P in
// registers), no score tensor outlives its kernel: the forward becomes one
// 'attention' node (O), and the gradient three 'attention-grad' nodes (dQ, dK, dV)
// sharing one body — Q, K, V, dO and the score operands in, the recomputed P, dP, the
// softmax backward and all three products — each with its own output. The body is an
// ordinary graph of the same ops as the nodes it replaces, so the float64 interpreter
// evaluates each of the three as any fused node, and its value is that of the node it
// replaces. The perf lowering runs the three as one kernel (lower.js).

const GRAD_LIMITS = { queries: 128, keys: 512, head: 128, ldsBytes: 150 * 1024, operands: 8 };

/** LDS bytes the gradient kernel stages: K and V, then the score tile with Q (or dO). */
function attentionGradLds(tq, tk, dh, dv) {
  const rows = roundUp(tk, 16), qrows = roundUp(tq, 16);
  const kv = rows * (roundUp(dh, 16) + 4) + rows * (roundUp(dv, 16) + 4);
  const tile = qrows * (rows + 4) + qrows * (Math.max(roundUp(dh, 16), roundUp(dv, 16)) + 4);
  return 4 * Math.max(kv, tile);
}

/** Why an attention's gradient cannot be one attention-grad kernel, or null. */
function attentionGradFits(q, k, v, others) {
  const r = q.length;
  const tq = q[r - 2], dh = q[r - 1], tk = k[r - 2], dv = v[r - 1];
  if (tq > GRAD_LIMITS.queries) return `${tq} queries`;
  if (tk > GRAD_LIMITS.keys) return `${tk} keys`;
  if (dh > GRAD_LIMITS.head || dv > GRAD_LIMITS.head) return `head sizes ${dh}, ${dv}`;
  if (attentionGradLds(tq, tk, dh, dv) > GRAD_LIMITS.ldsBytes) return 'tiles exceed LDS';
  if (others + 4 > GRAD_LIMITS.operands) return `${others + 4} operands`;
  if (size(q.slice(0, r - 2)) > 65535) return 'batch exceeds the grid';
  return null;
}

const swapsLast = (n) => n.op === 'transpose' && n.attrs.perm.every((p, d) => {
  const r = n.attrs.perm.length;
  return d < r - 2 ? p === d : p === (d === r - 2 ? r - 1 : r - 2);
});
const isElementwiseNode = (n) => (n.op === 'fused' && n.attrs.kind === 'elementwise')
  || ['add', 'sub', 'mul', 'div', 'neg', 'exp', 'log', 'relu', 'tanh', 'sqrt', 'step'].includes(n.op);

/**
 * Collapse every attention of a fused training step whose gradient the fused graph holds
 * (above). `keep`: original ids that must survive (as given to fuse). Returns a
 * fuse()-shaped result { graph, origin, index, groups } plus `attention` (the forward
 * nodes) and `attentionGrad`: [{ dq, dk, dv }] (new ids), so the lowering knows which
 * three share a body.
 */
function fuseAttentionTraining(fused, options) {
  const o = options || {};
  const g = fused.graph;
  const keepFused = new Set((o.keep || []).map((id) => fused.index.get(id)).filter((id) => id !== undefined));
  const cons = g.nodes.map(() => []);
  for (const n of g.nodes) for (const i of n.inputs) cons[i].push(n.id);
  const live = new Set();
  for (let id = g.nodes.length - 1; id >= 0; id--) {
    if (keepFused.has(id) || cons[id].some((c) => live.has(c))) live.add(id);
  }
  const liveReaders = (id) => Array.from(new Set(cons[id].filter((c) => live.has(c))));
  const last = (n) => n.shape.length - 1;
  const plans = [];
  const taken = new Set();
  for (const m2 of g.nodes) {
    const plan = matchTraining(g, m2, liveReaders, last, keepFused);
    if (!plan || plan.internal.some((id) => taken.has(id))) continue;
    for (const id of plan.internal) taken.add(id);
    plans.push(plan);
  }
  if (!plans.length) return Object.assign({}, fused, { attention: [], attentionGrad: [] });

  // Nodes that go: each plan's internal nodes, then every dead node reading a node gone.
  const gone = new Set(taken);
  for (let changed = true; changed;) {
    changed = false;
    for (const n of g.nodes) {
      if (gone.has(n.id) || !n.inputs.some((i) => gone.has(i))) continue;
      if (live.has(n.id) && !plans.some((p) => p.replaced.has(n.id))) throw new Error(`attention: node ${n.id} reads a node the fusion removes`);
      if (!live.has(n.id)) { gone.add(n.id); changed = true; }
    }
  }
  const replacement = new Map();   // old id -> { plan, role }
  for (const p of plans) for (const [role, id] of Object.entries(p.outputs)) replacement.set(id, { plan: p, role });
  const out = new Graph();
  const index = new Map();
  const origin = [];
  const attention = [], attentionGrad = [];
  const groupOf = new Map(fused.groups.map((gr) => [fused.index.get(gr.sink), gr]));
  const membersOf = (ids) => {
    const m = new Set();
    for (const id of ids) {
      const gr = groupOf.get(id);
      if (gr) for (const x of gr.members) m.add(x);
      else if (fused.origin[id] >= 0) m.add(fused.origin[id]);
    }
    return m;
  };
  const newGroups = [];
  for (const n of g.nodes) {
    const rep = replacement.get(n.id);
    if (gone.has(n.id) && !rep) continue;
    let id;
    if (!rep && n.op === 'fused') {
      id = out.nodes.length;
      out.nodes.push({ id, op: 'fused', inputs: n.inputs.map((i) => index.get(i)), attrs: n.attrs, shape: n.shape.slice() });
    } else if (!rep) {
      id = out.emit(n.op, n.inputs.map((i) => index.get(i)), n.attrs);
    } else {
      const p = rep.plan;
      const body = rep.role === 'o' ? p.forwardBody : p.gradBody;
      const kind = rep.role === 'o' ? 'attention' : 'attention-grad';
      id = out.nodes.length;
      const attrs = { kind, pattern: kind, body: body.graph, output: body.outputs[rep.role] };
      if (kind === 'attention-grad') attrs.part = rep.role;
      out.nodes.push({ id, op: 'fused', inputs: body.operands.map((i) => index.get(i)), attrs, shape: n.shape.slice() });
      const sink = fused.origin[n.id];
      // The gradient is one group (its three parts run as one launch): dQ's node is its sink.
      if (rep.role !== 'dk' && rep.role !== 'dv') {
        const members = membersOf(rep.role === 'o' ? p.groupNodes.o : p.groupNodes.dq.concat(p.groupNodes.dk, p.groupNodes.dv));
        newGroups.push({ sink, members, kind, root: sink, pattern: kind });
      }
      if (rep.role === 'o') attention.push({ sink, members: membersOf(p.groupNodes.o) });
      else {
        let rec = attentionGrad.find((r) => r.plan === p);
        if (!rec) { rec = { plan: p }; attentionGrad.push(rec); }
        rec[rep.role] = id;
      }
    }
    index.set(n.id, id);
    origin[id] = fused.origin[n.id];
  }
  const originalIndex = new Map();
  for (const [orig, fid] of fused.index) if (index.has(fid) && !gone.has(fid)) originalIndex.set(orig, index.get(fid));
  for (const [orig, fid] of fused.index) if (replacement.has(fid)) originalIndex.set(orig, index.get(fid));
  const removedSinks = new Set();
  for (const gr of fused.groups) if (gone.has(fused.index.get(gr.sink))) removedSinks.add(gr.sink);
  const groups = fused.groups.filter((gr) => !removedSinks.has(gr.sink)).concat(newGroups);
  return { graph: out, origin, index: originalIndex, groups, attention,
    attentionGrad: attentionGrad.map((r) => ({ dq: r.dq, dk: r.dk, dv: r.dv })) };
}

/**
 * The training-step attention whose forward ends in product `m2` (see above), or null:
 * { internal: node ids that go, replaced: the four nodes taking new bodies, outputs
 * { o, dq, dk, dv }, forwardBody, gradBody, groupNodes }.
 */
function matchTraining(g, m2, liveReaders, last, keepFused) {
  const N = g.nodes;
  if (m2.op !== 'matmul' || keepFused.has(m2.id)) return null;
  const pd = N[m2.inputs[0]];
  if (pd.op !== 'div' || keepFused.has(pd.id)) return null;
  const r1 = N[pd.inputs[0]], bc = N[pd.inputs[1]];
  if (r1.op !== 'fused' || r1.attrs.kind !== 'rowwise' || bc.op !== 'broadcast') return null;
  const sm = N[bc.inputs[0]];
  if (sm.op !== 'sum' || sm.inputs[0] !== r1.id || sm.attrs.axis !== last(N[r1.id]) || !sm.attrs.keepDims) return null;
  const rb = bodyOf(r1);
  const full = rb.nodes.filter((n) => n.op === 'input' && size(n.shape) === size(r1.shape));
  if (full.length !== 1) return null;
  const xPos = Number(full[0].attrs.name.slice(1));
  const m1 = N[r1.inputs[xPos]];
  if (m1.op !== 'matmul') return null;
  const qn = N[m1.inputs[0]], ktn = N[m1.inputs[1]];
  if (!swapsLast(ktn)) return null;
  const kn = N[ktn.inputs[0]], vn = N[m2.inputs[1]];
  const [q, k, v] = [qn.shape, kn.shape, vn.shape];
  if (q.length < 3 || k.length !== q.length || v.length !== q.length || size(q.slice(0, -2)) !== size(k.slice(0, -2))) return null;
  // The gradient: dV = matmul(transpose(P), dO) and dP = matmul(dO, transpose(V)).
  const ptn = liveReaders(pd.id).map((c) => N[c]).filter((c) => swapsLast(c));
  if (ptn.length !== 1) return null;
  const dvs = liveReaders(ptn[0].id).map((c) => N[c]).filter((c) => c.op === 'matmul' && c.inputs[0] === ptn[0].id);
  if (dvs.length !== 1) return null;
  const dv = dvs[0], don = N[dv.inputs[1]];
  const dps = liveReaders(don.id).map((c) => N[c])
    .filter((c) => c.op === 'matmul' && c.inputs[0] === don.id && swapsLast(N[c.inputs[1]]) && N[c.inputs[1]].inputs[0] === vn.id);
  if (dps.length !== 1) return null;
  const dp = dps[0], vtn = N[dp.inputs[1]];
  // Z: the softmax backward, the one live reader of dP, reading dP, R1, Sm or its broadcast.
  const zr = liveReaders(dp.id);
  if (zr.length !== 1) return null;
  const z = N[zr[0]];
  if (!(z.op === 'fused' && (z.attrs.kind === 'rowwise' || z.attrs.kind === 'elementwise')) && !isElementwiseNode(z)) return null;
  const zIn = new Set([dp.id, r1.id, sm.id, bc.id]);
  if (!z.inputs.every((i) => zIn.has(i) || N[i].op === 'const')) return null;
  // dS: Z, or Z's one live elementwise reader (the scale), read by the two products.
  let ds = z;
  const zReaders = liveReaders(z.id);
  if (zReaders.length === 1 && isElementwiseNode(N[zReaders[0]]) && N[zReaders[0]].inputs.every((i) => i === z.id || N[i].op === 'const')) {
    ds = N[zReaders[0]];
  }
  const dsReaders = liveReaders(ds.id).map((c) => N[c]);
  const dqs = dsReaders.filter((c) => c.op === 'matmul' && c.inputs[0] === ds.id);
  const dsts = dsReaders.filter((c) => swapsLast(c));
  if (dqs.length !== 1 || dsts.length !== 1 || dsReaders.length !== 2) return null;
  const dq = dqs[0];
  const kOf = N[dq.inputs[1]];
  const kViaKt = swapsLast(kOf) && kOf.inputs[0] === ktn.id;
  if (!(kViaKt || kOf.id === kn.id)) return null;
  const dks = liveReaders(dsts[0].id).map((c) => N[c]).filter((c) => c.op === 'matmul' && c.inputs[0] === dsts[0].id && c.inputs[1] === qn.id);
  if (dks.length !== 1 || liveReaders(dsts[0].id).length !== 1) return null;
  const dk = dks[0];
  // Every live reader of a node that goes is another node that goes or one of the four replaced.
  const internal = [m1.id, r1.id, sm.id, bc.id, pd.id, ptn[0].id, dp.id, z.id, ds.id, dsts[0].id];
  const uniq = Array.from(new Set(internal));
  const replaced = new Set([m2.id, dq.id, dk.id, dv.id]);
  const inSet = new Set(uniq);
  for (const id of uniq) {
    if (keepFused.has(id)) return null;
    for (const c of liveReaders(id)) if (!inSet.has(c) && !replaced.has(c)) return null;
  }
  // Views the gone nodes read stay only if something else reads them.
  for (const t of [ktn, vtn, kViaKt ? kOf : null]) {
    if (t && liveReaders(t.id).every((c) => inSet.has(c) || replaced.has(c))) uniq.push(t.id);
  }
  // R1's and Z's and dS's further operands (the mask and any other score operand).
  const others = [];
  for (const n of [r1, z, ds]) for (const i of n.inputs) {
    if ([m1.id, dp.id, r1.id, sm.id, bc.id, z.id].includes(i) || others.includes(i)) continue;
    others.push(i);
  }
  if (attentionGradFits(q, k, v, others.length)) return null;
  if (attentionFits(q, ktn.shape, v, r1.inputs.length - 1)) return null;
  const forwardBody = buildForwardBody(g, { m1, r1, xPos, pd, sm, m2, qn, ktn, vn });
  const gradBody = buildGradBody(g, { m1, r1, xPos, sm, bc, dp, z, ds, qn, kn, vn, don, others });
  return {
    internal: uniq, replaced, outputs: { o: m2.id, dq: dq.id, dk: dk.id, dv: dv.id },
    forwardBody, gradBody,
    groupNodes: { o: [m1.id, r1.id, sm.id, pd.id, m2.id], dq: [dp.id, z.id, ds.id, dq.id], dk: [dk.id], dv: [dv.id] },   // fused-graph ids
  };
}

/** Copy `body` (a fused node's Graph) into `b`, its inputs a{k} mapped by `inputFor(k, node)`. Returns the output's new id. */
function inline(b, body, output, inputFor) {
  const map = new Map();
  for (const n of body.nodes) {
    if (n.op === 'input') map.set(n.id, inputFor(Number(n.attrs.name.slice(1)), n));
    else map.set(n.id, b.emit(n.op, n.inputs.map((i) => map.get(i)), n.attrs));
  }
  return map.get(output);
}

/** The body of node `n` (a fused node's, or the one op on inputs a0..). */
function nodeBody(g, n) {
  if (n.op === 'fused') return { body: bodyOf(n), output: n.attrs.output };
  const b = new Graph();
  const ins = n.inputs.map((i, k) => b.input(`a${k}`, g.nodes[i].shape));
  return { body: b, output: b.emit(n.op, ins, n.attrs) };
}

/** The forward attention node's body: Q, Kt, R1's other operands, V (as fuseAttention builds it). */
function buildForwardBody(g, m) {
  const b = new Graph();
  const operands = [m.qn.id, m.ktn.id];
  const qIn = b.input('a0', m.qn.shape);
  const kIn = b.input('a1', m.ktn.shape);
  const scores = b.emit('matmul', [qIn, kIn], {});
  const e = inline(b, bodyOf(m.r1), m.r1.attrs.output, (k, n) => {
    if (k === m.xPos) return scores;
    operands.push(m.r1.inputs[k]);
    return b.input(`a${operands.length - 1}`, n.shape);
  });
  const s = b.emit('sum', [e], m.sm.attrs);
  const p = b.emit('div', [e, b.broadcast(s, g.nodes[m.r1.id].shape)], {});
  const vIn = b.input(`a${operands.length}`, m.vn.shape);
  operands.push(m.vn.id);
  const o = b.emit('matmul', [p, vIn], {});
  return { graph: b.toJSON(), outputs: { o }, operands };
}

/**
 * The gradient nodes' shared body: a0 Q, a1 K, a2 V, a3 dO, then the further operands;
 * the scores and P recomputed (R1's body, the row sum, the division), dP, Z's and dS's
 * bodies, and the three products dQ = dS·K, dK = dSᵀ·Q, dV = Pᵀ·dO.
 */
function buildGradBody(g, m) {
  const b = new Graph();
  const N = g.nodes;
  const operands = [m.qn.id, m.kn.id, m.vn.id, m.don.id].concat(m.others);
  const ins = operands.map((id, k) => b.input(`a${k}`, N[id].shape));
  const other = (id) => ins[operands.indexOf(id)];
  const kt = b.transpose(ins[1], swapPerm(m.kn.shape.length));
  const scores = b.emit('matmul', [ins[0], kt], {});
  const e = inline(b, bodyOf(m.r1), m.r1.attrs.output, (k) => (k === m.xPos ? scores : other(m.r1.inputs[k])));
  const s = b.emit('sum', [e], m.sm.attrs);
  const bs = b.broadcast(s, N[m.r1.id].shape);
  const p = b.emit('div', [e, bs], {});
  const vt = b.transpose(ins[2], swapPerm(m.vn.shape.length));
  const dp = b.emit('matmul', [ins[3], vt], {});
  const valueOf = (id) => (id === m.dp.id ? dp : id === m.r1.id ? e : id === m.sm.id ? s : id === m.bc.id ? bs : other(id));
  const zb = nodeBody(g, m.z);
  const z = inline(b, zb.body, zb.output, (k) => valueOf(m.z.inputs[k]));
  let ds = z;
  if (m.ds.id !== m.z.id) {
    const db = nodeBody(g, m.ds);
    ds = inline(b, db.body, db.output, (k) => (m.ds.inputs[k] === m.z.id ? z : other(m.ds.inputs[k])));
  }
  const dq = b.emit('matmul', [ds, ins[1]], {});
  const dk = b.emit('matmul', [b.transpose(ds, swapPerm(m.qn.shape.length)), ins[0]], {});
  const dv = b.emit('matmul', [b.transpose(p, swapPerm(m.qn.shape.length)), ins[3]], {});
  return { graph: b.toJSON(), outputs: { dq, dk, dv, ds, p }, operands };
}

const swapPerm = (r) => Array.from({ length: r }, (_, d) => (d < r - 2 ? d : d === r - 2 ? r - 1 : r - 2));

module.exports = { fuseAttention, fuseAttentionTraining, attentionFits, attentionGradFits, attentionLds, attentionGradLds,
  ATTENTION_LIMITS, GRAD_LIMITS };
