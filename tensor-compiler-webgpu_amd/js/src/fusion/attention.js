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

module.exports = { fuseAttention, attentionFits, attentionLds, ATTENTION_LIMITS };
