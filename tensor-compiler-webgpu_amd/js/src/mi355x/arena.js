'use strict';
// Liveness-based placement of a launch list's node buffers in one device
// allocation (the arena). The reference gives every node its own buffer for
// the whole run (src/gpu/runtime.js:68, src/fusion/trainer-fused.js:37 in
// abho7/tensor-compiler-webgpu); at config-5 scale that is most of a step's
// memory held for values that live for one or two launches.
//
// A launch list runs in order on one stream, so a buffer is live from the
// launch that writes it to the last launch that reads it (a launch's operands
// and its output are live together at that launch: no kernel here runs in
// place). The members of a batched launch run as one dispatch, so they count
// as one position: every operand and output of the batch is live together. Buffers whose values must outlive the launches — inputs and
// constants the host writes before running, and the nodes the caller reads or
// feeds back (`keep`) — are pinned for the whole program. Two buffers may
// share bytes only when their live ranges are disjoint. Placement is first fit
// in decreasing size over the buffers already placed whose ranges intersect,
// at `align`-byte offsets (256: the allocation granule hipMalloc gives).
//
// Only the perf path uses it: check-mode runs keep one canary-padded buffer per
// node, because every node is read back and judged.

/**
 * Plan the arena of `lowered` (a perf lowering of `graph`): { size, offsets: node -> byte
 * offset for every buffer owner (neither an alias nor folded), buffers: [{ id, bytes, lo, hi,
 * pinned, offset }] with live range [lo, hi] in launch indices (-1 .. MAX for pinned ones),
 * unshared: the bytes one buffer per node would take }. `keep`: node ids whose values the
 * caller reads or feeds back after the launches.
 */
function planArena(graph, lowered, options) {
  const o = options || {};
  const align = o.align || 256;
  const alias = new Map(lowered.aliases || []);
  const folded = new Set((lowered.folded || []).concat(lowered.dead || []));   // no buffer
  const owner = (id) => (alias.has(id) ? alias.get(id) : id);
  const bytes = (id) => Math.max(16, Math.ceil(graph.nodes[id].shape.reduce((p, d) => p * d, 1) * 4 / align) * align);
  const INF = Number.MAX_SAFE_INTEGER;
  const start = new Map(), end = new Map(), firstRead = new Map();
  const pinned = new Set();
  const pin = (id) => {
    const w = owner(id);
    if (folded.has(w)) throw new Error(`node ${id} is kept but has no buffer (folded)`);
    pinned.add(w);
  };
  for (const node of graph.nodes) {
    if (alias.has(node.id) || folded.has(node.id)) continue;
    if (node.op === 'input' || node.op === 'const') pinned.add(node.id);
  }
  for (const id of o.keep || []) pin(id);
  // The members of a batched launch run together: they share their first member's position.
  const step = lowered.launches.map((_, i) => i);
  for (const b of lowered.batches || []) for (let k = 1; k < b.count; k++) step[b.start + k] = b.start;
  lowered.launches.forEach((l, li) => {
    const i = step[li];
    for (const id of l.inputs) {
      const w = owner(id);
      if (folded.has(w)) throw new Error(`launch ${li} (node ${l.node}) reads folded node ${id}`);
      end.set(w, Math.max(end.has(w) ? end.get(w) : -1, i));
      if (!firstRead.has(w)) firstRead.set(w, i);
    }
    const w = owner(l.node);
    if (w !== l.node) throw new Error(`launch ${li} writes node ${l.node}, an alias of ${w}`);
    if (start.has(w)) throw new Error(`node ${w} is written by two launches`);
    start.set(w, i);
    end.set(w, Math.max(end.has(w) ? end.get(w) : i, i));
  });
  const buffers = [];
  for (const node of graph.nodes) {
    const id = node.id;
    if (alias.has(id) || folded.has(id)) continue;
    if (!pinned.has(id) && !start.has(id)) pinned.add(id);   // never written by a launch: the host owns it
    const lo = pinned.has(id) ? -1 : start.get(id);
    const hi = pinned.has(id) ? INF : end.get(id);
    if (!pinned.has(id) && firstRead.has(id) && firstRead.get(id) <= lo) throw new Error(`node ${id} is read before it is written`);
    buffers.push({ id, bytes: bytes(id), lo, hi, pinned: pinned.has(id) });
  }
  // Pinned buffers first, in node order; then the rest by decreasing size (ties: earlier first).
  const order = buffers.filter((b) => b.pinned).concat(
    buffers.filter((b) => !b.pinned).sort((x, y) => y.bytes - x.bytes || x.lo - y.lo || x.id - y.id));
  const placed = [];
  let size = 0;
  for (const b of order) {
    const clash = placed.filter((p) => p.lo <= b.hi && b.lo <= p.hi).sort((x, y) => x.offset - y.offset);
    let at = 0;
    for (const p of clash) {
      if (at + b.bytes <= p.offset) break;
      at = Math.max(at, p.offset + p.bytes);
    }
    b.offset = at;
    placed.push(b);
    size = Math.max(size, at + b.bytes);
  }
  const offsets = new Map(placed.map((b) => [b.id, b.offset]));
  const unshared = buffers.reduce((s, b) => s + b.bytes, 0);
  return { size: Math.max(size, align), offsets, buffers: placed, pinned, owner, unshared };
}

/** Every pair of buffers whose live ranges intersect must not share bytes; returns the first violation or null. */
function checkArena(plan) {
  const bs = plan.buffers.slice().sort((x, y) => x.offset - y.offset);
  for (let i = 0; i < bs.length; i++) {
    for (let j = i + 1; j < bs.length && bs[j].offset < bs[i].offset + bs[i].bytes; j++) {
      const a = bs[i], b = bs[j];
      if (a.lo <= b.hi && b.lo <= a.hi) return { a: a.id, b: b.id };
    }
  }
  return null;
}

module.exports = { planArena, checkArena };
