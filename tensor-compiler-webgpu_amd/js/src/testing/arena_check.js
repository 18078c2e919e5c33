'use strict';
// An independent check of an arena plan: run the launch list abstractly over the
// arena's bytes, each write tagging its buffer's range with the node it now holds
// (and untagging whatever it overlapped), and require every launch's operands,
// and at the end every pinned buffer, to still hold their own node intact. A plan
// that lets a buffer be overwritten while a later launch (or the caller) still
// needs it fails here, whatever the live-range arithmetic claimed. The members
// of a batched launch read and write as one step.

function simulateArena(graph, lowered, plan) {
  const owner = plan.owner;
  const where = new Map(plan.buffers.map((b) => [b.id, b]));
  let extents = [];   // [{ lo, hi, tag }] disjoint byte ranges holding a node's value
  const write = (id) => {
    const b = where.get(id);
    const lo = b.offset, hi = b.offset + b.bytes;
    const next = [];
    for (const e of extents) {
      if (e.hi <= lo || e.lo >= hi) { next.push(e); continue; }
      if (e.lo < lo) next.push({ lo: e.lo, hi: lo, tag: null });   // a clipped value is no value
      if (e.hi > hi) next.push({ lo: hi, hi: e.hi, tag: null });
    }
    next.push({ lo, hi, tag: id });
    extents = next;
  };
  const holds = (id) => {
    const b = where.get(id);
    return extents.some((e) => e.tag === id && e.lo === b.offset && e.hi === b.offset + b.bytes);
  };
  for (const b of plan.buffers) if (b.pinned) write(b.id);   // the host's uploads
  // The members of a batched launch run concurrently: all of them read, then all write.
  const unit = new Map((lowered.batches || []).map((b) => [b.start, b.count]));
  for (let i = 0; i < lowered.launches.length;) {
    const members = lowered.launches.slice(i, i + (unit.get(i) || 1));
    for (const l of members) {
      for (const id of l.inputs) {
        if (!holds(owner(id))) return { ok: false, launch: i, node: l.node, operand: id };
      }
    }
    for (const l of members) write(owner(l.node));
    // No kernel here runs in place: no output of the unit may land on an operand it reads.
    for (const l of members) {
      for (const id of l.inputs) {
        if (!members.some((m) => owner(m.node) === owner(id)) && !holds(owner(id))) return { ok: false, launch: i, node: l.node, overwrote: id };
      }
    }
    i += members.length;
  }
  for (const b of plan.buffers) if (b.pinned && !holds(b.id)) return { ok: false, launch: 'end', operand: b.id };
  return { ok: true };
}

/** Largest sum of live buffer bytes at any launch: no placement can use less. */
function peakLive(lowered, plan) {
  let peak = 0;
  for (let i = 0; i < lowered.launches.length; i++) {
    let live = 0;
    for (const b of plan.buffers) if (b.lo <= i && i <= b.hi) live += b.bytes;
    peak = Math.max(peak, live);
  }
  return peak;
}

module.exports = { simulateArena, peakLive };
