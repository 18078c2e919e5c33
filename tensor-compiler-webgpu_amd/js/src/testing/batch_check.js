'use strict';
// An independent check of the perf lowering's batched launches (lower.js
// batchPlan): the batched launch list must hold the same launches as the plain
// order, every launch must read only buffers already written (or written by no
// launch), the members of a batch must be launches of one single-kernel text
// with no data path between them, and a batched kernel's grid must carry one
// z-slice per member. Checked from the launch records alone, not from the
// planner's own bookkeeping.

function checkBatches(plain, batched) {
  const alias = new Map(batched.aliases || []);
  const owner = (id) => (alias.has(id) ? alias.get(id) : id);
  const L = batched.launches;
  const nodes = (ls) => ls.map((l) => l.node).sort((a, b) => a - b).join(',');
  if (L.length !== plain.launches.length || nodes(L) !== nodes(plain.launches)) return { ok: false, why: 'launches differ from the plain order' };
  const writerOf = new Map();
  L.forEach((l, i) => writerOf.set(owner(l.node), i));
  const unitOf = L.map((_, i) => i);
  let next = 0;
  for (const b of batched.batches || []) {
    if (b.start < next || b.count < 2 || b.start + b.count > L.length) return { ok: false, why: `batch at ${b.start} overlaps or is out of range` };
    next = b.start + b.count;
    const first = L[b.start];
    if (first.kernels.length !== 1) return { ok: false, why: `batch at ${b.start}: a multi-kernel launch` };
    if (b.kernel.grid[2] !== b.count || b.kernel.grid[0] !== first.kernels[0].grid[0] || b.kernel.grid[1] !== first.kernels[0].grid[1]) {
      return { ok: false, why: `batch at ${b.start}: grid ${b.kernel.grid} for ${b.count} members` };
    }
    for (let k = 0; k < b.count; k++) {
      const l = L[b.start + k];
      if (l.kernels.length !== 1 || l.kernels[0].name !== first.kernels[0].name || l.workspace) {
        return { ok: false, why: `batch at ${b.start}: member ${k} is not a launch of the same kernel` };
      }
      unitOf[b.start + k] = b.start;
    }
  }
  for (let i = 0; i < L.length; i++) {
    for (const id of L[i].inputs) {
      const w = writerOf.get(owner(id));
      if (w === undefined) continue;
      if (unitOf[w] === unitOf[i]) return { ok: false, why: `launch ${i} reads node ${id}, written in its own batch` };
      if (w > i) return { ok: false, why: `launch ${i} reads node ${id} before launch ${w} writes it` };
    }
  }
  // Launches that use the workspace keep their order (they share its bytes).
  const ws = (ls) => ls.filter((l) => l.workspace).map((l) => l.node).join(',');
  if (ws(L) !== ws(plain.launches)) return { ok: false, why: 'workspace users reordered' };
  return { ok: true, batches: (batched.batches || []).length, saved: (batched.batches || []).reduce((s, b) => s + b.count - 1, 0) };
}

/**
 * Planted mistakes for the check to refuse: `dependent` makes a batch of a launch
 * and a later launch of the same kernel that reads its output (placed right after
 * it); `early` moves a launch in front of the launch that writes its first operand.
 * Returns the modified lowering, or null when the list has no such pair.
 */
function plantBatchMistake(lowered, kind) {
  const alias = new Map(lowered.aliases || []);
  const owner = (id) => (alias.has(id) ? alias.get(id) : id);
  const L = lowered.launches;
  const pos = new Map(L.map((l, i) => [owner(l.node), i]));
  const inBatch = new Set();
  for (const b of lowered.batches || []) for (let k = 0; k < b.count; k++) inBatch.add(b.start + k);
  for (let j = 0; j < L.length; j++) {
    if (inBatch.has(j)) continue;
    for (const id of L[j].inputs) {
      const i = pos.get(owner(id));
      if (i === undefined || i >= j || inBatch.has(i)) continue;
      if (kind === 'dependent' && !(L[i].kernels.length === 1 && L[j].kernels.length === 1 && L[i].kernels[0].name === L[j].kernels[0].name)) continue;
      // Move launch j to position i + 1 (dependent) or i (early); batches past the move shift.
      const to = kind === 'dependent' ? i + 1 : i;
      if ((lowered.batches || []).some((b) => b.start < to && to < b.start + b.count)) continue;
      const order = L.slice();
      const [moved] = order.splice(j, 1);
      order.splice(to, 0, moved);
      const batches = (lowered.batches || []).map((b) => Object.assign({}, b, { start: b.start >= to && b.start < j ? b.start + 1 : b.start }));
      if (kind === 'dependent') {
        const k = L[i].kernels[0];
        batches.push({ start: i, count: 2, kernel: { name: `planted_${k.name}`, source: '', grid: [k.grid[0], k.grid[1], 2], block: k.block, lds: k.lds } });
        batches.sort((a, b) => a.start - b.start);
      }
      return Object.assign({}, lowered, { launches: order, batches });
    }
  }
  return null;
}

module.exports = { checkBatches, plantBatchMistake };
