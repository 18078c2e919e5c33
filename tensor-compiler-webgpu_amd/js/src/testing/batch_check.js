'use strict';
// An independent check of the perf lowering's batched launches (lower.js
// batchPlan): the batched launch list must hold the same launches as the plain
// order, every launch must read only buffers already written (or written by no
// launch), the members of a batch must be launches of the same kernel texts
// (or of matmul, elementwise or rowwise texts that differ, each member then run by its own case
// of the batched kernel, which holds exactly its own body) over the same grids (a column
// sum's text leaves its outer extent to the grid) with no data path between them, or
// one-kernel launches over grids that differ, each run by its own branch of a ragged
// batched kernel over its own range of the dispatch's workgroups, or
// the three parts of one attention gradient in one launch of their joint kernel; each
// batched kernel's grid must repeat the
// member kernel's grid once per member along z, and the members' workspace
// slices must be disjoint and inside the workspace. Checked from the launch
// records alone, not from the planner's own bookkeeping.

// Whether batched kernel `bk` runs, for member k, the body of kernel `x`: the switch case
// of k holds, before its break, exactly x's own entry-point body (its statements, with the
// member's z index read as the batched kernel reads it), over a set of structs that the
// batched text declares exactly as x declares its own (under the batched kernel's name).
function runsOwnBody(bk, k, x) {
  const at = bk.source.indexOf(`case ${k}u:`);
  if (at < 0) return false;
  const end = bk.source.indexOf('break;', at);
  if (end < at) return false;
  const kase = bk.source.slice(bk.source.indexOf('{', at) + 1, end);
  const m = kase.match(new RegExp(`(${bk.name}_v\\d+)_(?:av|bv|epi)`));
  if (/^tcmi_(ew|row)_/.test(x.name)) {
    // An elementwise or rowwise member declares no structs: its case is its own
    // statements alone.
    if (m || /\bstruct\b/.test(x.source)) return false;
  } else {
    if (!m) return false;
    const structs = (src, prefix) => (src.match(new RegExp(`struct ${prefix}_(?:av|bv|epi) \\{[\\s\\S]*?\\n\\};\\n`, 'g')) || [])
      .map((t) => t.split(prefix).join('@')).join('');
    const mine = structs(x.source, x.name);
    if (!(mine.length > 0 && structs(bk.source, m[1]) === mine)) return false;
  }
  // The member's own statements: its entry point's body, names and z index normalised.
  const sig = `${x.name}(const TcmiArgs A) {`;
  const own = x.source.slice(x.source.indexOf(sig) + sig.length).replace(/\}\s*$/, '');
  const norm = (t, prefix) => (prefix ? t.split(`${prefix}_`).join('@_') : t)
    .replace(/\((blockIdx\.z|wg\.z) % \d+u\)/g, '$1')
    .replace('const tcmi::Wg wg = tcmi::xcd_grouped();', '')
    .replace(/\s+/g, '');
  return norm(kase, m ? m[1] : null) === norm(own, x.name);
}

// Whether ragged batched kernel `bk` runs, for member k (workgroups [at, at + |grid|) of
// the dispatch), kernel `x` as its own launch would: the branch of k opens with exactly
// the range test, the member's argument block, and its own grid and place standing for
// gridDim and blockIdx (the decomposition of the workgroup's offset l in its range as
// (l % gx, (l / gx) % gy, l / (gx·gy))), then holds x's own statements, over structs
// declared as x declares its own.
function runsOwnRaggedBody(bk, k, x, at) {
  const [gx, gy, gz] = x.grid, count = gx * gy * gz;
  const marker = `if (tcmi_wg_ < ${at + count}u) {   // member ${k}: workgroups [${at}, ${at + count}), its grid ${gx} x ${gy} x ${gz}\n`;
  const start = bk.source.indexOf(marker);
  if (start < 0) return false;
  const rest = bk.source.slice(start + marker.length);
  const next = rest.search(/\n {2}\} else if \(tcmi_wg_ < |\n {2}\}\n\}\n$/);
  if (next < 0) return false;
  const branch = rest.slice(0, next);
  const head = [
    `const uint32_t tcmi_l_ = tcmi_wg_ - ${at}u;`,
    `const TcmiPtrs& A = B.m[${k}];`,
    `const uint3 gridDim = make_uint3(${gx}u, ${gy}u, ${gz}u);`,
    `const uint3 blockIdx = make_uint3(tcmi_l_ % ${gx}u, (tcmi_l_ / ${gx}u) % ${gy}u, tcmi_l_ / ${gx * gy}u);`,
  ];
  const lines = branch.split('\n');
  if (lines.length < head.length || head.some((h, i) => lines[i].trim() !== h)) return false;
  const body = lines.slice(head.length).join('\n');
  const m = body.match(new RegExp(`(${bk.name}_v\\d+)_`));
  const structs = (src, prefix) => (src.match(new RegExp(`struct ${prefix}_\\w+ \\{[\\s\\S]*?\\n\\};\\n`, 'g')) || [])
    .map((t) => t.split(prefix).join('@')).join('');
  if (m ? structs(bk.source, m[1]) !== structs(x.source, x.name) : structs(x.source, x.name) !== '') return false;
  const sig = `${x.name}(const TcmiArgs A) {`;
  const own = x.source.slice(x.source.indexOf(sig) + sig.length).replace(/\}\s*$/, '');
  const norm = (t, prefix) => (prefix ? t.split(`${prefix}_`).join('@_') : t).replace(/\s+/g, '');
  return norm(body, m ? m[1] : null) === norm(own, x.name);
}

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
    if (first.kernels.length === 1 && first.kernels[0].joint) {
      // An attention gradient's three parts in one launch of their joint kernel: members
      // dQ, dK, dV in that order, of one joint kernel, reading the same operands.
      const j = first.kernels[0].joint;
      const ms = L.slice(b.start, b.start + b.count);
      const ok = b.count === j.parts.length && b.kernels.length === 1 && b.kernels[0].name === j.name
        && b.kernels[0].source === j.source && b.kernels[0].grid.join() === j.grid.join()
        && ms.every((l, k) => l.kernels.length === 1 && l.kernels[0].joint && l.kernels[0].joint.name === j.name
          && l.kernels[0].part === j.parts[k] && l.inputs.join() === first.inputs.join() && !l.workspace);
      if (!ok) return { ok: false, why: `batch at ${b.start}: not the three parts of one attention gradient` };
      for (let k = 0; k < b.count; k++) unitOf[b.start + k] = b.start;
      continue;
    }
    if (b.ragged) {
      // Members of any one-kernel launches, each over its own grid, in consecutive ranges of
      // one dispatch's workgroups.
      const ms = L.slice(b.start, b.start + b.count);
      if (b.kernels.length !== 1 || b.wsStride || ms.some((l) => l.kernels.length !== 1 || l.workspace)) {
        return { ok: false, why: `batch at ${b.start}: a ragged batch of launches that are not one kernel each, or use the workspace` };
      }
      let at = 0;
      for (let k = 0; k < b.count; k++) {
        const x = ms[k].kernels[0];
        if (x.block.join() !== b.kernels[0].block.join() || x.lds || !runsOwnRaggedBody(b.kernels[0], k, x, at)) {
          return { ok: false, why: `batch at ${b.start}: member ${k} is not its own kernel over its own workgroups` };
        }
        at += x.grid[0] * x.grid[1] * x.grid[2];
        unitOf[b.start + k] = b.start;
      }
      if (b.kernels[0].grid.join() !== [at, 1, 1].join()) return { ok: false, why: `batch at ${b.start}: grid ${b.kernels[0].grid} for ${at} workgroups` };
      continue;
    }
    if (b.kernels.length !== first.kernels.length) return { ok: false, why: `batch at ${b.start}: ${b.kernels.length} batched kernels for ${first.kernels.length}` };
    for (let j = 0; j < b.kernels.length; j++) {
      const g = b.kernels[j].grid, m = first.kernels[j].grid;
      if (g[0] !== m[0] || g[1] !== m[1] || g[2] !== m[2] * b.count) return { ok: false, why: `batch at ${b.start}: grid ${g} for ${b.count} x ${m}` };
    }
    if (first.workspace && (b.wsStride < first.workspace || b.count * b.wsStride > batched.workspace)) {
      return { ok: false, why: `batch at ${b.start}: workspace slices of ${b.wsStride} bytes for ${first.workspace}` };
    }
    for (let k = 0; k < b.count; k++) {
      const l = L[b.start + k];
      const same = l.kernels.length === first.kernels.length && l.kernels.every((x, j) => {
        const y = first.kernels[j];
        if (x.grid.join() !== y.grid.join() || x.block.join() !== y.block.join() || x.lds !== y.lds) return false;
        if (x.name === y.name) return true;
        // Another matmul text (operand views, load modes, tiling or epilogue differ), or
        // another elementwise or rowwise body, over the same grid and workgroup: the
        // batched kernel must run this member's own body.
        const both = (re) => re.test(x.name) && re.test(y.name);
        return (both(/^tcmi_mm_/) || both(/^tcmi_ew_/) || both(/^tcmi_row_/)) && runsOwnBody(b.kernels[j], k, x);
      });
      if (!same || l.workspace !== first.workspace) return { ok: false, why: `batch at ${b.start}: member ${k} is not a launch of the same kernels` };
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
  return { ok: true, batches: (batched.batches || []).length, saved: (batched.batches || []).reduce((s, b) => s + b.count - 1, 0) };
}

/**
 * Planted mistakes for the check to refuse: `dependent` makes a batch of a launch
 * and a later launch of the same kernel that reads its output (placed right after
 * it); `early` moves a launch in front of the launch that writes its first operand;
 * `grid` gives a batch's last member its kernel over twice the z extent (the same
 * text over another grid, as a column sum of another outer extent has); `body`
 * exchanges, in the launch list, the first member of a batch whose members run
 * different bodies with a member of another kernel (each member's case of the batched
 * kernel then holds the other's body).
 * Returns the modified lowering, or null when the list has no such pair.
 */
function plantBatchMistake(lowered, kind) {
  if (kind === 'body') {
    const b = (lowered.batches || []).find((x) => x.kernels.length === 1 && (x.kernels[0].variants || x.kernels[0].ragged));
    if (!b) return null;
    const v = b.kernels[0].variants || b.kernels[0].ragged;
    const k = v.findIndex((name) => name !== v[0]);
    const launches = lowered.launches.slice();
    [launches[b.start], launches[b.start + k]] = [launches[b.start + k], launches[b.start]];
    return Object.assign({}, lowered, { launches });
  }
  if (kind === 'grid') {
    const b = (lowered.batches || [])[0];
    if (!b) return null;
    const launches = lowered.launches.slice();
    const last = launches[b.start + b.count - 1];
    launches[b.start + b.count - 1] = Object.assign({}, last, {
      kernels: last.kernels.map((k, j) => (j ? k : Object.assign({}, k, { grid: [k.grid[0], k.grid[1], 2 * k.grid[2]] }))) });
    return Object.assign({}, lowered, { launches });
  }
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
      if (kind === 'dependent' && L[i].kernels.map((k) => k.name).join(' ') !== L[j].kernels.map((k) => k.name).join(' ')) continue;
      // Move launch j to position i + 1 (dependent) or i (early); batches past the move shift.
      const to = kind === 'dependent' ? i + 1 : i;
      if ((lowered.batches || []).some((b) => b.start < to && to < b.start + b.count)) continue;
      const order = L.slice();
      const [moved] = order.splice(j, 1);
      order.splice(to, 0, moved);
      const batches = (lowered.batches || []).map((b) => Object.assign({}, b, { start: b.start >= to && b.start < j ? b.start + 1 : b.start }));
      if (kind === 'dependent') {
        const kernels = L[i].kernels.map((k) => ({ name: `planted_${k.name}`, source: '', grid: [k.grid[0], k.grid[1], 2 * k.grid[2]], block: k.block, lds: k.lds }));
        batches.push({ start: i, count: 2, kernels, wsStride: L[i].workspace ? Math.ceil(L[i].workspace / 256) * 256 : 0 });
        batches.sort((a, b) => a.start - b.start);
      }
      return Object.assign({}, lowered, { launches: order, batches });
    }
  }
  return null;
}

module.exports = { checkBatches, plantBatchMistake };
