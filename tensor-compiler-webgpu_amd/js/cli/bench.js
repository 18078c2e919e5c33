#!/usr/bin/env node
'use strict';
// Measurement of the MI355X backend on the benchmark's five configs, printed as one JSON
// document (bench.py turns it into the driver's one-line record).
//
//   node bench.js [--configs ceiling,c2,c3,c4] [--steps K] [--warmup W] [--programs P]
//                 [--reps N] [--c4-shapes all|small] [--quick] [--graphs] [--no-trainer-graphs] [--step-only]
//                 [--no-attention]
//                 [--roofline-only] [--gate FILE]
//
// --no-attention: c5's perf path without each attention and its gradient fused
// (fusion/attention.js fuseAttentionTraining), which it uses by default.
//
// --graphs: the c2 step's programs replayed as captured HIP graphs. The trainers
// of c1 and c5 replay each step as a captured HIP graph by default (a step is
// launch-bound at c1's size); --no-trainer-graphs issues their launches directly.
//
// --step-only (for profilers): c2 runs its step only, every program after the
// previous on one stream (the headline issues them over --c2-streams); c3 and c4 run each
// fused program --steps times after --warmup runs, with no timing loops; c1 and c5
// run --warmup + --steps trainer steps.
//
// c2  fused elementwise chains (P programs, forward + gradient) over [8192, 1024]:
//     the headline step = every fused program run once; K timed steps
//     bracketed by a sync and hipEvents on both sides.
// c3  softmax / logSoftmax forward + backward over [16384, 4096]
// c4  matmul + bias -> relu | tanh at three shapes, and its backward graph
// sweep  the reference's workload sweep: fused vs unfused (and recompute) per workload
// For every program: fused and unfused timed against each other (ABBA), every
// launch timed alone (for per-fusion-group speedups and the dominant kernel's
// average duration), algorithmic bytes and matmul flops.

const { size } = require('../src/ir/shapes');
const { fuse } = require('../src/fusion/fuse');
const { lowerMI355X } = require('../src/mi355x/lower');
const { HipRunner, Concurrent } = require('../src/mi355x/runner');
const { HipBench, summarize, verdict, median } = require('../src/mi355x/bench');
const { chainWorkload, chainInputs } = require('../src/builders/chains');
const cfg = require('../src/builders/configs');

const HBM_PEAK_GBS = 8000;
const FP32_MFMA_PEAK_TFLOPS = 157.3;

function arg(name, dflt) {
  const i = process.argv.indexOf(`--${name}`);
  return i >= 0 && process.argv[i + 1] !== undefined ? process.argv[i + 1] : dflt;
}
const flag = (name) => process.argv.includes(`--${name}`);
const log = (m) => process.stderr.write(`bench: ${m}\n`);

/** Prepare a program for `graph` with `inputs` uploaded. */
function prepared(runner, graph, lowered, inputs, opts) {
  const p = runner.prepare(graph, lowered, opts);
  for (const node of graph.nodes) if (node.op === 'input') p.write(node.id, inputs[node.attrs.name]);
  return p;
}

/**
 * Time every dispatch of `program` alone, as the program issues it: µs per launch
 * (median, min and max of a few repetitions). A batched dispatch is timed whole and
 * its time shared among its member launches (`batched`: the member count) in
 * proportion to their work (flops where every member has them, algorithmic bytes where
 * none has: evenly among identical members; members whose bodies differ may differ in
 * size), so a member costs what it costs inside its batch, not what it would cost by
 * itself. A ragged batch's members are timed each alone.
 */
function timeLaunches(runner, bench, program, reps) {
  const out = [];
  const L = program.lowered;
  const batchAt = new Map((L.batches || []).map((b) => [b.start, b]));
  for (let i = 0; i < L.launches.length;) {
    // A ragged batch's members (small kernels of different kinds and grids) are timed
    // each alone: no share of their dispatch would stand for one of them.
    const b = batchAt.get(i) && !batchAt.get(i).ragged ? batchAt.get(i) : null;
    const members = L.launches.slice(i, i + (b ? b.count : 1));
    const lowered = { launches: members, workspace: L.workspace };
    if (b) lowered.batches = [Object.assign({}, b, { start: 0 })];
    const one = runner.prepare(program.graph, lowered, { buffers: program.bufs });
    const r = bench.time({ one }, { reps: reps || 5, warmup: 1, targetMs: 0.5, direct: true });
    const n = members.length;
    const byFlops = members.every((l) => l.flops > 0);
    const work = members.map((l) => (byFlops ? l.flops : l.bytes || 0));
    const total = work.reduce((s, w) => s + w, 0);
    members.forEach((l, k) => {
      const share = total > 0 ? work[k] / total : 1 / n;
      out.push({ node: l.node, kind: l.kind, pattern: l.pattern || null, code: l.code, bytes: l.bytes, flops: l.flops,
        us: r.stats.one.median * share, minUs: r.stats.one.min * share, maxUs: r.stats.one.max * share, rowFolds: l.rowFolds || null, absorbed: l.absorbed || null,
        formed: l.formed || null, batched: n > 1 ? n : undefined, joint: b && b.joint ? true : undefined });
    });
    one.destroy();
    i += n;
  }
  return out;
}

/**
 * Fused against unfused for every fusion group of `f` (fuse.js:228 groups), including
 * groups where fusion is neutral or slower: the group's fused launch timed alone against
 * the summed times of its members' unfused launches, each timed alone. A group wins or
 * loses only when the ranges do not overlap (the fused launch's min-max against the
 * members' summed mins and maxes). A launch that also forms the reductions folded into
 * it (the perf lowering's row folds), the producers of their operands formed in the
 * same launch, the producers an elementwise launch absorbed and the values a launch
 * forms from what their own launches would read, does their work as well: the unfused
 * launches of those nodes (of their groups' members, where one is a group's sink) count
 * on its side too (`folded`: their node ids in the unfused graph). A node that several
 * launches compute counts a 1/k share in each of their k groups.
 */
function groupVerdicts(f, launchF, launchU) {
  const fusedAt = new Map(launchF.map((l) => [l.node, l]));
  const unfusedAt = new Map(launchU.map((l) => [l.node, l]));
  const groupAt = new Map();
  for (const g of f.groups) if (f.index.has(g.sink)) groupAt.set(f.index.get(g.sink), g);
  const original = new Map();
  for (const [id, fid] of f.index) if (!original.has(fid)) original.set(fid, id);
  // The fused nodes a launch computes besides its own: reductions and producers folded
  // into it, producers it absorbed, values it forms (with what their own launches fold
  // and absorb). Each is keyed by its group's sink (or its original node).
  const takenBy = (fl, own) => {
    const fids = [];
    const absorbed = (records) => { for (const a of records || []) { fids.push(a.producer); absorbed(a.absorbed); } };
    const folds = (rfs) => { for (const rf of rfs || []) fids.push(...(rf.producer === undefined ? [rf.reduction] : [rf.reduction, rf.producer])); };
    absorbed(fl.absorbed);
    folds(fl.rowFolds);
    for (const v of fl.formed || []) { fids.push(v.value); folds(v.rowFolds); absorbed(v.absorbed); }
    const keys = new Map();
    for (const fid of fids) {
      const g2 = groupAt.get(fid);
      if (g2 === own) continue;
      const id = g2 ? g2.sink : original.get(fid);
      if (id !== undefined) keys.set(id, g2 ? g2.members : [id]);
    }
    return keys;
  };
  // A node several launches compute (a value formed by each of its readers) counts
  // a share of its unfused time in each of their groups, so no unfused launch counts twice.
  const ownerOf = (fl) => groupAt.get(fl.node) || null;
  const takers = new Map();
  for (const fl of launchF) for (const id of takenBy(fl, ownerOf(fl)).keys()) takers.set(id, (takers.get(id) || 0) + 1);
  const groups = [];
  for (const g of f.groups) {
    if (!f.index.has(g.sink)) continue;
    const fl = fusedAt.get(f.index.get(g.sink));
    if (!fl) continue;
    const weight = new Map(Array.from(g.members, (m) => [m, 1]));
    const taken = takenBy(fl, g);
    for (const [id, members] of taken) for (const m of members) if (!weight.has(m)) weight.set(m, 1 / takers.get(id));
    const sum = { median: 0, min: 0, max: 0 };
    let launches = 0;
    for (const [m, w] of weight) {
      const u = unfusedAt.get(m);
      if (!u) continue;
      sum.median += w * u.us; sum.min += w * u.minUs; sum.max += w * u.maxUs; launches++;
    }
    if (!launches) continue;
    // A group whose launch is one part of a joint launch (an attention gradient's dQ, dK
    // and dV in one kernel) takes the whole launch's time: the group holds all three.
    const whole = fl.joint ? fl.batched : 1;
    const v = verdict(sum, { median: fl.us * whole, min: fl.minUs * whole, max: fl.maxUs * whole });
    groups.push({ sink: g.sink, kind: g.kind, pattern: g.pattern, members: weight.size, unfusedLaunches: launches,
      fusedUs: fl.us * whole, unfusedUs: sum.median, speedup: v.speedup, verdict: v.verdict,
      folded: taken.size ? Array.from(taken.keys()) : undefined });
  }
  return groups;
}

/** Win / loss / noise counts of a list of group verdicts, with the worst (lowest speedup) group. */
function groupSummary(groups) {
  const out = { groups: groups.length, win: 0, loss: 0, noise: 0, worst: null };
  for (const g of groups) {
    out[g.verdict]++;
    if (!out.worst || g.speedup < out.worst.speedup) out.worst = g;
  }
  return out;
}

/**
 * One graph, fused and unfused: ABBA timing of the two programs, every launch
 * alone, per-group speedups. `inputs` by name.
 */
function measureGraph(runner, bench, name, graph, keep, inputs, opts) {
  const o = opts || {};
  // Both variants in the perf lowering (reshapes share buffers, transposes read in
  // place by their matmuls): what the trainer runs; outputs equal the plain lowering's.
  const f = fuse(graph, { keep });
  const lf = lowerMI355X(f.graph, { perf: true, keep: keep.map((id) => f.index.get(id)) });
  const lu = lowerMI355X(graph, { perf: true, keep, rowFolds: false });
  runner.functions([lf, lu]);
  // With o.arena, each program's node buffers share one allocation by live range.
  const pf = prepared(runner, f.graph, lf, inputs, o.arena ? { arena: { keep: keep.map((id) => f.index.get(id)) } } : undefined);
  const pu = prepared(runner, graph, lu, inputs, o.arena ? { arena: { keep } } : undefined);
  const t = bench.time({ fused: pf, unfused: pu }, { reps: o.reps });
  const launchF = timeLaunches(runner, bench, pf, o.launchReps);
  const launchU = o.skipUnfusedLaunches ? null : timeLaunches(runner, bench, pu, o.launchReps);
  // Outputs of both variants: bitwise agreement is reported, parity is the tests' job.
  pf.run(); pu.run(); pf.sync();
  let same = 0, total = 0;
  for (const id of keep) {
    const a = pf.read(f.index.get(id)), b = pu.read(id);
    total += a.length;
    for (let i = 0; i < a.length; i++) if (Object.is(a[i], b[i])) same++;
  }
  const bytesF = lf.launches.reduce((s, l) => s + l.bytes, 0);
  const bytesU = lu.launches.reduce((s, l) => s + l.bytes, 0);
  // The fusion contract's count of the same program: one launch per fused node (the
  // reference's own accounting of a fused program, workloads.js:155-175).
  const bytesC = lowerMI355X(f.graph).launches.reduce((s, l) => s + l.bytes, 0);
  const flops = lf.launches.reduce((s, l) => s + (l.flops || 0), 0);
  const groups = launchU ? groupVerdicts(f, launchF, launchU) : [];
  const res = {
    name, launches: { fused: lf.launches.length, unfused: lu.launches.length }, k: t.k,
    fused: t.stats.fused, unfused: t.stats.unfused, verdict: verdict(t.stats.unfused, t.stats.fused),
    bytes: { fused: bytesF, unfused: bytesU, contract: bytesC }, flops,
    gbs: { fused: bytesF / (t.stats.fused.median * 1e3), unfused: bytesU / (t.stats.unfused.median * 1e3) },
    tflops: flops ? { fused: flops / (t.stats.fused.median * 1e6), unfused: flops / (t.stats.unfused.median * 1e6) } : null,
    bitwiseSameOutputs: { same, total }, groups, launchF, launchU,
  };
  if (o.keepPrograms) res.programs = { pf, pu };
  else { pf.destroy(); pu.destroy(); }
  return res;
}

/**
 * The dominant kernel of a set of launch timings, aggregated by kernel name:
 * the one moving the most algorithmic bytes (or, for matmuls, flops) in all —
 * a choice that does not depend on timing noise, so a profile of the same
 * command names the same kernel.
 */
function dominant(launches) {
  const by = new Map();
  for (const l of launches) {
    const e = by.get(l.code) || { code: l.code, kind: l.kind, pattern: l.pattern, count: 0, us: 0, bytes: 0, flops: 0 };
    e.count++; e.us += l.us; e.bytes += l.bytes; e.flops += l.flops || 0;
    by.set(l.code, e);
  }
  let best = null;
  const weight = (e) => (e.flops || e.bytes);
  for (const e of by.values()) if (!best || weight(e) > weight(best)) best = e;
  if (!best) return null;
  const avgUs = best.us / best.count, bytes = best.bytes / best.count;
  return Object.assign(best, { avgUs, bytesPerLaunch: bytes, gbs: bytes / (avgUs * 1e3),
    tflops: best.flops ? best.flops / best.count / (avgUs * 1e6) : null });
}

/** The fused kernel moving the most algorithmic bytes per step, from the lowerings alone (no timing). */
function dominantByBytes(programs) {
  const launches = [];
  for (const p of programs) for (const l of p.launches) if (l.kind.startsWith('fused-')) launches.push(Object.assign({ us: 0 }, l));
  const d = dominant(launches);
  return d ? { code: d.code, kind: d.kind, pattern: d.pattern, count: d.count, bytes: d.bytes, bytesPerLaunch: d.bytes / d.count } : null;
}

/** Copies a cold launch rotates over: at least 8, and enough to span COLD_SPAN bytes. */
const COLD_SETS = 8;
/** Four times the 256 MB last-level cache: a set is long evicted when its turn comes again. */
const COLD_SPAN = 4 * 256 * 2 ** 20;

/**
 * Launch `l` of program `p` timed cold: copies of every buffer it reads and writes (at
 * least COLD_SETS of them, and enough to span COLD_SPAN bytes), the launch issued on set
 * i mod the set count, k launches back to back between two events, k chosen for >= 4 ms
 * (or `runs` launches untimed, for a profiler). Returns the average µs per launch, the
 * set count and the bytes the sets span.
 */
function coldLaunch(runner, bench, p, l, runs) {
  const a = runner.a;
  const ids = Array.from(new Set(l.inputs.concat([l.node])));
  const perSet = ids.reduce((acc, id) => acc + p.n[id] * 4, 0);
  const COLD = Math.max(COLD_SETS, Math.ceil(COLD_SPAN / perSet));
  const sets = [];
  let span = 0;
  for (let s = 0; s < COLD; s++) {
    const bufs = p.bufs.slice();
    const owned = [];
    for (const id of ids) {
      const bytes = p.n[id] * 4;
      const h = a.malloc(bytes);
      a.d2d(h, 0, p.bufs[id], 0, bytes);
      bufs[id] = h;
      owned.push(h);
      span += bytes;
    }
    const prog = runner.prepare(p.graph, { launches: [l], workspace: p.lowered.workspace }, { buffers: bufs });
    sets.push({ prog, owned });
  }
  a.sync();
  const issue = (k) => { for (let i = 0; i < k; i++) sets[i % COLD].prog.run(); };
  let out;
  if (runs) {
    issue(runs);
    a.sync();
    out = { runs, sets: COLD, spanBytes: span };
  } else {
    issue(2 * COLD);
    a.sync();
    a.eventRecord(bench.start);
    issue(COLD);
    a.eventRecord(bench.end);
    const one = a.eventElapsed(bench.start, bench.end) / COLD;
    const k = Math.max(COLD, Math.ceil(4 / one / COLD) * COLD);
    const reps = [];
    bench.region(() => {
      for (let r = 0; r < 9; r++) {
        a.eventRecord(bench.start);
        issue(k);
        a.eventRecord(bench.end);
        reps.push(a.eventElapsed(bench.start, bench.end) / k);
      }
    });
    const st = summarize(reps);
    out = { avgUs: st.median, minUs: st.min, maxUs: st.max, k, reps: reps.length, sets: COLD, spanBytes: span };
  }
  for (const s of sets) { s.prog.destroy(); for (const h of s.owned) a.free(h); }
  return out;
}

// ---- configs -----------------------------------------------------------------------

function c2(runner, bench, opts) {
  const R = 8192, C = 1024;
  const P = Number(arg('programs', opts.quick ? 2 : 8));
  const K = Number(arg('steps', 20)), W = Number(arg('warmup', 3));
  const programs = [];
  const results = [];
  // --roofline-only (for the profile behind `roofline`): the programs are built and only
  // the roofline kernel's cold measurement runs.
  const rooflineOnly = flag('roofline-only');
  const stepOnly = flag('step-only') || rooflineOnly;
  const arena = flag('arena');
  for (let s = 0; s < P; s++) {
    const w = chainWorkload(s, R, C);
    const inputs = chainInputs(s, R, C);
    for (const kind of ['forward', 'gradient']) {
      const v = w[kind];
      log(`c2 program ${s} ${kind}`);
      if (stepOnly) {
        // Profiling mode: only the programs of the step, no per-variant timing.
        const f = fuse(v.graph, { keep: v.keep });
        const lf = lowerMI355X(f.graph, { perf: true, keep: v.keep.map((id) => f.index.get(id)) });
        runner.functions(lf);
        programs.push(prepared(runner, f.graph, lf, inputs, arena ? { arena: { keep: v.keep.map((id) => f.index.get(id)) } } : undefined));
        results.push({ name: `c2-p${s}-${kind}`, bytes: { fused: lf.launches.reduce((q, l) => q + l.bytes, 0),
          contract: lowerMI355X(f.graph).launches.reduce((q, l) => q + l.bytes, 0) }, launchF: [],
          launches: launchRecords(lf) });
        continue;
      }
      const r = measureGraph(runner, bench, `c2-p${s}-${kind}`, v.graph, v.keep, inputs, { keepPrograms: true, reps: opts.reps, arena });
      r.ops = w.ops;
      programs.push(r.programs.pf);
      r.programs.pu.destroy();
      delete r.programs;
      results.push(r);
    }
  }
  if (rooflineOnly) {
    // The cold measurement exactly as the bench makes it, and nothing else of the step:
    // a tracer's average over this command's launches of the kernel is the same figure.
    const dom = dominantByBytes(programs);
    const p = programs.find((q) => q.launches.some((x) => x.code === dom.code));
    dom.cold = coldLaunch(runner, bench, p, p.launches.find((x) => x.code === dom.code), 0);
    dom.avgUs = dom.cold.avgUs;
    dom.gbs = dom.bytesPerLaunch / (dom.avgUs * 1e3);
    for (const q of programs) q.destroy();
    return { config: 'c2', rooflineOnly: true, shape: [R, C], programs: P, dominant: dom, results };
  }
  // The headline step: every fused program once; W warm-up steps, then K timed steps
  // bracketed by hipEvents. The 16 programs are independent (each its own buffers), so
  // the step issues them as one concurrent group over --c2-streams streams (default 3:
  // 2, 3 and 4 measured, 3 and 4 fastest), balanced by bytes; the sequential step, every program
  // after the previous on one stream (with --graphs: each a replayed HIP graph), is
  // timed beside it.
  const timeSteps = (issue) => {
    for (let i = 0; i < W; i++) issue();
    runner.a.sync();
    const t0 = process.hrtime.bigint();
    runner.a.eventRecord(bench.start);
    for (let i = 0; i < K; i++) issue();
    runner.a.eventRecord(bench.end);
    const ms = runner.a.eventElapsed(bench.start, bench.end);
    runner.a.sync();
    return { msPerStep: ms / K, wallMsPerStep: Number(process.hrtime.bigint() - t0) / 1e6 / K };
  };
  const timeStepsChecked = (issue) => bench.region(() => timeSteps(issue));
  const go = bench.graphs ? (p) => p.replay() : (p) => p.run();
  for (const p of programs) if (bench.graphs) p.capture();
  const sequential = timeStepsChecked(() => { for (const p of programs) go(p); });
  // Profiling mode runs the sequential step only, so each kernel's traced duration is its own.
  const S = Number(arg('c2-streams', 3));
  const group = stepOnly ? null : new Concurrent(runner, programs, S);
  const headline = stepOnly ? sequential : timeStepsChecked(() => group.run());
  const ms = headline.msPerStep * K, wallMs = headline.wallMsPerStep * K;
  const stepBytes = results.reduce((s, r) => s + r.bytes.fused, 0);
  const contractBytes = results.reduce((s, r) => s + r.bytes.contract, 0);
  // The roofline kernel: the fused kernel moving the most algorithmic bytes per step,
  // chosen without timing so a profile of the same step names the same kernel (each
  // fused body is its own kernel, at one size, so its average is well defined). Its
  // duration: the launch alone in its own program's buffers, 21 repetitions' median.
  const all = stepOnly ? [] : [].concat.apply([], results.map((r) => r.launchF)).filter((l) => l.kind.startsWith('fused-'));
  const dom = stepOnly ? null : dominant(all);
  if (dom) {
    const p = programs.find((q) => q.launches.some((x) => x.code === dom.code));
    const l = p.launches.find((x) => x.code === dom.code);
    // Warm: the launch alone in its own program's buffers, repeated back to back (its
    // 235 MB fit the 256 MB last-level cache, so repeats find operands cached).
    {
      const one = runner.prepare(p.graph, { launches: [l], workspace: p.lowered.workspace }, { buffers: p.bufs });
      const t = bench.time({ one }, { reps: 21, warmup: 3, targetMs: 1, direct: true });
      one.destroy();
      dom.warm = { avgUs: t.stats.one.median, gbs: dom.bytesPerLaunch / (t.stats.one.median * 1e3), reps: 21 };
    }
    // Cold: the figure `roofline` reports. The launch rotates over copies of its operands
    // and output spanning at least four times the last-level cache, so between two
    // launches on one set the other sets' bytes have passed through it: every launch
    // reads its operands from HBM.
    dom.cold = coldLaunch(runner, bench, p, l, 0);
    dom.avgUs = dom.cold.avgUs;
    dom.gbs = dom.bytesPerLaunch / (dom.avgUs * 1e3);
  }
  for (const p of programs) p.destroy();
  sequential.gbs = stepBytes / (sequential.msPerStep * 1e6);
  const schedule = stepOnly ? { streams: 1 } : { streams: S, bytesPerStream: group.load, sequential };
  const groups = groupSummary([].concat.apply([], results.map((r) => r.groups || [])));
  return { config: 'c2', shape: [R, C], programs: P, steps: K, warmup: W, arena, schedule, msPerStep: ms / K, wallMsPerStep: wallMs / K,
    stepBytes, gbs: stepBytes / ((ms / K) * 1e6), contractBytes, contractGbs: contractBytes / ((ms / K) * 1e6),
    dominant: dom, groups, results };
}

/**
 * Profiling mode (--step-only): the fused program of `graph` in the perf lowering
 * run `--steps` times after `--warmup` runs, nothing else timed, so a profiler
 * sees each of its kernels a known number of times. Returns every launch's kernel
 * names with its algorithmic bytes and flops.
 */
function runOnly(runner, name, graph, keep, inputs, fuseOptions) {
  const K = Number(arg('steps', 20)), W = Number(arg('warmup', 3));
  const f = fuse(graph, Object.assign({ keep }, fuseOptions || {}));
  const lf = lowerMI355X(f.graph, { perf: true, keep: keep.map((id) => f.index.get(id)) });
  runner.functions(lf);
  const p = prepared(runner, f.graph, lf, inputs);
  for (let i = 0; i < W + K; i++) p.run();
  p.sync();
  p.destroy();
  return { name, runs: W + K, launches: launchRecords(lf) };
}

/**
 * Every launch of a lowering with its kernel names, algorithmic bytes and flops (for
 * profile summaries); each batched launch as one more record, its members' work summed.
 */
function launchRecords(lowered) {
  const recs = lowered.launches.map((l) => ({ node: l.node, kind: l.kind, pattern: l.pattern || null,
    kernels: l.kernels.map((k) => k.name), bytes: l.bytes, flops: l.flops || 0 }));
  for (const b of lowered.batches || []) {
    const ms = lowered.launches.slice(b.start, b.start + b.count);
    const kind = b.ragged ? `ragged x${b.count} (${Array.from(new Set(ms.map((l) => l.kind))).join(', ')})` : `batched ${ms[0].kind} x${b.count}`;
    recs.push({ node: ms[0].node, kind, pattern: ms[0].pattern || null, kernels: b.kernels.map((k) => k.name),
      bytes: ms.reduce((q, l) => q + l.bytes, 0), flops: ms.reduce((q, l) => q + (l.flops || 0), 0), members: ms.map((l) => l.node) });
  }
  return recs;
}

/**
 * The attention extension on the transformer's forward pass (config 5's structure
 * at batch 64, and the reference's at batch 16): the contract's fusion (matmul,
 * softmax group, matmul per attention) against fuse(..., { attention: true }) (one
 * kernel per attention), ABBA-timed in the perf lowering, with each attention
 * kernel's own duration against the three launches it replaces.
 */
function attention(runner, bench, opts) {
  const tf = require('../src/builders/transformer');
  const { Rng } = require('../src/testing/rng');
  const results = [];
  const cases = [['c5-forward', tf.C5_CONFIG, 96, opts.quick ? 8 : 64], ['reference-forward', tf.REFERENCE_CONFIG, 16, 16]];
  for (const [name, cfg, V, B] of cases) {
    log(`attention ${name}`);
    const fwd = tf.buildForward(V, B, cfg);
    const keep = [fwd.logits, fwd.loss];
    const inputs = {};
    const init = tf.initParams(V, 1, cfg);
    for (const k of Object.keys(init)) inputs[k] = Float32Array.from(init[k]);
    const rng = new Rng(V * 1000 + B);
    const rows = B * cfg.T;
    const onehot = () => { const a = new Float32Array(rows * V); for (let i = 0; i < rows; i++) a[i * V + rng.int(0, V - 1)] = 1; return a; };
    inputs.x = onehot();
    inputs.y = onehot();
    if (flag('step-only')) {
      // Profiling mode: the forward pass with attention fused, nothing else timed.
      results.push(runOnly(runner, `attention-${name}`, fwd.graph, keep, inputs, { attention: true }));
      continue;
    }
    const fc = fuse(fwd.graph, { keep });
    const fa = fuse(fwd.graph, { keep, attention: true });
    const lc = lowerMI355X(fc.graph, { perf: true, keep: keep.map((id) => fc.index.get(id)) });
    const la = lowerMI355X(fa.graph, { perf: true, keep: keep.map((id) => fa.index.get(id)) });
    runner.functions([lc, la]);
    const pc = prepared(runner, fc.graph, lc, inputs);
    const pa = prepared(runner, fa.graph, la, inputs);
    const t = bench.time({ contract: pc, attention: pa }, { reps: opts.reps });
    const tc = timeLaunches(runner, bench, pc), ta = timeLaunches(runner, bench, pa);
    pc.run(); pa.run(); pc.sync();
    const yc = pc.read(fc.index.get(fwd.logits)), ya = pa.read(fa.index.get(fwd.logits));
    let maxDiff = 0;
    for (let i = 0; i < yc.length; i++) maxDiff = Math.max(maxDiff, Math.abs(yc[i] - ya[i]));
    const usOf = (launches, node) => { const l = launches.find((x) => x.node === node); return l ? l.us : 0; };
    const groups = fa.attention.map((g) => {
      const kernel = ta.find((x) => x.node === fa.index.get(g.sink));
      let replaced = 0;
      for (const m of g.members) if (fc.index.has(m)) replaced += usOf(tc, fc.index.get(m));
      return { sink: g.sink, kernelUs: kernel.us, replacedUs: replaced, speedup: replaced / kernel.us,
        tflops: kernel.flops / (kernel.us * 1e6), code: kernel.code };
    });
    pc.destroy();
    pa.destroy();
    results.push({ name, B, launches: { contract: lc.launches.length, attention: la.launches.length },
      contract: t.stats.contract, attention: t.stats.attention, verdict: verdict(t.stats.contract, t.stats.attention),
      maxAbsDiffLogits: maxDiff, groups });
  }
  return { config: 'attention', results, stepOnly: flag('step-only') };
}

function c3(runner, bench, opts) {
  const R = opts.quick ? 2048 : cfg.C3_SHAPE[0], C = cfg.C3_SHAPE[1];
  const { x, dy, shifted } = cfg.c3Inputs(R, C);
  const results = [];
  const programs = [];
  for (const fn of ['softmax', 'logSoftmax']) {
    const g = cfg.c3Graphs(fn, R, C);
    if (flag('step-only')) {
      results.push(runOnly(runner, `c3-${fn}-forward`, g.forward.graph, g.forward.keep, { x }));
      results.push(runOnly(runner, `c3-${fn}-backward`, g.gradient.graph, g.gradient.keep, { x, d0: dy }));
      continue;
    }
    const keep = (r) => { programs.push(r.programs.pf); r.programs.pu.destroy(); delete r.programs; return r; };
    log(`c3 ${fn} forward`);
    results.push(keep(measureGraph(runner, bench, `c3-${fn}-forward`, g.forward.graph, g.forward.keep, { x },
      { reps: opts.reps, keepPrograms: true })));
    log(`c3 ${fn} backward`);
    results.push(keep(measureGraph(runner, bench, `c3-${fn}-backward`, g.gradient.graph, g.gradient.keep, { x, d0: dy },
      { reps: opts.reps, keepPrograms: true })));
  }
  if (flag('step-only')) return { config: 'c3', shape: [R, C], results };
  const all = [].concat.apply([], results.map((r) => r.launchF));
  const bytes = results.reduce((s, r) => s + r.bytes.fused, 0);
  const us = results.reduce((s, r) => s + r.fused.median, 0);
  // The programs are timed repeated on their own buffers, where a program's re-reads of
  // its 268 MB tensors partly hit the 256 MB last-level cache; the dominant kernel is
  // also timed cold, as config 2's roofline kernel is (operands rotated over sets that
  // span several times that cache), for an HBM figure beside the warm one.
  const dom = dominant(all);
  if (dom) {
    const p = programs.find((q) => q.launches.some((x) => x.code === dom.code));
    dom.cold = coldLaunch(runner, bench, p, p.launches.find((x) => x.code === dom.code), 0);
    dom.cold.gbs = dom.bytesPerLaunch / (dom.cold.avgUs * 1e3);
  }
  for (const p of programs) p.destroy();
  return { config: 'c3', shape: [R, C], shiftedRows: shifted.length, gbs: bytes / (us * 1e3), dominant: dom,
    groups: groupSummary([].concat.apply([], results.map((r) => r.groups))), results };
}

function c4(runner, bench, opts) {
  const shapes = opts.quick || arg('c4-shapes', 'all') === 'small' ? [cfg.C4_SHAPES[0]] : cfg.C4_SHAPES;
  const results = [];
  for (const [M, K, N] of shapes) {
    const { X, W, bias, dY } = cfg.c4Inputs(M, K, N);
    for (const act of ['relu', 'tanh']) {
      const g = cfg.c4Graphs(act, M, K, N);
      if (flag('step-only')) {
        results.push(runOnly(runner, `c4-${M}x${K}x${N}-${act}-forward`, g.forward.graph, g.forward.keep, { X, W, bias }));
        results.push(runOnly(runner, `c4-${M}x${K}x${N}-${act}-backward`, g.gradient.graph, g.gradient.keep, { X, W, bias, d0: dY }));
        continue;
      }
      log(`c4 ${M}x${K}x${N} ${act} forward`);
      results.push(measureGraph(runner, bench, `c4-${M}x${K}x${N}-${act}-forward`, g.forward.graph, g.forward.keep,
        { X, W, bias }, { reps: opts.reps || 16 }));
      log(`c4 ${M}x${K}x${N} ${act} backward`);
      results.push(measureGraph(runner, bench, `c4-${M}x${K}x${N}-${act}-backward`, g.gradient.graph, g.gradient.keep,
        { X, W, bias, d0: dY }, { reps: opts.reps || 8 }));
    }
  }
  if (flag('step-only')) return { config: 'c4', shapes, results };
  const mm = [].concat.apply([], results.map((r) => r.launchF)).filter((l) => l.flops);
  return { config: 'c4', shapes, dominant: dominant(mm), groups: groupSummary([].concat.apply([], results.map((r) => r.groups))), results };
}

/**
 * A training step (configs 1 and 5) through the fused trainer: K timed steps of
 * train(x, y) — batch upload, every launch, device-side parameter feedback, loss
 * readback — after W warm-up steps, timed by the wall clock (the contract of
 * FusedTrainer.train, one sync per step); the same K steps with the batch already
 * in HBM timed by hipEvents; fused against unfused step time; launches per step;
 * time by kernel kind from every launch timed alone.
 */
function trainStep(runner, bench, name, req, opts) {
  const { modelStep } = require('../src/builders/models');
  const { fusedStep, HipTrainer } = require('../src/mi355x/trainer');
  const m = modelStep(req);
  // The perf path fuses each attention and its gradient (fusion/attention.js) unless
  // --no-attention; the contract-only lowering beside it never does.
  const attention = !!req.attention && !flag('no-attention');
  const fs = fusedStep(m.step, { attention });
  // The unfused step in the perf lowering (views, batching) without anything that forms
  // one node's value inside another's launch (no folds, absorption or relus on load).
  const lu = lowerMI355X(m.step.graph, { perf: true, keep: [m.step.loss, m.step.logits].concat(Object.values(m.step.outputs)),
    rowFolds: false, loadOps: false });
  // The fused step under the fusion contract alone: the same lowering of the fused graph.
  const fsContract = fusedStep(m.step, { contract: true });
  runner.functions([fs.lowered, lu, fsContract.lowered]);
  // Timed steps after 5 warm-ups: 40 of config 5's 2.2 ms step; 400 of config 1's step of
  // about 35–70 µs (40 of them, under 3 ms, once read 9.6–10.0k steps/s through train()
  // where 400 read 15.2–15.3k in the same code).
  const K = Number(arg('train-steps', opts.quick ? 3 : name === 'c1' ? 400 : 40)), W = opts.quick ? 2 : 5;
  const batch = m.batch(0);
  const graph = !flag('no-trainer-graphs');
  const trainer = new HipTrainer(runner, fs, m.params, m.state, { graph });
  if (flag('step-only')) {
    // Profiling mode: --warmup + --steps trainer steps, nothing else run.
    const n = Number(arg('warmup', 3)) + Number(arg('steps', 20));
    for (let i = 0; i < n; i++) trainer.train(batch.x, batch.y);
    trainer.destroy();
    return { config: name, info: m.info, stepOnly: true, runs: n, graphReplay: graph, attention,
      results: [{ name: `${name}-step`, launches: launchRecords(fs.lowered) }] };
  }
  for (let i = 0; i < W; i++) trainer.train(batch.x, batch.y);
  // A step through train() uploads the batch and reads the loss back (trainer-fused.js:
  // 59-81); it creates nothing. The batch-resident steps move no data at all.
  const STEP_IO = ['h2d', 'd2h'];
  const t0 = process.hrtime.bigint();
  let loss = 0;
  bench.region(() => { for (let i = 0; i < K; i++) loss = trainer.train(batch.x, batch.y); }, STEP_IO);
  const wallMs = Number(process.hrtime.bigint() - t0) / 1e6 / K;
  // Batch resident: the steps' launches only, K steps between two events.
  runner.a.sync();
  const residentMs = bench.region(() => {
    runner.a.eventRecord(bench.start);
    for (let i = 0; i < K; i++) trainer.advance();
    runner.a.eventRecord(bench.end);
    return runner.a.eventElapsed(bench.start, bench.end) / K;
  });
  const p = trainer.program;
  // Unfused step (same graph, no fusion), batch resident.
  const pu = runner.prepare(m.step.graph, lu);
  const all = Object.assign({}, m.params, m.state, { x: batch.x, y: batch.y });
  all[m.step.cotangent] = [1];
  for (const node of m.step.graph.nodes) if (node.op === 'input') pu.write(node.id, all[node.attrs.name]);
  const tc = new HipTrainer(runner, fsContract, m.params, m.state, { graph });
  tc.train(batch.x, batch.y);
  const t = bench.time({ fused: p, unfused: pu, contract: tc.program }, { reps: opts.quick ? 3 : 8, warmup: 2 });
  const contract = { launches: fsContract.lowered.launches.length, dispatches: tc.program.dispatches,
    residentMsPerStep: t.stats.contract.median / 1e3, residentStepsPerSec: 1e6 / t.stats.contract.median,
    verdict: verdict(t.stats.unfused, t.stats.contract), fullOverContract: verdict(t.stats.contract, t.stats.fused) };
  tc.destroy();
  // Time by kind (each launch alone), and every fusion group against its members'
  // unfused launches, each timed alone.
  const launches = timeLaunches(runner, bench, p, 3);
  const launchesU = timeLaunches(runner, bench, pu, 3);
  const groupList = groupVerdicts(fs.fusion, launches, launchesU);
  const byKind = {};
  for (const l of launches) {
    const e = byKind[l.kind] || (byKind[l.kind] = { launches: 0, us: 0, bytes: 0, flops: 0 });
    e.launches++; e.us += l.us; e.bytes += l.bytes; e.flops += l.flops || 0;
  }
  for (const k of Object.keys(byKind)) {
    const e = byKind[k];
    e.gbs = e.bytes / (e.us * 1e3);
    if (e.flops) e.tflops = e.flops / (e.us * 1e6);
  }
  pu.destroy();
  trainer.destroy();
  // The same trainer with its intermediate buffers in a liveness arena.
  const ta = new HipTrainer(runner, fs, m.params, m.state, { graph, arena: true });
  for (let i = 0; i < W; i++) ta.train(batch.x, batch.y);
  const ta0 = process.hrtime.bigint();
  bench.region(() => { for (let i = 0; i < K; i++) ta.train(batch.x, batch.y); }, STEP_IO);
  const arenaWallMs = Number(process.hrtime.bigint() - ta0) / 1e6 / K;
  runner.a.sync();
  const arenaResidentMs = bench.region(() => {
    runner.a.eventRecord(bench.start);
    for (let i = 0; i < K; i++) ta.advance();
    runner.a.eventRecord(bench.end);
    return runner.a.eventElapsed(bench.start, bench.end) / K;
  });
  const plan = ta.program.arena;
  const arena = { bytes: plan.size, unshared: plan.unshared, msPerStep: arenaWallMs, residentMsPerStep: arenaResidentMs,
    stepsPerSec: 1e3 / arenaWallMs, residentStepsPerSec: 1e3 / arenaResidentMs };
  ta.destroy();
  // Independent launches on several streams (--streams N, issued directly: multi-stream
  // programs are not captured into graphs). Measured slower than one stream here: each
  // cross-stream wait costs more than the overlap it buys.
  const streamRuns = {};
  const nStreams = Number(arg('streams', 1));
  if (nStreams > 1) {
    const ts = new HipTrainer(runner, fs, m.params, m.state, { streams: nStreams });
    for (let i = 0; i < W; i++) ts.train(batch.x, batch.y);
    const ts0 = process.hrtime.bigint();
    for (let i = 0; i < K; i++) ts.train(batch.x, batch.y);
    const wall = Number(process.hrtime.bigint() - ts0) / 1e6 / K;
    runner.a.sync();
    runner.a.eventRecord(bench.start);
    for (let i = 0; i < K; i++) ts.advance();
    runner.a.eventRecord(bench.end);
    const resident = runner.a.eventElapsed(bench.start, bench.end) / K;
    streamRuns[nStreams] = { msPerStep: wall, residentMsPerStep: resident, stepsPerSec: 1e3 / wall, residentStepsPerSec: 1e3 / resident,
      criticalPath: ts.program.dag.criticalPath, waits: ts.program.dag.waits.length };
    ts.destroy();
  }
  // The same step with every launch dispatched by itself (no batched launches).
  const fsPlain = fusedStep(m.step, { batch: false, attention });
  const tp = new HipTrainer(runner, fsPlain, m.params, m.state, { graph });
  for (let i = 0; i < W; i++) tp.train(batch.x, batch.y);
  const tp0 = process.hrtime.bigint();
  bench.region(() => { for (let i = 0; i < K; i++) tp.train(batch.x, batch.y); }, STEP_IO);
  const plainWall = Number(process.hrtime.bigint() - tp0) / 1e6 / K;
  runner.a.sync();
  const plainResident = bench.region(() => {
    runner.a.eventRecord(bench.start);
    for (let i = 0; i < K; i++) tp.advance();
    runner.a.eventRecord(bench.end);
    return runner.a.eventElapsed(bench.start, bench.end) / K;
  });
  const unbatched = { dispatches: tp.program.dispatches, msPerStep: plainWall, residentMsPerStep: plainResident,
    stepsPerSec: 1e3 / plainWall, residentStepsPerSec: 1e3 / plainResident };
  tp.destroy();
  const flops = fs.lowered.launches.reduce((q, l) => q + (l.flops || 0), 0);
  return { config: name, info: m.info, steps: K, warmup: W, lossLast: loss, arena, streams: streamRuns, graphReplay: graph, attention,
    stepsPerSec: 1e3 / wallMs, msPerStep: wallMs, residentMsPerStep: residentMs, residentStepsPerSec: 1e3 / residentMs,
    launches: { fused: fs.lowered.launches.length, unfused: lu.launches.length },
    dispatches: p.dispatches, batches: (fs.lowered.batches || []).length, unbatched, contract,
    fused: t.stats.fused, unfused: t.stats.unfused, verdict: verdict(t.stats.unfused, t.stats.fused),
    matmulFlopsPerStep: flops, matmulTflopsResident: flops / (residentMs * 1e9), byKind,
    groups: groupSummary(groupList), groupList };
}

function c1(runner, bench, opts) { return trainStep(runner, bench, 'c1', { model: 'mlp' }, opts); }
function c5(runner, bench, opts) { return trainStep(runner, bench, 'c5', { model: 'transformer', B: opts.quick ? 8 : 64, attention: true }, opts); }

/**
 * The reference's workload sweep (src/fusion/workloads.js:71-120): every graph
 * workload's variants (unfused, fused, recompute, matmul-only) in the perf
 * lowering, timed against each other in ABBA order; per workload the median and
 * range of each variant, its launches and algorithmic bytes, and the fused-vs-
 * unfused (and recompute-vs-fused) speedup and win / loss / noise verdict,
 * including the workloads built so that fusion loses.
 */
function sweep(runner, bench, opts) {
  const { workloads } = require('../src/builders/workloads');
  // The correctness gate (workloads.js:351-374, web/m4-bench.html:120-150 there): every
  // variant was run once and judged against the float64 oracle before timing (bench.py
  // writes the verdicts to --gate); a workload any of whose variants failed is not timed.
  const gateFile = arg('gate', null);
  const gate = gateFile ? JSON.parse(require('fs').readFileSync(gateFile, 'utf8')) : null;
  const rows = [];
  let timed = 0;
  for (const w of workloads()) {
    const g = gate ? gate[w.id] : null;
    if (gate && !(g && g.pass)) {
      rows.push({ id: w.id, family: w.family, params: w.params, gate: g || { pass: false, reason: 'not judged' }, timed: false });
      log(`sweep ${w.id}: failed its gate, not timed`);
      continue;
    }
    timed++;
    const m = w.make();
    const variants = {}, info = {};
    for (const v of w.variants) {
      let graph, lowered, only;
      if (v === 'unfused') {
        graph = m.graph;
        lowered = lowerMI355X(m.graph, { perf: true, keep: m.outputs, rowFolds: false });
      } else {
        const f = fuse(m.graph, { keep: m.outputs, recompute: v === 'recompute' });
        graph = f.graph;
        lowered = lowerMI355X(f.graph, { perf: true, keep: m.outputs.map((id) => f.index.get(id)) });
        if (v === 'matmul-only') only = (l) => !!l.flops;
      }
      runner.functions(lowered);
      const launches = lowered.launches.filter((l) => !only || only(l));
      variants[v] = prepared(runner, graph, lowered, m.inputs, only ? { only } : undefined);
      info[v] = { launches: launches.length, bytes: launches.reduce((q, l) => q + l.bytes, 0), flops: launches.reduce((q, l) => q + (l.flops || 0), 0) };
    }
    const t = bench.time(variants, { reps: opts.reps || 16 });
    const row = { id: w.id, family: w.family, params: w.params, gate: g, timed: true, k: t.k, variants: {} };
    for (const v of w.variants) {
      const st = t.stats[v];
      row.variants[v] = Object.assign({ medianUs: st.median * 1e3, minUs: st.min * 1e3, maxUs: st.max * 1e3, gbs: info[v].bytes / (st.median * 1e6) }, info[v]);
    }
    if (t.stats.fused) row.fused = verdict(t.stats.unfused, t.stats.fused);
    if (t.stats.recompute) row.recompute = verdict(t.stats.fused, t.stats.recompute);
    rows.push(row);
    for (const v of w.variants) variants[v].destroy();
    if (timed % 20 === 0) log(`sweep: ${timed} workloads timed`);
  }
  // Per family: workloads, fused wins / losses / noise, median and range of the speedup.
  const families = {};
  for (const r of rows) {
    if (!r.fused) continue;
    const f = families[r.family] || (families[r.family] = { workloads: 0, win: 0, loss: 0, noise: 0, speedups: [] });
    f.workloads++;
    f[r.fused.verdict] = (f[r.fused.verdict] || 0) + 1;
    f.speedups.push(r.fused.speedup);
  }
  for (const f of Object.values(families)) {
    f.speedups.sort((a, b) => a - b);
    f.speedup = { median: median(f.speedups), min: f.speedups[0], max: f.speedups[f.speedups.length - 1] };
    delete f.speedups;
  }
  return { config: 'sweep', gated: !!gate, timedWorkloads: timed, workloads: rows, families };
}

/** The bandwidth ceiling (workloads.js:312-345): copy and pure read of 1 GiB, grid-strided, 1024 x 256 threads. */
function ceiling(runner, bench) {
  const a = runner.a;
  const bytes = 2 ** 30;
  const src = a.malloc(bytes), dst = a.malloc(bytes);
  a.fill32(src, 0, 0x3f800000, bytes / 4);
  const out = {};
  for (const mode of ['copy', 'read']) {
    const run = () => (mode === 'copy' ? a.ceilingCopy(dst, src, bytes, 1024) : a.ceilingRead(dst, src, bytes, 1024));
    for (let i = 0; i < 3; i++) run();
    const ms = [];
    for (let r = 0; r < 10; r++) {
      a.eventRecord(bench.start);
      for (let i = 0; i < 5; i++) run();
      a.eventRecord(bench.end);
      ms.push(a.eventElapsed(bench.start, bench.end) / 5);
    }
    const med = median(ms);
    out[mode] = { bytes: mode === 'copy' ? 2 * bytes : bytes, us: med * 1e3, gbs: (mode === 'copy' ? 2 * bytes : bytes) / (med * 1e6) };
  }
  a.free(src); a.free(dst);
  return Object.assign({ config: 'ceiling', kernel: { copy: 'k_copy16', read: 'k_read16' }, blocks: 1024 }, out);
}

async function main() {
  const runner = HipRunner.create();
  const bench = new HipBench(runner, { graphs: flag('graphs') });
  const opts = { quick: flag('quick'), reps: arg('reps') ? Number(arg('reps')) : undefined };
  const which = arg('configs', 'ceiling,c2,c3,c4,c1,c5').split(',');
  const out = { device: runner.info(), peaks: { hbmGBs: HBM_PEAK_GBS, fp32MfmaTFLOPs: FP32_MFMA_PEAK_TFLOPS }, configs: {} };
  const fns = { c2, c3, c4, c1, c5, ceiling, sweep, attention };
  for (const c of which) {
    if (!fns[c]) throw new Error(`unknown config ${c}`);
    const t0 = Date.now();
    out.configs[c] = fns[c](runner, bench, opts);
    out.configs[c].seconds = (Date.now() - t0) / 1e3;
    log(`${c} done in ${out.configs[c].seconds.toFixed(1)} s`);
  }
  out.timedRegionsChecked = bench.checked;
  bench.destroy();
  process.stdout.write(JSON.stringify(out));
}

main().catch((e) => {
  process.stderr.write(`${e.stack || e}\n`);
  process.exit(1);
});
