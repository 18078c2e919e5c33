'use strict';
// Timing on the MI355X: the reference's protocol (src/fusion/bench.js:124-216
// and src/fusion/measure-m4.js:229-234 in abho7/tensor-compiler-webgpu) on HIP:
//   * a repetition is k back-to-back runs of a prepared program, bracketed by
//     two hipEvents on the stream the kernels run on; k is chosen from a
//     single run so one repetition lasts >= 2 ms (bench.js:178-181);
//   * every buffer, argument block and function handle is made before the
//     timed region; a program run is one native call issuing all its launches
//     (or, with `graphs`, the replay of a HIP graph captured once);
//   * 5 warm-up repetitions per variant, then 32 repetitions in ABBA order;
//   * summaries are median/min/max microseconds per program run, and two
//     variants win or lose against each other only when their min-max ranges
//     do not overlap (verdict), speedup being the ratio of medians;
//   * the library's counters of object-creating calls and host<->device copies
//     (tcmi_counters) are read on both sides of the repetitions, and a timed
//     region that created anything or moved data throws (bench.js:41-47,175-192
//     there). `leak` (the counters' self-test) allocates inside every repetition,
//     which must make time() throw.

const WARMUP = 5;
const REPS = 32;
const TARGET_MS = 2;
const MAX_K = 4096;

function median(a) {
  const s = a.slice().sort((x, y) => x - y);
  const n = s.length;
  return n % 2 ? s[(n - 1) / 2] : (s[n / 2 - 1] + s[n / 2]) / 2;
}

function summarize(msPerRun) {
  const us = msPerRun.map((x) => x * 1e3);
  return { median: median(us), min: Math.min.apply(null, us), max: Math.max.apply(null, us), n: us.length };
}

function verdict(base, other) {
  const speedup = base.median / other.median;
  const v = other.max < base.min ? 'win' : other.min > base.max ? 'loss' : 'noise';
  return { speedup, verdict: v };
}

/** The counters that moved between two readings of tcmi_counters, by name. */
function created(before, after) {
  const out = {};
  for (const k of Object.keys(after)) if (after[k] !== before[k]) out[k] = after[k] - before[k];
  return out;
}

class TimedRegionError extends Error {
  constructor(what) {
    super(`objects created or data moved inside a timed region: ${JSON.stringify(what)}`);
    this.name = 'TimedRegionError';
    this.created = what;
  }
}

class HipBench {
  constructor(runner, options) {
    this.a = runner.a;
    this.graphs = !!(options && options.graphs);
    this.start = this.a.eventCreate();
    this.end = this.a.eventCreate();
    this.checked = 0;     // timed regions whose counters were checked
  }

  /**
   * Run `body` as a timed region: the counters must not move across it, except the
   * kinds listed in `allow` (a training step's batch upload and loss readback).
   * Returns body's result; throws TimedRegionError otherwise.
   */
  region(body, allow) {
    const before = this.a.counters();
    const r = body();
    const moved = created(before, this.a.counters());
    for (const k of allow || []) delete moved[k];
    if (Object.keys(moved).length) throw new TimedRegionError(moved);
    this.checked++;
    return r;
  }

  /**
   * One repetition: k runs of `program` between two events; ms per run. By
   * default the k runs' launches are issued directly, all in one native call,
   * so the GPU runs them back to back; with `graphs` the program is captured
   * once as a HIP graph and replayed k times.
   */
  rep(program, k, direct, leak) {
    const a = this.a;
    a.eventRecord(this.start);
    if (direct) program.runTimes(k);
    else for (let i = 0; i < k; i++) program.replay();
    if (leak) a.free(a.malloc(256));
    a.eventRecord(this.end);
    return a.eventElapsed(this.start, this.end) / k;
  }

  /** k for `program`: a repetition of at least TARGET_MS. */
  chooseK(program, opts) {
    const target = (opts && opts.targetMs) || TARGET_MS;
    const direct = !this.graphs || !!(opts && opts.direct);
    if (!direct) program.capture();
    this.rep(program, 1, direct);
    const one = this.rep(program, 1, direct);
    return Math.max(1, Math.min(MAX_K, Math.ceil(target / Math.max(one, 1e-4))));
  }

  /**
   * Time several variants (name -> Program) of one workload: k from the first
   * variant, warm-ups, then `reps` repetitions in ABBA order.
   * Returns { k, stats: {name: summary}, msPerRun: {name: [..]} }.
   */
  time(variants, opts) {
    const o = opts || {};
    const names = Object.keys(variants);
    const direct = !this.graphs || !!o.direct;
    const k = o.k || this.chooseK(variants[names[0]], o);
    for (const n of names) {
      if (!direct) variants[n].capture();
      for (let i = 0; i < (o.warmup === undefined ? WARMUP : o.warmup); i++) this.rep(variants[n], k, direct);
    }
    const msPerRun = {};
    for (const n of names) msPerRun[n] = [];
    const reps = o.reps || REPS;
    this.region(() => {
      for (let b = 0; b < reps; b++) {
        const order = b % 2 === 0 ? names : names.slice().reverse();
        for (const n of order) msPerRun[n].push(this.rep(variants[n], k, direct, !!o.leak));
      }
    });
    const stats = {};
    for (const n of names) stats[n] = summarize(msPerRun[n]);
    return { k, stats, msPerRun };
  }

  destroy() {
    this.a.eventDestroy(this.start);
    this.a.eventDestroy(this.end);
  }
}

module.exports = { HipBench, TimedRegionError, created, summarize, verdict, median, WARMUP, REPS, TARGET_MS };
