'use strict';
// Stream schedule of a launch list: independent launches on different streams,
// so that one launch's ramp-up and tail overlap another's instead of each
// launch waiting for the whole GPU to drain. The reference submits every launch
// to one in-order WebGPU queue (src/gpu/runtime.js:86-101 in
// abho7/tensor-compiler-webgpu); the results here are the same bits, because
// every launch still runs after the launches whose outputs it reads.
//
// A launch depends on the launch that wrote each of its operands (aliases
// resolved to the buffer's owner), and on the previous launch that used the
// workspace (split-K partials and column-sum partials share one scratch
// buffer). Each node buffer is written once per run, so those are the only
// hazards within a run; runs are ordered against each other by the fork and
// join tcmi_launch_dag adds. A launch goes on the stream whose last launch is
// its latest predecessor, if any is, else on the stream that has been idle
// longest; it waits, per other stream, for its latest predecessor there unless
// that stream has already been waited for up to it.

/**
 * Schedule `launches` (records of a lowering, in order) over `streams` streams.
 * `owner(id)`: the node whose buffer `id` uses. Returns, per kernel (a launch's
 * kernels stay together, in order, on its stream): streamOf (Uint8Array),
 * recordEvent (Int32Array, -1 for none), waitBegin (Uint32Array, count + 1),
 * waits (Uint32Array of event slots), and `events`, the slots used; plus
 * `criticalPath`, the longest dependency chain in launches.
 */
function scheduleLaunches(launches, streams, owner) {
  if (!(streams >= 1 && streams <= 4)) throw new Error(`streams must be 1..4, got ${streams}`);
  const n = launches.length;
  const writer = new Map();
  const preds = [];
  const depth = [];
  let lastWs = -1;
  launches.forEach((l, i) => {
    const p = new Set();
    for (const id of l.inputs) {
      const w = writer.get(owner(id));
      if (w !== undefined) p.add(w);
    }
    if (l.workspace > 0) {
      if (lastWs >= 0) p.add(lastWs);
      lastWs = i;
    }
    preds.push(Array.from(p).sort((a, b) => a - b));
    depth.push(1 + preds[i].reduce((d, j) => Math.max(d, depth[j]), 0));
    writer.set(owner(l.node), i);
  });
  const streamOfLaunch = new Array(n);
  const last = new Array(streams).fill(-1);          // last launch on each stream
  const waited = [];                                  // waited[s][t]: launch of t that s has waited for
  for (let s = 0; s < streams; s++) waited.push(new Array(streams).fill(-1));
  const waitsOf = [];                                 // launch indices each launch waits for
  for (let i = 0; i < n; i++) {
    let s = -1;
    for (let t = 0; t < streams; t++) if (last[t] >= 0 && preds[i].includes(last[t]) && (s < 0 || last[t] > last[s])) s = t;
    if (s < 0) {
      s = 0;
      for (let t = 1; t < streams; t++) if (last[t] < last[s]) s = t;
    }
    const w = [];
    for (let t = 0; t < streams; t++) {
      if (t === s) continue;
      let latest = -1;
      for (const j of preds[i]) if (streamOfLaunch[j] === t && j > latest) latest = j;
      if (latest >= 0 && latest > waited[s][t]) {
        w.push(latest);
        waited[s][t] = latest;
      }
    }
    streamOfLaunch[i] = s;
    last[s] = i;
    waitsOf.push(w);
  }
  // Event slots for the launches some other launch waits for.
  const slot = new Map();
  for (const w of waitsOf) for (const j of w) if (!slot.has(j)) slot.set(j, slot.size);
  const kernels = launches.reduce((c, l) => c + l.kernels.length, 0);
  const streamOf = new Uint8Array(kernels);
  const recordEvent = new Int32Array(kernels).fill(-1);
  const waitBegin = new Uint32Array(kernels + 1);
  const waitList = [];
  let k = 0;
  launches.forEach((l, i) => {
    l.kernels.forEach((_, j) => {
      streamOf[k] = streamOfLaunch[i];
      waitBegin[k] = waitList.length;
      if (j === 0) for (const p of waitsOf[i]) waitList.push(slot.get(p));
      if (j === l.kernels.length - 1 && slot.has(i)) recordEvent[k] = slot.get(i);
      k++;
    });
  });
  waitBegin[kernels] = waitList.length;
  return { streams, streamOf, recordEvent, waitBegin, waits: Uint32Array.from(waitList), events: slot.size,
    criticalPath: n ? Math.max(...depth) : 0, launches: n };
}

module.exports = { scheduleLaunches };
