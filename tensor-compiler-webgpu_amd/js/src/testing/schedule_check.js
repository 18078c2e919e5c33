'use strict';
// An independent check of a stream schedule: replay it with vector clocks, the
// way in-order streams and event waits order work, and require every launch to
// run after the launch that wrote each operand it reads and after the previous
// workspace user. The clocks know nothing of how the scheduler chose streams or
// waits, so a dropped or misplaced wait fails here.

function checkSchedule(launches, sched, owner) {
  const S = sched.streams;
  const clock = [];                       // per stream: latest launch of each stream known complete
  for (let s = 0; s < S; s++) clock.push(new Array(S).fill(-1));
  const after = [];                       // clock right after each launch (what its event carries)
  const kernelOf = [];                    // launch -> its first and last kernel index
  let k = 0;
  for (const l of launches) { kernelOf.push([k, k + l.kernels.length - 1]); k += l.kernels.length; }
  const eventLaunch = new Map();          // event slot -> launch that records it (latest)
  const onStream = [];
  const writer = new Map();
  let lastWs = -1;
  for (let i = 0; i < launches.length; i++) {
    const l = launches[i];
    const [k0, k1] = kernelOf[i];
    const s = sched.streamOf[k0];
    for (let kk = k0; kk <= k1; kk++) if (sched.streamOf[kk] !== s) return { ok: false, launch: i, why: 'kernels of one launch on two streams' };
    for (let w = sched.waitBegin[k0]; w < sched.waitBegin[k0 + 1]; w++) {
      const j = eventLaunch.get(sched.waits[w]);
      if (j === undefined) return { ok: false, launch: i, why: `waits for event ${sched.waits[w]} before it is recorded` };
      for (let t = 0; t < S; t++) clock[s][t] = Math.max(clock[s][t], after[j][t]);
    }
    // Every predecessor must be known complete on this stream (or be earlier on it).
    const need = [];
    for (const id of l.inputs) if (writer.has(owner(id))) need.push(writer.get(owner(id)));
    if (l.workspace > 0 && lastWs >= 0) need.push(lastWs);
    for (const j of need) {
      const t = onStream[j];
      if (clock[s][t] < j) return { ok: false, launch: i, why: `may run before launch ${j} (stream ${t})` };
    }
    clock[s][s] = i;
    after[i] = clock[s].slice();
    onStream[i] = s;
    if (sched.recordEvent[k1] >= 0) eventLaunch.set(sched.recordEvent[k1], i);
    writer.set(owner(l.node), i);
    if (l.workspace > 0) lastWs = i;
  }
  return { ok: true };
}

module.exports = { checkSchedule };
