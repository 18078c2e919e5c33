'use strict';
// Seeded random numbers: mulberry32 (a public-domain 32-bit generator), so a
// run is reproducible from one integer. It is the generator the reference's
// src/testing/rng.js uses, kept bit-compatible so that parameters drawn with
// the reference's seeding (e.g. its transformer's initParams) are the values
// its committed PyTorch goldens were computed from. Normal draws (which the
// reference has none of) use Box–Muller on two uniforms.

class Rng {
  constructor(seed) { this.state = seed >>> 0; }

  /** Uniform in [0, 1). */
  next() {
    this.state = (this.state + 0x6d2b79f5) >>> 0;
    let t = this.state;
    t = Math.imul(t ^ (t >>> 15), t | 1);
    t ^= t + Math.imul(t ^ (t >>> 7), t | 61);
    return ((t ^ (t >>> 14)) >>> 0) / 4294967296;
  }

  int(lo, hi) { return lo + Math.floor(this.next() * (hi - lo + 1)); }
  uniform(lo, hi) { return lo + (hi - lo) * this.next(); }
  pick(list) { return list[Math.floor(this.next() * list.length)]; }
  chance(p) { return this.next() < p; }
  array(n, lo, hi) {
    if (lo === undefined) { lo = -1; hi = 1; }
    const out = new Array(n);
    for (let i = 0; i < n; i++) out[i] = this.uniform(lo, hi);
    return out;
  }

  /** One N(0, 1) draw (Box–Muller; the second value of each pair is kept for the next call). */
  normal() {
    if (this.spare !== undefined) { const s = this.spare; this.spare = undefined; return s; }
    let u = this.next();
    while (u === 0) u = this.next();
    const v = this.next();
    const r = Math.sqrt(-2 * Math.log(u));
    this.spare = r * Math.sin(2 * Math.PI * v);
    return r * Math.cos(2 * Math.PI * v);
  }

  /** `n` float32 draws from N(0, std^2) into a Float32Array. */
  normalF32(n, std) {
    const out = new Float32Array(n);
    for (let i = 0; i < n; i++) out[i] = std * this.normal();
    return out;
  }

  shuffle(list) {
    const a = list.slice();
    for (let i = a.length - 1; i > 0; i--) {
      const j = Math.floor(this.next() * (i + 1));
      const t = a[i]; a[i] = a[j]; a[j] = t;
    }
    return a;
  }
}

module.exports = { Rng };
