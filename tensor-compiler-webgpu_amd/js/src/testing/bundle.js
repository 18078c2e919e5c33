'use strict';
// A result bundle: what a CLI run on the GPU writes for an out-of-process
// checker to read — manifest.json (graphs, ids, where each array lives) plus
// data.f32, every float32 array of the run back to back.

const fs = require('fs');
const path = require('path');

class Bundle {
  constructor(dir) {
    this.dir = dir;
    fs.mkdirSync(dir, { recursive: true });
    this.file = path.join(dir, 'data.f32');
    this.fd = fs.openSync(this.file, 'w');
    this.offset = 0;  // in float32 elements
    this.manifest = { cases: [] };
  }

  /** Append a float array; returns { offset, n } in elements. */
  put(values) {
    const f = values instanceof Float32Array ? values : Float32Array.from(values);
    fs.writeSync(this.fd, Buffer.from(f.buffer, f.byteOffset, f.byteLength));
    const at = { offset: this.offset, n: f.length };
    this.offset += f.length;
    return at;
  }

  add(entry) { this.manifest.cases.push(entry); }

  close(extra) {
    fs.closeSync(this.fd);
    Object.assign(this.manifest, extra || {});
    fs.writeFileSync(path.join(this.dir, 'manifest.json'), JSON.stringify(this.manifest));
  }
}

module.exports = { Bundle };
