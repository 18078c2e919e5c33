'use strict';
// Loads the N-API addon over the tcmi C ABI (csrc/napi_addon.cpp -> lib/tcmi.node)
// and points it at the kernel headers and the code-object cache. There is no
// fallback: without the built addon every runner call fails with this error.

const path = require('path');
const fs = require('fs');

const PKG = path.resolve(__dirname, '..', '..', '..');
const LIB = path.join(PKG, 'lib');
const INCLUDE = path.join(PKG, 'csrc', 'kernels');
const CACHE = process.env.TCMI_KCACHE || path.join(PKG, '_build', 'kcache');

let loaded = null;

function addon() {
  if (loaded) return loaded;
  const file = path.join(LIB, 'tcmi.node');
  if (!fs.existsSync(file)) {
    throw new Error(`the MI355X backend is not built: ${file} is missing (run __graft_entry__.build())`);
  }
  const a = require(file);
  a.setIncludeDir(INCLUDE);
  a.setCacheDir(CACHE);
  loaded = a;
  return a;
}

module.exports = { addon, PKG, LIB, INCLUDE, CACHE };
