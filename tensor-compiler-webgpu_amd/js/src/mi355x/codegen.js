'use strict';
// HIP source for every launch the MI355X lowering plans, as text, so it can be
// generated and inspected without a GPU. The runner compiles it with hiprtc.
//
// The reference generates one WGSL kernel per fused node from its body
// (src/fusion/codegen-fused.js:154-362 in abho7/tensor-compiler-webgpu) and
// one per plain op (src/gpu/codegen.js). Here the kernel *skeletons* are
// hand-written for gfx950 and live in csrc/kernels/tcmi_device.h and
// tcmi_gemm.h; this file writes only what varies per launch:
//   * the body of the fused node as straight-line float arithmetic, every
//     value a register, each op through the shared tcmi::op_* helpers (so a
//     fused body rounds exactly as the chain of unfused kernels does);
//   * the load of every operand, classified by how its index follows from the
//     output index (flat, a contiguous `span` of axes, or a general gather),
//     and hoisted into 128-bit loads where the classification allows;
//   * the u32 parameter block P (sizes and index maps), so one kernel text
//     serves every size of the same structure and class.
//
// Kernel kinds:
//   elementwise  grid-stride loop, 4 elements per thread per step (float4)
//   rowwise      one workgroup per row, the row's operands held in registers
//                across every reduction phase (read from HBM once), max-shift
//                and normalisation applied in-kernel
//   colreduce    sum/max over a non-last axis: split-n partials + a final pass
//   gemm         fp32 MFMA matmul with the fused epilogue applied at the store

const { size, strides } = require('../ir/shapes');

const MAX_P = 48;
const MAX_IN = 8;
const WG = 256;

const f32 = new Float32Array(1);
const u32 = new Uint32Array(f32.buffer);
/** The exact float32 bits of `v` (rounded to nearest), as a C++ expression. */
function literal(v) {
  f32[0] = v;
  return `tcmi::f32_bits(0x${u32[0].toString(16).padStart(8, '0')}u)`;
}

/** FNV-1a over a string, as 8 hex digits (kernel names). */
function fnv(s) {
  let h = 0x811c9dc5;
  for (let i = 0; i < s.length; i++) {
    h ^= s.charCodeAt(i);
    h = Math.imul(h, 0x01000193) >>> 0;
  }
  return h.toString(16).padStart(8, '0');
}

const UNARY = { neg: 'op_neg', exp: 'op_exp', log: 'op_log', relu: 'op_relu', tanh: 'op_tanh', sqrt: 'op_sqrt',
  step: 'op_step', stopGradient: 'op_copy', copy: 'op_copy' };
const BINARY = { add: 'op_add', sub: 'op_sub', mul: 'op_mul', div: 'op_div' };

/**
 * How a gather node (broadcast or transpose of its input) maps its output
 * flat index to its source flat index: { mode: 'zero' | 'span' | 'general', ... }.
 */
function classifyGather(node, inShape) {
  const out = node.shape;
  if (node.op === 'broadcast') {
    const lead = out.length - inShape.length;
    const kept = [];
    for (let d = 0; d < out.length; d++) if (d >= lead && inShape[d - lead] !== 1) kept.push(d);
    if (kept.length === 0) return { mode: 'zero' };
    let contiguous = true;
    for (let k = 1; k < kept.length; k++) if (kept[k] !== kept[k - 1] + 1) contiguous = false;
    if (contiguous) {
      const d0 = kept[0], d1 = kept[kept.length - 1];
      return { mode: 'span', inner: size(out.slice(d1 + 1)), extent: size(out.slice(d0, d1 + 1)) };
    }
  }
  // General: per output axis, its extent and the source stride (lower.js:31-62's gather strides).
  const st = gatherStrides(node, inShape);
  return { mode: 'general', extents: out.slice(), strides: st };
}

function gatherStrides(node, inShape) {
  const out = node.shape;
  const natural = strides(inShape);
  if (node.op === 'broadcast') {
    const lead = out.length - inShape.length;
    return out.map((_, i) => (i < lead || inShape[i - lead] === 1 ? 0 : natural[i - lead]));
  }
  if (node.op === 'transpose') return node.attrs.perm.map((p) => natural[p]);
  if (node.op === 'reshape') return strides(out);
  throw new Error(`not a gather: ${node.op}`);
}

/**
 * The straight-line body writer shared by every kernel kind. A context is an
 * index expression (the flat index at which values are wanted); every body
 * value is computed once per context. `hooks` lets a kernel kind supply the
 * loads of operands and the values of nodes it treats specially (the matmul
 * root of an epilogue, the reductions of a rowwise body).
 */
/** A kernel whose parameter words (its sizes and index maps) would not fit one argument block. */
class ParamOverflow extends Error {
  constructor(message) { super(message); this.name = 'ParamOverflow'; }
}

class Emitter {
  constructor(body, params, hooks, slack) {
    this.b = body;
    this.params = params;
    this.hooks = hooks;
    this.memo = new Map();
    this.counter = 0;
    this.gatherBase = new Map();
    // Elements an operand may be read past its end (only the deliberately broken
    // bounds check of a sabotaged kernel reads one past, into the canary pad).
    this.slack = slack || 0;
  }

  fresh(prefix) { return `${prefix}${this.counter++}`; }

  /**
   * Index expression of the source of gather node `node` read in `ctx`. Every
   * context carries `limit`, one past the largest index it can produce; the
   * gather's own output must cover it and its largest source index must fall
   * inside its source, so every load the kernel makes is proved in bounds here.
   */
  gatherIndex(node, ctx) {
    const inShape = this.b.nodes[node.inputs[0]].shape;
    const g = classifyGather(node, inShape);
    if (ctx.limit === undefined || ctx.limit > size(node.shape) + this.slack) {
      throw new Error(`gather node ${node.id}: read at ${ctx.limit} indices, has ${size(node.shape)} elements`);
    }
    let maxSrc = 0;
    if (g.mode === 'span') maxSrc = g.extent - 1;
    else if (g.mode === 'general') g.extents.forEach((e, d) => { maxSrc += (e - 1) * g.strides[d]; });
    if (maxSrc >= size(inShape)) throw new Error(`gather node ${node.id}: source index ${maxSrc} outside ${size(inShape)} elements`);
    if (g.mode === 'zero') return { idx: '0u', g };
    const key = `${node.id}`;
    let base = this.gatherBase.get(key);
    if (base === undefined) {
      base = this.params.length;
      if (g.mode === 'span') this.params.push(g.inner, g.extent);
      else {
        const rank = g.extents.length;
        this.params.push(rank);
        for (let d = rank - 1; d >= 0; d--) this.params.push(g.extents[d], g.strides[d]);
      }
      if (this.params.length > MAX_P) throw new ParamOverflow(`kernel parameters exceed ${MAX_P} words`);
      this.gatherBase.set(key, base);
    }
    // The index maps are baked into the kernel text as constants (the lowering
    // knows every shape): divisions and remainders by powers of two become
    // shifts and masks, the rest multiplications. P keeps them for inspection.
    if (g.mode === 'span') {
      if (g.inner === 1) return { idx: `((${ctx.idx}) % ${g.extent}u)`, g, base };
      return { idx: `(((${ctx.idx}) / ${g.inner}u) % ${g.extent}u)`, g, base };
    }
    let e = '0u';
    let rem = `(${ctx.idx})`;
    const terms = [];
    for (let d = g.extents.length - 1; d >= 0; d--) {
      const ext = g.extents[d], st = g.strides[d];
      if (st !== 0 && ext > 1) terms.push(`((${rem}) % ${ext}u) * ${st}u`);
      rem = `(${rem}) / ${ext}u`;
    }
    if (terms.length) e = terms.join(' + ');
    return { idx: `(${e})`, g, base };
  }

  value(id, ctx, lines) {
    const key = `${ctx.key}|${id}`;
    if (this.memo.has(key)) return this.memo.get(key);
    const node = this.b.nodes[id];
    let v;
    const special = this.hooks.special ? this.hooks.special(id, ctx, lines) : undefined;
    if (special !== undefined) {
      v = special;
    } else if (node.op === 'input') {
      if (ctx.limit === undefined || ctx.limit > size(node.shape) + this.slack) {
        throw new Error(`operand ${node.attrs.name}: read at ${ctx.limit} indices, has ${size(node.shape)} elements`);
      }
      v = this.hooks.load(Number(node.attrs.name.slice(1)), ctx, lines, node);
    } else if (node.op === 'const') {
      v = literal(typeof node.attrs.value === 'number' ? node.attrs.value : node.attrs.value[0]);
    } else if (node.op === 'reshape') {
      v = this.value(node.inputs[0], ctx, lines);
    } else if (node.op === 'broadcast' || node.op === 'transpose') {
      const src = this.b.nodes[node.inputs[0]];
      if (src.op === 'const') {
        v = this.value(src.id, ctx, lines);
      } else {
        const gi = this.gatherIndex(node, ctx);
        const child = { key: `${ctx.key}>${node.id}`, idx: gi.idx, parent: ctx, gather: gi, root: false, row: ctx.row,
          limit: size(src.shape) };
        v = this.value(src.id, child, lines);
      }
    } else if (BINARY[node.op]) {
      const a = this.value(node.inputs[0], ctx, lines);
      const c = this.value(node.inputs[1], ctx, lines);
      v = this.fresh('v');
      lines.push(`const float ${v} = tcmi::${BINARY[node.op]}(${a}, ${c});`);
    } else if (UNARY[node.op]) {
      const a = this.value(node.inputs[0], ctx, lines);
      v = this.fresh('v');
      lines.push(`const float ${v} = tcmi::${UNARY[node.op]}(${a});`);
    } else {
      throw new Error(`mi355x codegen: no rule for '${node.op}' in this kernel kind`);
    }
    this.memo.set(key, v);
    return v;
  }
}

const inputCount = (b) => b.nodes.filter((n) => n.op === 'input').length;

function checkOperands(b) {
  const k = inputCount(b);
  if (k > MAX_IN) throw new Error(`kernel has ${k} operands; the argument block holds ${MAX_IN}`);
  return k;
}

function kernelText(kind, bodyText) {
  const name = `tcmi_${kind}_${fnv(bodyText)}`;
  return { name, source: bodyText.replace(/__KERNEL__/g, name) };
}

const indent = (lines, pad) => lines.map((l) => pad + l).join('\n');

// ---- elementwise ------------------------------------------------------------------

/**
 * A fused (or one-op) elementwise body over n output elements, output node
 * `output` of body graph `b`. A grid-stride loop over float4 groups with at
 * most `blocks` workgroups (below): each trip a thread loads U groups spaced one grid apart (every
 * operand load of all U issued before any arithmetic), computes, and stores
 * (non-temporally by default: the output is not re-read by this kernel). A
 * scalar tail handles n % 4. Operands read at the output index are float4
 * loads; a span load is a float4 when its 4 lanes are contiguous in the source,
 * one scalar when they share an element, else 4 scalars.
 * `tuning`: { unroll (U), nt (default true), ntl (non-temporal loads of the full-size
 * operands, default false), blocks }. Defaults by size, from
 * whole-program sweeps on the MI355X: up to 8192 workgroups, U = 1 below 2^25
 * elements, so up to 2^23 elements every thread handles one group and the loop runs
 * once (config 2's 32 MB tensors, with the runtime's staggered allocations: its
 * step 5.79 -> 5.97-5.99 TB/s and its largest kernel read cold 5.18 -> 5.45 TB/s
 * against 2048 workgroups; 1024 workgroups or U = 2 were slower on the step); 512
 * workgroups, U = 2 from 2^25 up (config 3's 268 MB tensors: 6 % faster over its
 * programs).
 */
function elementwiseKernel(b, output, outShape, opts) {
  const o = opts || {};
  const tune = o.tuning || {};
  const n = size(outShape);
  const large = n >= 2 ** 25;
  // Two float4 groups a thread per pass: measured 2 % faster than one on a cold 2^23-element
  // three-operand kernel at 8192 blocks (one group a thread taken, the second guarded out:
  // the difference is the compiled loop), neutral on the small kernels of the training steps.
  const U = tune.unroll || 2;
  // Non-temporal stores unless the lowering says the next launch reads the output
  // (streamOut false), which then finds it in the caches; tuning nt forces either way.
  const nt = tune.nt === undefined ? o.streamOut !== false : !!tune.nt;
  // Non-temporal loads: every full-size operand (tuning ntl), or those at the positions
  // `o.lastReads` lists (the lowering's last reads of their buffers).
  const ntlAt = new Set(tune.ntl ? [] : (o.lastReads || []));
  const ntl = (k) => !!tune.ntl || ntlAt.has(k);
  const maxBlocks = tune.blocks || (large ? 512 : 8192);
  checkOperands(b);
  if (n >= 2 ** 31) throw new Error(`elementwise kernel over ${n} elements exceeds the 32-bit index space`);
  const params = [n];

  // Vector pass: hoisted loads fill per-group arrays in `hoist`; lane code in `lane`.
  const decl = [];
  const hoist = [];
  const hoisted = new Map();
  const hoistAs = (key, type, expr) => {
    if (!hoisted.has(key)) {
      const h = `H${hoisted.size}`;
      decl.push(`${type} ${h}[${U}];`);
      hoist.push(`${h}[j] = ${expr};`);
      hoisted.set(key, h);
    }
    return hoisted.get(key);
  };
  const vecEmitter = new Emitter(b, params, {
    load(k, ctx, lines) {
      if (ctx.root) {
        const load = ntl(k) ? `__builtin_nontemporal_load(reinterpret_cast<const tcmi::f4*>(A.in[${k}]) + v)`
          : `reinterpret_cast<const tcmi::f4*>(A.in[${k}])[v]`;
        return `${hoistAs(`full${k}`, 'tcmi::f4', load)}[j][l]`;
      }
      const g = ctx.gather;
      if (ctx.parent && ctx.parent.root && g) {
        if (g.g.mode === 'zero') return `${hoistAs(`zero${k}`, 'float', `A.in[${k}][0]`)}[j]`;
        if (g.g.mode === 'span' && g.g.inner === 1 && g.g.extent % 4 === 0) {
          return `${hoistAs(`spanv${k}|${ctx.key}`, 'tcmi::f4',
            `reinterpret_cast<const tcmi::f4*>(A.in[${k}])[(i0 % ${g.g.extent}u) >> 2]`)}[j][l]`;
        }
        if (g.g.mode === 'span' && g.g.inner % 4 === 0) {
          return `${hoistAs(`spans${k}|${ctx.key}`, 'float', `A.in[${k}][(i0 / ${g.g.inner}u) % ${g.g.extent}u]`)}[j]`;
        }
      }
      const v = `L${lines.length}_${k}`;
      lines.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
      return v;
    },
  });
  const lane = [];
  const vout = vecEmitter.value(output, { key: 'i', idx: 'i', root: true, limit: n }, lane);

  // Scalar tail: the same body, every load scalar. The reference's sabotage
  // 'fused-bounds-off-by-one' (codegen-fused.js:160) lets one thread past the
  // end: it reads every flat operand and writes the output at index n, one
  // element into the canary pad that check-mode buffers carry (the record is
  // marked so the runner refuses it without canaries); gathers stay in range
  // (every axis index is taken modulo its extent).
  const offByOne = o.sabotage === 'fused-bounds-off-by-one';
  const tailEmitter = new Emitter(b, params, {
    load(k, ctx, lines) {
      const v = `T${lines.length}_${k}`;
      lines.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
      return v;
    },
  }, offByOne ? 1 : 0);
  tailEmitter.gatherBase = vecEmitter.gatherBase;  // same parameter offsets
  const tail = [];
  const tout = tailEmitter.value(output, { key: 'i', idx: 'i', root: true, limit: offByOne ? n + 1 : n }, tail);

  const guard = offByOne ? 'threadIdx.x <= (n & 3u)' : 'threadIdx.x < (n & 3u)';
  const store = nt ? '__builtin_nontemporal_store(o4, reinterpret_cast<tcmi::f4*>(A.out) + v);'
    : 'reinterpret_cast<tcmi::f4*>(A.out)[v] = o4;';
  const text = `extern "C" __global__ void __launch_bounds__(${WG}) __KERNEL__(const TcmiArgs A) {
  const uint32_t n = ${n}u;
  const uint32_t nv = n >> 2;
  const uint32_t stride = gridDim.x * ${WG}u;
  for (uint32_t base = blockIdx.x * ${WG}u + threadIdx.x; base < nv; base += ${U}u * stride) {
${indent(decl, '    ')}
#pragma unroll
    for (int j = 0; j < ${U}; ++j) {
      const uint32_t v = base + j * stride;
      if (v < nv) {
        const uint32_t i0 = v << 2;
${indent(hoist, '        ')}
      }
    }
#pragma unroll
    for (int j = 0; j < ${U}; ++j) {
      const uint32_t v = base + j * stride;
      if (v < nv) {
        const uint32_t i0 = v << 2;
        float r[4];
#pragma unroll
        for (int l = 0; l < 4; ++l) {
          const uint32_t i = i0 + l;
${indent(lane, '          ')}
          r[l] = ${vout};
        }
        const tcmi::f4 o4 = {r[0], r[1], r[2], r[3]};
        ${store}
      }
    }
  }
  if (blockIdx.x == 0 && ${guard}) {
    const uint32_t i = (nv << 2) + threadIdx.x;
${indent(tail, '    ')}
    A.out[i] = ${tout};
  }
}
`;
  const k = kernelText('ew', text);
  const groups = Math.max(1, Math.min(Math.ceil(Math.max(1, n >> 2) / WG), maxBlocks));
  return { name: k.name, source: k.source, params: Uint32Array.from(params), grid: [groups, 1, 1], block: [WG, 1, 1], lds: 0, workspace: 0,
    needsPad: offByOne };
}

// ---- rowwise ------------------------------------------------------------------------

const isReduce = (n) => n.op === 'sum' || n.op === 'max';

/**
 * A rowwise body: last-axis sum/max reductions of element-tier values ([R, C])
 * and row-tier values ([R, 1]) built from them, output at element or row tier.
 * Every element-tier operand load is made once into registers and reused by
 * every phase, so each input is read from HBM once, whatever the number of
 * reductions. A row is owned by L lanes: for C >= 2048 a whole workgroup of
 * 256 (reduced through LDS), otherwise a group of 16, 32 or 64 lanes of one
 * wavefront — enough for about two float4 slots per lane — reduced by
 * butterfly shuffles, with 256 / L rows per workgroup, so short
 * rows (attention's 128, LayerNorm's 256) still move a full workgroup's worth
 * of data per launch slot. Rows are walked grid-stride.
 */
function rowwiseKernel(b, output, opts) {
  const o = opts || {};
  // Operand positions whose full-size loads are the lowering's last reads of their
  // buffers: loaded non-temporally (row length a multiple of 4 only).
  const streamed = new Set(o.lastReads || []);
  // Full-size output that the next launch does not read: stored non-temporally, so it
  // does not displace data that launch reads from the caches (tuning nto forces either way).
  const tuneRow = o.tuning || {};
  const ntOut = tuneRow.nto === undefined ? o.streamOut === true : !!tuneRow.nto;
  checkOperands(b);
  const reductions = b.nodes.filter(isReduce);
  if (!reductions.length) throw new Error('rowwise kernel without a reduction');
  const S = b.nodes[reductions[0].inputs[0]].shape;
  const C = S[S.length - 1];
  const R = size(S) / C;
  if (size(S) >= 2 ** 31) throw new Error('rowwise kernel exceeds the 32-bit index space');
  const vec = C % 4 === 0;
  const W = vec ? 4 : 1;                     // elements per slot
  const pow2 = (x) => 2 ** Math.ceil(Math.log2(Math.max(1, x)));
  const lanes = o.tuning && o.tuning.lanes;
  // Lanes per row: 256 (the workgroup) for long rows; otherwise enough for two
  // slots per lane, 16 to 64 (an on-device sweep: one slot per lane left short
  // rows' loads too thin, more than four made the register cache too large).
  const T = lanes || (C >= 2048 ? 256 : Math.min(64, Math.max(16, pow2(Math.ceil(C / (2 * W))))));
  const BLOCK = 256;
  const G = BLOCK / T;                        // rows per workgroup
  const E = Math.max(1, Math.ceil(C / (W * T)));  // slots per thread
  const params = [R, C];
  const rowTier = (id) => size(b.nodes[id].shape) === R && size(b.nodes[id].shape) !== R * C;
  const outRow = rowTier(output) || (R === size(b.nodes[output].shape) && C !== 1 && size(b.nodes[output].shape) !== R * C);

  // Loads at the element index: cached per load site in registers. `fills` keeps
  // each cache's kind in first-use order; the kernel text declares and fills them.
  const fills = [];
  const caches = new Map();
  const reduced = new Map();
  const rowLines = [];    // row-tier statements, emitted as they are first needed
  const rowNames = new Set();
  let em;
  const ROW = { key: 'r', idx: 'r', root: false, row: true, limit: R };
  const elemCtx = () => ({ key: 'e', idx: 'e', root: true, limit: R * C });
  const cache = (ck, k, mode) => {
    if (!caches.has(ck)) {
      const c = `X${caches.size}`;
      caches.set(ck, c);
      fills.push({ c, k, mode });
    }
    return caches.get(ck);
  };

  const hooks = {
    special(id, ctx, lines) {
      if (reduced.has(id)) return reduced.get(id);
      const n = b.nodes[id];
      if (!ctx.row && rowTier(id) && n.op !== 'input' && n.op !== 'const') return em.value(id, ROW, rowLines);
      if (n.op === 'broadcast' && !ctx.row && rowTier(n.inputs[0])) {
        const src = b.nodes[n.inputs[0]];
        if (src.op !== 'input' && src.op !== 'const') return em.value(src.id, ROW, rowLines);
      }
      return undefined;
    },
    load(k, ctx, lines, node) {
      if (ctx.row) {
        // A row-tier operand at the row index. Row lines are taken out per phase and emitted
        // in the row loop's scope one phase after another, so a name is kept unique by suffix.
        let v = `R${rowLines.length}_${k}`;
        if (rowNames.has(v)) v = `${v}_${rowNames.size}`;
        rowNames.add(v);
        lines.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
        return v;
      }
      if (ctx.root) {
        // The lowering's last read of a buffer is streamed past the caches.
        const c = cache(`full${k}`, k, !vec ? 'scalar' : streamed.has(k) ? 'nt' : 'vec');
        return vec ? `tcmi::lane4(${c}[s], l)` : `${c}[s]`;
      }
      const g = ctx.gather;
      if (vec && ctx.parent && ctx.parent.root && g && g.g.mode === 'span' && g.g.inner === 1 && g.g.extent === C) {
        // A per-column vector (LayerNorm gain/bias): cached like a full operand.
        return `tcmi::lane4(${cache(`col${k}`, k, 'col')}[s], l)`;
      }
      const v = `L${lines.length}_${k}`;
      lines.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
      return v;
    },
  };
  // The lines filling cache `f` into array `dst` from the row at `rowBase`.
  const fillLines = (f, dst) => {
    const head = [`#pragma unroll`];
    if (f.mode === 'nt') {
      return head.concat([`for (int s = 0; s < ${E}; ++s) { const uint32_t c0 = (ln + s * ${T}u) * 4u;`,
        `  tcmi::f4 t = {0.f, 0.f, 0.f, 0.f};`,
        `  if (c0 < C) t = __builtin_nontemporal_load(reinterpret_cast<const tcmi::f4*>(A.in[${f.k}] + rowBase) + (c0 >> 2));`,
        `  ${dst}[s] = make_float4(t[0], t[1], t[2], t[3]); }`]);
    }
    if (f.mode === 'vec' || f.mode === 'col') {
      const src = f.mode === 'col' ? `A.in[${f.k}]` : `A.in[${f.k}] + rowBase`;
      return head.concat([`for (int s = 0; s < ${E}; ++s) { const uint32_t c0 = (ln + s * ${T}u) * 4u;`,
        `  ${dst}[s] = c0 < C ? reinterpret_cast<const float4*>(${src})[c0 >> 2] : make_float4(0.f, 0.f, 0.f, 0.f); }`]);
    }
    return head.concat([`for (int s = 0; s < ${E}; ++s) { const uint32_t c0 = ln + s * ${T}u;`,
      `  ${dst}[s] = c0 < C ? A.in[${f.k}][rowBase + c0] : 0.f; }`]);
  };
  const cacheType = (f) => (f.mode === 'scalar' ? 'float' : 'float4');
  em = new Emitter(b, params, hooks);

  // One element loop: `body` runs for every valid element with `e` its flat index.
  const loop = (bodyLines) => vec
    ? `#pragma unroll
for (int s = 0; s < ${E}; ++s) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t c = (ln + s * ${T}u) * 4u + l;
    if (c < C) {
      const uint32_t e = rowBase + c;
${indent(bodyLines, '      ')}
    }
  }
}`
    : `#pragma unroll
for (int s = 0; s < ${E}; ++s) {
  const uint32_t c = ln + s * ${T}u;
  if (c < C) {
    const uint32_t e = rowBase + c;
${indent(bodyLines, '    ')}
  }
}`;

  const phases = [];
  const shortTree = o.sabotage === 'layernorm-tree-short' && o.pattern === 'layernorm';
  reductions.forEach((rd, k) => {
    for (const key of Array.from(em.memo.keys())) if (key.startsWith('e')) em.memo.delete(key);
    const rowBefore = rowLines.length;
    const inner = [];
    const v = em.value(rd.inputs[0], elemCtx(), inner);
    const isMax = rd.op === 'max';
    const pre = rowLines.splice(rowBefore);
    const acc = `acc${k}`;
    const reduce = (v) => (T === 256 ? `tcmi::block_reduce<${isMax}, 256>(${v}, red)` : `tcmi::group_reduce<${isMax}, ${T}>(${v})`);
    let result = reduce(acc);
    if (shortTree) result = reduce(`ln < ${T / 2}u ? ${acc} : ${isMax ? '(-TCMI_INF)' : '0.f'}`);
    if (o.sabotage === 'softmax-no-max' && isMax && (o.pattern === 'softmax' || o.pattern === 'log-softmax')) result = '0.f';
    phases.push(...pre,
      `float ${acc} = ${isMax ? '(-TCMI_INF)' : '0.f'};`,
      loop(inner.concat([`${acc} = tcmi::red_${isMax ? 'max' : 'sum'}(${acc}, ${v});`])),
      `const float red${k} = ${result};`);
    reduced.set(rd.id, `red${k}`);
  });
  for (const key of Array.from(em.memo.keys())) if (key.startsWith('e')) em.memo.delete(key);
  let store;
  if (outRow) {
    const rowBefore = rowLines.length;
    const v = em.value(output, ROW, rowLines);
    const pre = rowLines.splice(rowBefore);
    store = [...pre, `if (ln == 0) A.out[r] = ${v};`];
  } else {
    const rowBefore = rowLines.length;
    const inner = [];
    const v = em.value(output, elemCtx(), inner);
    const pre = rowLines.splice(rowBefore);
    if (vec) {
      // Compute the 4 lanes of each slot, then one 128-bit store.
      store = [...pre, `#pragma unroll
for (int s = 0; s < ${E}; ++s) {
  const uint32_t c0 = (ln + s * ${T}u) * 4u;
  if (c0 < C) {
    float o4[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t c = c0 + l;
      const uint32_t e = rowBase + c;
${indent(inner, '      ')}
      o4[l] = ${v};
    }
    ${ntOut ? '__builtin_nontemporal_store(tcmi::f4{o4[0], o4[1], o4[2], o4[3]}, reinterpret_cast<tcmi::f4*>(A.out + rowBase) + (c0 >> 2));'
    : 'reinterpret_cast<float4*>(A.out + rowBase)[c0 >> 2] = make_float4(o4[0], o4[1], o4[2], o4[3]);'}
  }
}`];
    } else {
      store = [...pre, loop(inner.concat([`A.out[e] = ${v};`]))];
    }
  }
  const cacheDecl = [];
  for (const f of fills) cacheDecl.push(`${cacheType(f)} ${f.c}[${E}];`, ...fillLines(f, f.c));
  const text = `extern "C" __global__ void __launch_bounds__(${BLOCK}) __KERNEL__(const TcmiArgs A) {
${T === 256 ? '  __shared__ float red[4];\n' : ''}  const uint32_t R = ${R}u;
  const uint32_t C = ${C}u;
  const uint32_t ln = threadIdx.x % ${T}u;     // lane within the row's group
  for (uint32_t r = blockIdx.x * ${G}u + threadIdx.x / ${T}u; r < R; r += gridDim.x * ${G}u) {
    const uint32_t rowBase = r * C;
${indent(cacheDecl, '    ')}
${indent(phases, '    ')}
${indent(store, '    ')}
  }
}
`;
  const k = kernelText('row', text);
  const cap = (o.tuning && o.tuning.blocks) || 65536;
  const groups = Math.max(1, Math.min(Math.ceil(R / G), cap));
  return { name: k.name, source: k.source, params: Uint32Array.from(params), grid: [groups, 1, 1], block: [BLOCK, 1, 1], lds: 0, workspace: 0 };
}

// ---- column reductions (sum / max over a non-last axis) --------------------------------

/**
 * out[o, j] = reduce_k x[o, k, j] over [outer, n, inner] with inner > 1: the
 * column sums autodiff emits for every broadcast operand (bias gradients).
 * Vector form (inner % 4 == 0): a workgroup owns 256 columns (each lane a
 * float4 of them) and a chunk of rows; its 4 wavefronts take every 4th row of
 * the chunk, 128-bit loads, and their partials meet in LDS. Enough row chunks
 * are made to give every CU work; each chunk's partial goes to the workspace,
 * and a second kernel combines the chunks, again 4 wavefronts per column tile.
 * Every output sums its terms in a fixed order (deterministic). Scalar form
 * (inner % 4 != 0): the same with one column per lane.
 */
/** Elements up to which a column reduction runs in one launch (256 KB of fp32). */
const COLRED_ONE_PASS = 1 << 16;

function colreduceKernels(op, outer, n, inner, tuning, producer, chain) {
  const tune = tuning || {};
  const isMax = op === 'max';
  const init = isMax ? '(-TCMI_INF)' : '0.f';
  const comb = isMax ? 'tcmi::red_max' : 'tcmi::red_sum';
  const vec = inner % 4 === 0;
  const W = vec ? 4 : 1;
  const colsPerBlock = 64 * W;
  const colBlocks = Math.ceil(inner / colsPerBlock);
  const want = tune.blocks || 1024;
  // Up to COLRED_ONE_PASS elements the rows are not split: one launch, whose workgroups
  // each sum whole columns, costs less than a second kernel combining chunks (config 1's
  // bias gradients over 128 rows).
  let splits = !tune.blocks && outer * n * inner <= COLRED_ONE_PASS ? 1
    : Math.max(1, Math.min(Math.ceil(want / Math.max(1, colBlocks * outer)), Math.ceil(n / 32)));
  const chunk = Math.ceil(n / splits);
  splits = Math.ceil(n / chunk);
  const T = vec ? 'tcmi::f4' : 'float';
  const zero = vec ? `tcmi::f4{${init}, ${init}, ${init}, ${init}}` : init;
  const combV = vec
    ? (a, b) => `tcmi::f4{${comb}(${a}[0], ${b}[0]), ${comb}(${a}[1], ${b}[1]), ${comb}(${a}[2], ${b}[2]), ${comb}(${a}[3], ${b}[3])}`
    : (a, b) => `${comb}(${a}, ${b})`;
  const ld = (ptr, idx) => (vec ? `reinterpret_cast<const tcmi::f4*>(${ptr})[(${idx}) >> 2]` : `(${ptr})[${idx}]`);
  const st = (ptr, idx, v) => (vec ? `reinterpret_cast<tcmi::f4*>(${ptr})[(${idx}) >> 2] = ${v};` : `(${ptr})[${idx}] = ${v};`);
  // A producer formed in place (`producer`: { body, output }, an elementwise body over the
  // launch's operands A.in[0..], its value of the reduced operand's shape): each element
  // the reduction reads is the body at that element's flat index g0 (+ its lane in a
  // 4-column group), through the same emitter and op helpers as an elementwise kernel, so
  // the same bits as reading the producer's output. Operands of the full size load a
  // 4-column group at once; others (broadcast rows or columns) load at their index map.
  // The launch's parameter words are these five, then the producer's gather maps: the
  // emitter starts on them, so its word limit and the offsets it records count them.
  const pparams = [outer, n, inner, splits, chunk];
  let formed = '';
  if (producer) {
    if (outer * n * inner >= 2 ** 32) throw new Error('column reduction with a producer: operand past 2^32 elements');
    const lines = [];
    const full = new Set();
    const em = new Emitter(producer.body, pparams, {
      load(k, ctx, ls) {
        if (ctx.root && vec) {
          if (!full.has(k)) { ls.push(`const tcmi::f4 F${k} = reinterpret_cast<const tcmi::f4*>(A.in[${k}])[g0 >> 2];`); full.add(k); }
          return `F${k}[${ctx.lane}]`;
        }
        const v = `L${ls.length}_${k}`;
        ls.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
        return v;
      },
    });
    const outs = [];
    for (let l = 0; l < W; l++) {
      outs.push(em.value(producer.output, { key: `e${l}`, idx: l ? `(g0 + ${l}u)` : 'g0', root: true, lane: l, limit: outer * n * inner }, lines));
    }
    formed = [`      const uint32_t g0 = (o * n + k) * inner + j;`, ...lines.map((x) => `      ${x}`),
      `      const ${T} v = ${vec ? `tcmi::f4{${outs.join(', ')}}` : outs[0]};`].join('\n');
  }
  // A chain applied to each sum before the store (`chain`: { body, output, sumAt }, the
  // body of the sum's one reader, its inputs at the positions sumAt reading the sum and
  // every other input loaded at the output's flat index): the launch is that reader's, its
  // operands the chain's own with the sum's operand at sumAt[0].
  const xin = chain ? chain.sumAt[0] : 0;
  if (chain && producer) throw new Error('a column sum folded into its reader forms no producer');
  // Each lane's chain in a scope of its own (an emitter per lane: the sum it reads is
  // that lane's); the lowering folds only chains of elementwise ops of one size, which
  // read every operand, the sum included, at the element they store.
  const store = (idx, v) => {
    if (!chain) return st('A.out', idx, v);
    const parts = [];
    for (let l = 0; l < W; l++) {
      const lines = [];
      const at = l ? `(${idx} + ${l}u)` : `(${idx})`;
      const em = new Emitter(chain.body, pparams, {
        load(k, ctx, ls) {
          if (ctx.idx !== at) throw new Error('a column sum folded into its reader: an operand read at another element');
          if (chain.sumAt.includes(k)) return vec ? `${v}[${l}]` : v;
          const x = `C${ls.length}_${k}`;
          ls.push(`const float ${x} = A.in[${k}][${ctx.idx}];`);
          return x;
        },
      });
      const out = em.value(chain.output, { key: `c${l}`, idx: at, root: true, lane: l, limit: outer * inner }, lines);
      parts.push(`{ ${lines.join(' ')} y${l} = ${out}; }`);
    }
    const ys = Array.from({ length: W }, (_, l) => `y${l}`);
    return `{ float ${ys.join(', ')}; ${parts.join(' ')} ${st('A.out', idx, vec ? `tcmi::f4{${ys.join(', ')}}` : 'y0')} }`;
  };
  const first = `extern "C" __global__ void __launch_bounds__(256) __KERNEL__(const TcmiArgs A) {
  __shared__ ${T} part[4][64];
  const uint32_t n = ${n}u, inner = ${inner}u, splits = ${splits}u, chunk = ${chunk}u;
  const uint32_t lane = threadIdx.x & 63u, g = threadIdx.x >> 6;
  const uint32_t j = blockIdx.x * ${colsPerBlock}u + lane * ${W}u;
  const uint32_t s = blockIdx.y, o = blockIdx.z;
  const uint32_t k0 = s * chunk;
  const uint32_t k1 = min(n, k0 + chunk);
  ${T} acc = ${zero};
  if (j < inner) {
${producer ? '' : `    const float* __restrict__ x = A.in[${xin}] + (size_t)o * n * inner;\n`}#pragma unroll 8
    for (uint32_t k = k0 + g; k < k1; k += 4u) {
${producer ? formed : `      const ${T} v = ${ld('x', '(size_t)k * inner + j')};`}
      acc = ${combV('acc', 'v')};
    }
  }
  part[g][lane] = acc;
  __syncthreads();
  if (g == 0 && j < inner) {
    ${T} r = part[0][lane];
    r = ${combV('r', 'part[1][lane]')};
    r = ${combV('r', 'part[2][lane]')};
    r = ${combV('r', 'part[3][lane]')};
    if (splits == 1u) { ${store('(size_t)o * inner + j', 'r')} }
    else { ${st('A.ws', '((size_t)o * splits + s) * inner + j', 'r')} }
  }
}
`;
  const k1 = kernelText('colred', first);
  const launches = [{ name: k1.name, source: k1.source, grid: [colBlocks, splits, outer], block: [256, 1, 1], lds: 0 }];
  if (splits > 1) {
    // 16 column groups x 16 split groups per workgroup: every CU of a good share of
    // the chip reads a slice of the partials, 16 split rows per thread at most.
    const groupsPerBlock = 16;
    const second = `extern "C" __global__ void __launch_bounds__(256) __KERNEL__(const TcmiArgs A) {
  __shared__ ${T} part[16][${groupsPerBlock}];
  const uint32_t inner = ${inner}u, splits = ${splits}u;
  const uint32_t c = threadIdx.x & ${groupsPerBlock - 1}u, g = threadIdx.x / ${groupsPerBlock}u;
  const uint32_t j = (blockIdx.x * ${groupsPerBlock}u + c) * ${W}u;
  const uint32_t o = blockIdx.y;
  ${T} acc = ${zero};
  if (j < inner) {
    const float* __restrict__ w = A.ws + (size_t)o * splits * inner;
#pragma unroll 8
    for (uint32_t s = g; s < splits; s += 16u) {
      const ${T} v = ${ld('w', '(size_t)s * inner + j')};
      acc = ${combV('acc', 'v')};
    }
  }
  part[g][c] = acc;
  __syncthreads();
  if (g == 0 && j < inner) {
    ${T} r = part[0][c];
#pragma unroll
    for (int q = 1; q < 16; ++q) r = ${combV('r', 'part[q][c]')};
    ${store('(size_t)o * inner + j', 'r')}
  }
}
`;
    const k2 = kernelText('colfin', second);
    launches.push({ name: k2.name, source: k2.source, grid: [Math.ceil(inner / (W * groupsPerBlock)), outer, 1], block: [256, 1, 1], lds: 0 });
  }
  return { launches, params: Uint32Array.from(pparams), workspace: splits > 1 ? outer * splits * inner * 4 : 0 };
}

// ---- matmul with epilogue ----------------------------------------------------------------

/**
 * Tiling of a matmul: MFMA tiles per wavefront (T: the workgroup owns 32T x 32T
 * of the output), K chunks (split-K) and the LDS slice depth (bk). Rules, from
 * a sweep of every (T, bk, chunks) on the MI355X over the configs' shapes:
 *   - T = 4 when M, N >= 128 and that still gives the 256 CUs a workgroup each;
 *     T = 2 when that gives every CU a workgroup (or when K is long, see below);
 *     T = 1 otherwise;
 *   - K is split only when it is long (>= 2048) and the output leaves fewer than
 *     two workgroups per CU: into chunks of >= 256 (at most 32) so that about
 *     1024 workgroups run — a few per CU hide each other's memory latency; a
 *     short K is never split (the partial-sum traffic costs more than it saves);
 *   - bk = 64 for T = 1, 32 for T = 2, 16 for T = 4 (the deeper slice feeds the
 *     small tiles more work per round trip to memory).
 * Every choice depends on (batch, M, N, K) alone, not on the operands' layouts,
 * so a matmul gives the same bits (the split fixes the order of the K sum)
 * whether its operands are materialised or read through views.
 */
function gemmTiling(batch, M, N, K, tuning, peers) {
  // A tuning's `byShape` entry for this product ('batch x M x N x K') overrides it.
  const t = Object.assign({}, tuning || {}, ((tuning || {}).byShape || {})[`${batch}x${M}x${N}x${K}`] || {});
  // Products of this shape that may share one dispatch (1 if unknown): they share the
  // chip, so the K split aims at its workgroup count over all of them.
  const P = peers || 1;
  // Tile counts of 32T x 32T: the T and split rules are stated on them.
  const blocks = (T) => batch * Math.ceil(M / (32 * T)) * Math.ceil(N / (32 * T));
  const longK = K >= 2048;
  let T;
  if (t.tile) T = t.tile;
  else if (M >= 128 && N >= 128 && blocks(4) >= 256) T = 4;
  else if (M >= 64 && N >= 64 && (blocks(2) >= 256 || longK)) T = 2;
  else T = 1;
  // A tile that would pad the product by more than an eighth drops to 32 x 32, which
  // divides any multiple of 32 (config 5's vocabulary of 96: 64-wide tiles did a third
  // more MFMA work). An on-device sweep of its three such products (the logits, the
  // output and embedding weight gradients): 32 x 32 tiles 18-31 % faster than 64-wide
  // tiles or 48- and 96-wide ones, the products' bits unchanged.
  const padded = (T2) => {
    const bn = 16 * (T2 >= 2 && N >= 64 * T2 ? 4 : 2) * T2;
    return Math.ceil(M / (32 * T2)) * 32 * T2 * Math.ceil(N / bn) * bn;
  };
  const unpad = !t.tile && !t.waves && t.pad !== false && T > 1 && padded(T) * 8 > 9 * M * N;
  if (unpad) T = 1;
  let chunks = 1;
  if (t.splitk !== undefined) chunks = t.splitk;
  else if (longK && blocks(T) < 512) chunks = Math.max(1, Math.min(Math.ceil(1024 / (blocks(T) * P)), Math.floor(K / 256), 32));
  let chunkK = Math.ceil(Math.ceil(K / chunks) / 16) * 16;
  chunks = Math.ceil(K / chunkK);
  // Wavefronts along N: 4 (a 32T x 64T tile, 512 threads) wherever N fills the wider
  // tile and T >= 2, with 32-deep slices; and the MFMA phase at raised wave priority.
  // An on-device sweep of every config-4 and config-5 product: 5-15 % faster than 2
  // wavefronts wherever N >= 64T, slower where N is narrower.
  const wn = t.waves || (T >= 2 && N >= 64 * T ? 4 : 2);
  // K groups inside a workgroup: where 32 x 32 tiles leave at most two workgroups per CU
  // and K is not split across workgroups, 2 or 4 groups of four wavefronts each sum a
  // part of K (their sums added in order in LDS), so more wavefronts keep loads in
  // flight and the matrix cores fed on each CU.
  // Unpadded products (above) take two groups up to 1024 tiles (the logits: 7.2 -> 6.7 us).
  const kw = t.kw || (T === 1 && chunks === 1 && blocks(1) <= 512 && K >= 256 ? (K >= 512 ? 4 : 2)
    : unpad && chunks === 1 && blocks(1) <= 1024 && K >= 256 ? 2 : 1);
  const bk = t.bk || (kw > 1 ? 32 : wn === 4 ? 32 : T === 1 ? 64 : T === 2 ? 32 : 16);
  const pf = t.pf || 2;
  const prio = t.prio !== undefined ? !!t.prio : true;
  // Per-wavefront accumulator tiles along M (tm) and N (tn): T x T unless tuned.
  const tm = t.tm || T, tn = t.tn || T;
  const wide = batch * Math.ceil(M / (32 * tm)) * Math.ceil(N / (16 * wn * tn));
  return { T, tm, tn, chunks, chunkK, bk, pf, wn, prio, kw, blocks: wide * chunks };
}

/**
 * Floats of the LDS pool (tcmi::lds_pool) tcmi_gemm.h's gemm_f32 takes for tiling `tl`
 * and operand load modes (0 row-major, 1 transposed, 2 strided): both staged slices of
 * each K group's A and B tiles, rows padded by 4, and the K groups' hand-over area.
 */
function gemmPoolFloats(tl, amode, bmode) {
  const BM = 32 * tl.tm, BN = 16 * tl.wn * tl.tn, BK = tl.bk;
  const aK = amode === 1, bN = bmode === 1;
  const aTile = (aK ? BK : BM) * (aK ? BM + 4 : BK + 4);
  const bTile = (bN ? BN : BK) * (bN ? BK + 4 : BN + 4);
  const threads = 128 * tl.wn;
  return tl.kw * 2 * (aTile + bTile) + (tl.kw > 1 ? (tl.kw - 1) * threads * tl.tm * tl.tn * 4 : 0);
}

// The op a view applies to every element it loads (view.op: 'relu'), as the view struct's
// OP member (tcmi_gemm.h vop); nothing for a plain view, whose text stays as it was.
const LOAD_OPS = { relu: 1 };
function loadOp(v) {
  if (!v.op) return '';
  if (!LOAD_OPS[v.op]) throw new Error(`no operand load op '${v.op}'`);
  return `\n  static constexpr int OP = ${LOAD_OPS[v.op]};   // ${v.op} on load`;
}

/**
 * Index `x` over mixed-radix factors [[extent, stride], ...] (outer to inner): the
 * expression Σ_f ((x / inner_f) % extent_f) · stride_f, the outermost factor without the
 * modulo (the kernels form offsets of in-range indices only); extent-1 and stride-0
 * factors add nothing.
 */
function factorTerms(x, fs) {
  const terms = [];
  let inner = 1;
  for (let d = fs.length - 1; d >= 0; d--) {
    const [e, st] = fs[d];
    if (e > 1 && st !== 0) {
      const idx = inner === 1 ? x : `(${x} / ${inner}u)`;
      terms.push(`(size_t)(${d === 0 ? idx : `${idx} % ${e}u`}) * ${st}u`);
    }
    inner *= e;
  }
  return terms.length ? terms.join(' + ') : '0';
}

/**
 * The view struct of a matmul operand (tcmi_gemm.h): element (b, r, c) at
 * batch(b) + r·SR + c·SC of its buffer, and the load mode its layout allows.
 * `view` = { batch: [[extent, stride], ...], sr, sc } (null: dense row-major
 * [batch, R, C]); R, C the operand's extents. A mapped view ({ batch, r, c }: the row
 * and column indices over mixed-radix factors [[extent, stride], ...], as a chain of
 * transposes and reshapes lays them out) places the element at batch(b) + row(r) +
 * col(c) instead, and takes 128-bit loads along c (or r) where c's (r's) innermost
 * factor is contiguous, holds whole groups of 4, and every other stride is a multiple
 * of 4 (so each load is aligned and inside one group).
 */
function operandView(name, view, batchDims, R, C) {
  const v = view || { batch: batchDims.map((e, d) => [e, R * C * size(batchDims.slice(d + 1))]), sr: C, sc: 1 };
  const strides = v.batch.map((x) => x[1]);
  const batchTerms = factorTerms('b', v.batch);
  const batchLimit = v.batch.reduce((t, [e, st]) => t + (e - 1) * st, 0);
  if (v.r || v.c) {
    const rf = v.r || [[R, v.sr]], cf = v.c || [[C, v.sc]];
    const all4 = (fs) => fs.every(([e, st]) => e === 1 || st % 4 === 0) && strides.every((st) => st % 4 === 0);
    const along = (fs, other, ext) => {
      const [e, st] = fs[fs.length - 1];
      return st === 1 && e % 4 === 0 && ext % 4 === 0 && all4(fs.slice(0, -1)) && all4(other);
    };
    const mode = along(cf, rf, C) ? 0 : along(rf, cf, R) ? 1 : 2;
    const text = `struct ${name} {
  static constexpr bool MAPPED = true;${loadOp(v)}
  static __device__ __forceinline__ size_t batch(uint32_t b) { return ${batchTerms}; }
  static __device__ __forceinline__ size_t row(uint32_t r) { return ${factorTerms('r', rf)}; }
  static __device__ __forceinline__ size_t col(uint32_t c) { return ${factorTerms('c', cf)}; }
};
`;
    const span = (fs) => fs.reduce((t, [e, st]) => t + (e - 1) * st, 0);
    return { text, mode, limit: 1 + batchLimit + span(rf) + span(cf), mapped: true };
  }
  const others4 = (x) => strides.every((s) => s % 4 === 0) && x % 4 === 0;
  let mode = 2;
  if (v.sc === 1 && C % 4 === 0 && others4(v.sr)) mode = 0;
  else if (v.sr === 1 && R % 4 === 0 && others4(v.sc)) mode = 1;
  const text = `struct ${name} {
  static constexpr size_t SR = ${v.sr}, SC = ${v.sc};${loadOp(v)}
  static __device__ __forceinline__ size_t batch(uint32_t b) { return ${batchTerms}; }
};
`;
  // One past the largest element offset the kernel can address.
  const limit = 1 + batchLimit + (R - 1) * v.sr + (C - 1) * v.sc;
  return { text, mode, limit };
}

/**
 * A matmul-epilogue body (or a plain matmul): the body's matmul node is the
 * root, every other body op runs on its accumulator at the store. Epilogue
 * operands are read at the output's flat index (or through their gathers).
 * `views` ({ a, b }, optional): the matmul operands are read in place through
 * these strided views of other buffers (a transposed operand not materialised);
 * `sizes` ({ a, b }) are those buffers' element counts, against which every
 * view is proved in bounds.
 */
function gemmKernel(b, output, opts) {
  const o = opts || {};
  checkOperands(b);
  const root = b.nodes.find((n) => n.op === 'matmul');
  const ia = Number(b.nodes[root.inputs[0]].attrs.name.slice(1));
  const ib = Number(b.nodes[root.inputs[1]].attrs.name.slice(1));
  const as = b.nodes[root.inputs[0]].shape, bs = b.nodes[root.inputs[1]].shape;
  const batchDims = as.slice(0, -2);
  const batch = size(batchDims), M = as[as.length - 2], K = as[as.length - 1], N = bs[bs.length - 1];
  if (batch * M * N >= 2 ** 31 || batch * M * K >= 2 ** 31 || batch * K * N >= 2 ** 31) {
    throw new Error('matmul exceeds the 32-bit index space');
  }
  const views = o.views || {};
  const params = [batch, M, K, N];
  // Sabotage (the reference's 'epilogue-before-bias', codegen-fused.js:228-243): the
  // activation sees the bare sum and the bias is added after it.
  let biasAdd = null;
  if (o.sabotage === 'epilogue-before-bias') {
    const add = b.nodes.find((n) => n.op === 'add' && n.inputs.includes(root.id) && !n.inputs.every((i) => i === root.id));
    if (add && add.id !== output) biasAdd = add;
  }
  const tl = gemmTiling(batch, M, N, K, o.tuning, o.peers);
  const total = batch * M * N;
  // A group formed with recomputation may read its matmul through a broadcast or
  // transpose, at another element's index than the one being stored. The product
  // is then formed in the workspace first (the split-K path, with one chunk if the
  // shape asks for none) and the second kernel reads element j's sum there, the
  // chunks added in order: the bits the reduction forms for j itself.
  let gathered = false;
  const em = new Emitter(b, params, {
    special: (id, ctx, lines) => {
      if (biasAdd && id === biasAdd.id) return 'acc';
      if (id !== root.id) return undefined;
      if (ctx.root) return 'acc';
      gathered = true;
      const v = em.fresh('m');
      lines.push(`const float ${v} = tcmi::gemm_product_at(A, ${ctx.idx}, ${total}u, ${tl.chunks}u);`);
      return v;
    },
    load(k, ctx, lines) {
      const v = `L${lines.length}_${k}`;
      lines.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
      return v;
    },
  });
  const lines = [];
  const rootCtx = { key: 'i', idx: 'i', root: true, limit: total };
  let out = em.value(output, rootCtx, lines);
  if (biasAdd) {
    const other = biasAdd.inputs.find((i) => i !== root.id);
    const ov = em.value(other, rootCtx, lines);
    const t = em.fresh('v');
    lines.push(`const float ${t} = tcmi::op_add(${out}, ${ov});`);
    out = t;
  }
  const av = operandView('__KERNEL___av', views.a, batchDims, M, K);
  const bv = operandView('__KERNEL___bv', views.b, bs.slice(0, -2), K, N);
  const split = tl.chunks > 1 || gathered;
  const sizes = o.sizes || {};
  const need = { a: sizes.a !== undefined ? sizes.a : batch * M * K, b: sizes.b !== undefined ? sizes.b : batch * K * N };
  if (av.limit > need.a || bv.limit > need.b) throw new Error(`matmul operand view out of bounds (${av.limit}/${need.a}, ${bv.limit}/${need.b})`);
  const epi = `struct __KERNEL___epi {
  template <class Args>
  __device__ __forceinline__ float operator()(const Args& A, uint32_t i, float acc) const {
${indent(lines, '    ')}
    return ${out};
  }
};
`;
  const threads = 128 * tl.wn * tl.kw;
  const variant = tl.kw > 1 ? `, ${tl.wn}, ${tl.prio}, ${tl.kw}` : tl.wn === 2 && !tl.prio ? '' : `, ${tl.wn}, ${tl.prio}`;
  // A launch split along K places the tiles of each chunk on one XCD (tcmi::xcd_grouped),
  // so they share its L2 for the A and B panels they all read.
  const grouped = tl.chunks > 1;
  // The tile's place passed explicitly: a ragged batch runs this text with blockIdx
  // standing for the member's own place (raggedKernel).
  const place = grouped ? ', wg.z, wg.x, wg.y' : ', blockIdx.z, blockIdx.x, blockIdx.y';
  const main = `extern "C" __global__ void __launch_bounds__(${threads}) __KERNEL__(const TcmiArgs A) {
${grouped ? `  ${XCD_GROUPED}
` : ''}  tcmi::gemm_f32<${tl.tm}, ${tl.tn}, ${tl.bk}, ${tl.pf}, ${av.mode}, ${bv.mode}, ${split}, __KERNEL___av, __KERNEL___bv, __KERNEL___epi${variant}>(A, A.in[${ia}], A.in[${ib}],
      ${batch}u, ${M}u, ${K}u, ${N}u, ${tl.chunks}u, ${tl.chunkK}u${place});
}
`;
  const text = `#include "tcmi_gemm.h"\n${av.text}${bv.text}${epi}${main}`;
  const k = kernelText('mm', text);
  const kernels = [{ name: k.name, source: k.source, grid: [Math.ceil(N / (16 * tl.wn * tl.tn)), Math.ceil(M / (32 * tl.tm)), batch * tl.chunks],
    block: [threads, 1, 1], lds: 0, pool: gemmPoolFloats(tl, av.mode, bv.mode) }];
  let workspace = 0;
  if (split) {
    // The reduction kernel shares the epilogue struct of the partial kernel's text.
    const vecOut = N % 4 === 0;
    const red = `#include "tcmi_gemm.h"\n${epi}extern "C" __global__ void __launch_bounds__(256) __KERNEL___red(const TcmiArgs A) {
  tcmi::gemm_splitk_reduce<${vecOut}, __KERNEL___epi>(A, ${total}u, ${tl.chunks}u);
}
`;
    const rk = kernelText('mmred', red);
    const rname = `${rk.name}_red`;
    kernels.push({ name: rname, source: rk.source, grid: [Math.max(1, Math.min(Math.ceil(total / (vecOut ? 4 : 1) / 256), 2048)), 1, 1], block: [256, 1, 1], lds: 0 });
    workspace = tl.chunks * total * 4;
  }
  return { name: k.name, source: k.source, kernels, params: Uint32Array.from(params), grid: kernels[0].grid, block: [threads, 1, 1],
    lds: 0, workspace, flops: 2 * batch * M * N * K, tiling: tl, modes: [av.mode, bv.mode] };
}

// ---- attention (the fusion extension of fusion/attention.js) ------------------------

/**
 * A fused attention node's body: a0 = Q [batch, TQ, DH], a1 = Kt [batch, DH, TK],
 * scores = matmul(a0, a1), the score body (elementwise ops and last-axis
 * reductions over the scores and further operands), then matmul(P, V) with V the
 * last operand — the body's output. One workgroup per (16·W query rows, batch
 * index), W = min(8, ceil(TQ / 16)) wavefronts, over tcmi_attention.h: the body below runs on the score registers, its
 * reductions across each row's four lanes. `views` ({ q, k, v }) read those
 * operands in place through strided views of other buffers (`sizes`: their
 * element counts, against which every view is proved in bounds).
 */
function attentionKernel(b, output, opts) {
  const o = opts || {};
  checkOperands(b);
  const m2 = b.nodes[output];
  const m1 = b.nodes.find((n) => n.op === 'matmul' && n.id !== output);
  if (m2.op !== 'matmul' || !m1) throw new Error('attention body: expected matmul(body(matmul(Q, Kt)), V)');
  const operandOf = (id) => {
    const n = b.nodes[id];
    if (n.op !== 'input') throw new Error('attention body: the products\' operands must be body inputs');
    return Number(n.attrs.name.slice(1));
  };
  const iq = operandOf(m1.inputs[0]), ik = operandOf(m1.inputs[1]), iv = operandOf(m2.inputs[1]);
  const qs = b.nodes[m1.inputs[0]].shape, ks = b.nodes[m1.inputs[1]].shape, vs = b.nodes[m2.inputs[1]].shape;
  const r = qs.length;
  const batchDims = qs.slice(0, r - 2);
  const batch = size(batchDims), TQ = qs[r - 2], DH = qs[r - 1], TK = ks[r - 1], DV = vs[r - 1];
  if (batch * TQ * TK >= 2 ** 31 || batch * TQ * DV >= 2 ** 31) throw new Error('attention exceeds the 32-bit index space');
  if (batch > 65535) throw new Error(`attention batch ${batch} exceeds the grid`);
  const sOut = m2.inputs[0];
  const reductions = b.nodes.filter((n) => isReduce(n) && n.id > m1.id && n.id < m2.id);
  for (const rd of reductions) {
    const src = b.nodes[rd.inputs[0]].shape;
    if (rd.attrs.axis !== src.length - 1 || size(src) !== batch * TQ * TK) throw new Error('attention body: reductions must be over the keys');
  }
  const R = batch * TQ, C = TK;
  const params = [batch, TQ, DH, TK, DV];
  const rowTier = (id) => size(b.nodes[id].shape) === R && size(b.nodes[id].shape) !== R * C;
  if (size(b.nodes[sOut].shape) !== R * C) throw new Error('attention body: P must cover every score');

  const reduced = new Map();
  const rowLines = [];
  const caches = new Map();
  const cacheFill = [];
  const NT = Math.ceil(TK / 16);
  let em;
  const ROW = { key: 'r', idx: 'r', root: false, row: true, limit: R };
  const elemCtx = () => ({ key: 'e', idx: 'e', root: true, limit: R * C });
  em = new Emitter(b, params, {
    special(id, ctx) {
      if (id === m1.id) {
        if (ctx.row || !ctx.root) throw new Error('attention body: the scores are read at their own index only');
        return 'sacc[jt][l]';
      }
      if (reduced.has(id)) return reduced.get(id);
      const n = b.nodes[id];
      if (!ctx.row && rowTier(id) && n.op !== 'input' && n.op !== 'const') return em.value(id, ROW, rowLines);
      if (n.op === 'broadcast' && !ctx.row && rowTier(n.inputs[0])) {
        const src = b.nodes[n.inputs[0]];
        if (src.op !== 'input' && src.op !== 'const') return em.value(src.id, ROW, rowLines);
      }
      return undefined;
    },
    load(k, ctx, lines) {
      if (ctx.key.startsWith('e')) {
        // An operand read at a score's index (directly or through gathers): loaded once,
        // for every score of the lane, into registers that every phase reads.
        const ck = `${k}|${ctx.idx}`;
        if (!caches.has(ck)) {
          const c = `C${caches.size}`;
          caches.set(ck, c);
          cacheFill.push(`float ${c}[${NT}][4];`, `#pragma unroll
for (int jt = 0; jt < ${NT}; ++jt) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t c = 16u * jt + 4u * q + l;
    const uint32_t e = rowBase + c;
    ${c}[jt][l] = rowOk && c < ${TK}u ? A.in[${k}][${ctx.idx}] : 0.f;
  }
}`);
        }
        return `${caches.get(ck)}[jt][l]`;
      }
      const v = `L${lines.length}_${k}`;
      lines.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
      return v;
    },
  });
  // One pass over this lane's scores of its row: `e` the flat index in [batch·TQ, TK].
  const loop = (bodyLines) => `#pragma unroll
for (int jt = 0; jt < ${Math.ceil(TK / 16)}; ++jt) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t c = 16u * jt + 4u * q + l;
    if (rowOk && c < ${TK}u) {
      const uint32_t e = rowBase + c;
${indent(bodyLines, '      ')}
    }
  }
}`;
  const phases = [];
  reductions.forEach((rd, k) => {
    for (const key of Array.from(em.memo.keys())) if (key.startsWith('e')) em.memo.delete(key);
    const rowBefore = rowLines.length;
    const inner = [];
    const v = em.value(rd.inputs[0], elemCtx(), inner);
    const isMax = rd.op === 'max';
    const pre = rowLines.splice(rowBefore);
    phases.push(...pre,
      `float acc${k} = ${isMax ? '(-TCMI_INF)' : '0.f'};`,
      loop(inner.concat([`acc${k} = tcmi::red_${isMax ? 'max' : 'sum'}(acc${k}, ${v});`])),
      `const float red${k} = tcmi::quad16_reduce<${isMax}>(acc${k});`);
    reduced.set(rd.id, `red${k}`);
  });
  for (const key of Array.from(em.memo.keys())) if (key.startsWith('e')) em.memo.delete(key);
  const rowBefore = rowLines.length;
  const inner = [];
  const pv = em.value(sOut, elemCtx(), inner);
  const pre = rowLines.splice(rowBefore);
  const pLoop = `#pragma unroll
for (int jt = 0; jt < ${Math.ceil(TK / 16)}; ++jt) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t c = 16u * jt + 4u * q + l;
    float pe = 0.f;
    if (rowOk && c < ${TK}u) {
      const uint32_t e = rowBase + c;
${indent(inner, '      ')}
      pe = ${pv};
    }
    p[jt][l] = pe;
  }
}`;
  const views = o.views || {};
  const sizes = o.sizes || {};
  const qv = operandView('__KERNEL___qv', views.q, batchDims, TQ, DH);
  const kv = operandView('__KERNEL___kv', views.k, batchDims, DH, TK);
  const vv = operandView('__KERNEL___vv', views.v, batchDims, TK, DV);
  // The attention kernel addresses its operands by SR and SC and loads them as they are:
  // a mapped view or a load op never reaches it.
  if (qv.mapped || kv.mapped || vv.mapped || [views.q, views.k, views.v].some((v) => v && v.op)) {
    throw new Error('attention operand read through a mapped view or a load op');
  }
  const need = (slot, dense) => (sizes[slot] !== undefined ? sizes[slot] : dense);
  if (qv.limit > need('q', batch * TQ * DH) || kv.limit > need('k', batch * DH * TK) || vv.limit > need('v', batch * TK * DV)) {
    throw new Error('attention operand view out of bounds');
  }
  // Wavefronts per workgroup: one per 16 query rows, up to 8 (128 rows share one K and V tile).
  const WAVES = (o.tuning && o.tuning.waves) || Math.min(8, Math.ceil(TQ / 16));
  const THREADS = 64 * WAVES;
  const text = `#include "tcmi_attention.h"
${qv.text}${kv.text}${vv.text}extern "C" __global__ void __launch_bounds__(${THREADS}) __KERNEL__(const TcmiArgs A) {
  using G = tcmi::AttnTiles<${TK}, ${DH}, ${DV}>;
  __shared__ __attribute__((aligned(16))) float Ks[G::ROWS * G::KS];
  __shared__ __attribute__((aligned(16))) float Vs[G::ROWS * G::VS];
  const uint32_t b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t16 = lane & 15, q = lane >> 4;
  const uint32_t row = blockIdx.x * ${16 * WAVES}u + wave * 16u + t16;   // this lane's query row
  tcmi::attn_zero_padding<${TK}, ${DH}, ${DV}, ${THREADS}>(Ks, Vs);
  // Every global load of the K and V tiles issued at once; V lands in LDS after the scores.
  using Kst = tcmi::AttnStage<${TK}, ${DH}, G::KS, ${kv.mode}, true, __KERNEL___kv, ${THREADS}>;
  using Vst = tcmi::AttnStage<${TK}, ${DV}, G::VS, ${vv.mode}, false, __KERNEL___vv, ${THREADS}>;
  tcmi::f4 kr[Kst::PER], vr[Vst::PER];
  Kst::load(kr, A.in[${ik}], b);
  Vst::load(vr, A.in[${iv}], b);
  tcmi::f4 qf[G::DH16];
  tcmi::attn_q<${TQ}, ${DH}, G::DH16, ${qv.mode}, __KERNEL___qv>(qf, A.in[${iq}], b, row, q);
  const bool rowOk = row < ${TQ}u;
  const uint32_t r = b * ${TQ}u + (rowOk ? row : 0u);   // the score row (rows past TQ compute nothing)
  const uint32_t rowBase = r * ${TK}u;
${indent(cacheFill, '  ')}
  Kst::store(kr, Ks);
  __syncthreads();
  tcmi::f4 sacc[G::NT];
  tcmi::attn_scores<G::NT, G::DH16, G::KS>(sacc, qf, Ks, t16, q);
  Vst::store(vr, Vs);
${indent(phases, '  ')}
  tcmi::f4 p[${NT}];
${indent(pre.concat([pLoop]), '  ')}
  __syncthreads();
  tcmi::f4 oacc[G::DV16];
  tcmi::attn_pv<G::NT, G::DV16, G::VS>(oacc, p, Vs, t16, q);
  tcmi::attn_store<${TQ}, ${DV}, G::DV16>(A.out, oacc, b, row, q);
}
`;
  const k = kernelText('attn', text);
  const lds = 4 * (NT * 16) * (Math.ceil(DH / 16) * 16 + 4 + Math.ceil(DV / 16) * 16 + 4);
  return { name: k.name, source: k.source, params: Uint32Array.from(params), grid: [Math.ceil(TQ / (16 * WAVES)), batch, 1],
    block: [THREADS, 1, 1], lds: 0, ldsStatic: lds, workspace: 0, flops: 2 * batch * TQ * TK * (DH + DV),
    modes: [qv.mode, kv.mode, vv.mode] };
}

// ---- the attention gradient (fusion/attention.js, fuseAttentionTraining) -------------

const GRAD_PARTS = ['dq', 'dk', 'dv'];

/**
 * The parts of an attention-grad body (its inputs a0 Q, a1 K, a2 V, a3 dO, then score
 * operands): the scores S = matmul(a0, transpose(a1)), dP = matmul(a3, transpose(a2)),
 * and the three products dQ = matmul(dS, a1), dK = matmul(transpose(dS), a0) and
 * dV = matmul(transpose(P), a3), as fuseAttentionTraining builds it.
 */
function gradBodyParts(b) {
  const N = b.nodes;
  const inputAt = (id, k) => N[id].op === 'input' && N[id].attrs.name === `a${k}`;
  const tOf = (id, k) => N[id].op === 'transpose' && inputAt(N[id].inputs[0], k);
  const mm = N.filter((n) => n.op === 'matmul');
  const one = (pred, what) => {
    const f = mm.filter(pred);
    if (f.length !== 1) throw new Error(`attention-grad body: expected one ${what}`);
    return f[0];
  };
  const S = one((n) => inputAt(n.inputs[0], 0) && tOf(n.inputs[1], 1), 'score product');
  const dP = one((n) => inputAt(n.inputs[0], 3) && tOf(n.inputs[1], 2), 'dP product');
  const dQ = one((n) => inputAt(n.inputs[1], 1) && !inputAt(n.inputs[0], 0), 'dQ product');
  const dK = one((n) => inputAt(n.inputs[1], 0) && N[n.inputs[0]].op === 'transpose', 'dK product');
  const dV = one((n) => inputAt(n.inputs[1], 3) && N[n.inputs[0]].op === 'transpose', 'dV product');
  const ds = dQ.inputs[0];
  if (N[dK.inputs[0]].inputs[0] !== ds) throw new Error('attention-grad body: dK must read the dQ product\'s dS');
  return { S, dP, dQ, dK, dV, ds, p: N[dV.inputs[0]].inputs[0] };
}

/** The part ('dq' | 'dk' | 'dv') node `output` of an attention-grad body is. */
function gradPart(b, output) {
  const x = gradBodyParts(b);
  const part = output === x.dQ.id ? 'dq' : output === x.dK.id ? 'dk' : output === x.dV.id ? 'dv' : null;
  if (!part) throw new Error('attention-grad body: the output must be one of its three products');
  return part;
}

/**
 * The text of a kernel forming `parts` of an attention-grad body (tcmi_attention.h's
 * gradient): one workgroup per batch index, W = ceil(TQ / 16) wavefronts. With `joint`,
 * one launch writes all three, member 0 (dQ), 1 (dK) and 2 (dV) of a batched launch's
 * argument block; otherwise the one part goes to A.out. Every part is formed by the same
 * code in either form (the body's values below, then the part's product), so a part's
 * bits do not depend on which others the kernel forms.
 */
function attnGradText(b, parts, opts) {
  const o = opts || {};
  checkOperands(b);
  const x = gradBodyParts(b);
  const N = b.nodes;
  const shapeOf = (k) => N.find((n) => n.op === 'input' && n.attrs.name === `a${k}`).shape;
  const qs = shapeOf(0), ks = shapeOf(1), vs = shapeOf(2), os = shapeOf(3);
  const r = qs.length;
  const batchDims = qs.slice(0, r - 2);
  const batch = size(batchDims), TQ = qs[r - 2], DH = qs[r - 1], TK = ks[r - 2], DV = vs[r - 1];
  if (ks[r - 1] !== DH || vs[r - 2] !== TK || os[r - 2] !== TQ || os[r - 1] !== DV) throw new Error('attention-grad body: operand shapes');
  if (TQ > 128) throw new Error(`attention-grad: ${TQ} queries (at most 128 in one workgroup)`);
  if (batch * TQ * TK >= 2 ** 31) throw new Error('attention-grad exceeds the 32-bit index space');
  if (batch > 65535) throw new Error(`attention-grad batch ${batch} exceeds the grid`);
  const want = new Set(parts);
  const needDs = want.has('dq') || want.has('dk');
  const needP = want.has('dv');
  const R = batch * TQ, C = TK;
  const params = [batch, TQ, DH, TK, DV];
  const rowTier = (id) => size(N[id].shape) === R && size(N[id].shape) !== R * C;
  // The body's values the kernel forms: dS and/or P, and the reductions they depend on.
  const goals = [].concat(needDs ? [x.ds] : [], needP ? [x.p] : []);
  const deps = new Set();
  const walk = (id) => {
    if (deps.has(id)) return;
    deps.add(id);
    if (id === x.S.id || id === x.dP.id) return;
    for (const i of N[id].inputs) walk(i);
  };
  for (const gl of goals) walk(gl);
  const needDp = deps.has(x.dP.id);
  const reductions = N.filter((n) => isReduce(n) && deps.has(n.id));
  for (const rd of reductions) {
    const src = N[rd.inputs[0]].shape;
    if (rd.attrs.axis !== src.length - 1 || size(src) !== R * C) throw new Error('attention-grad body: reductions must be over the keys');
  }
  const NT = Math.ceil(TK / 16);
  const reduced = new Map();
  const rowLines = [];
  const caches = new Map();
  const cacheFill = [];
  let em;
  const ROW = { key: 'r', idx: 'r', root: false, row: true, limit: R };
  const elemCtx = () => ({ key: 'e', idx: 'e', root: true, limit: R * C });
  em = new Emitter(b, params, {
    special(id, ctx) {
      if (id === x.S.id || id === x.dP.id) {
        if (ctx.row || !ctx.root) throw new Error('attention-grad body: the scores are read at their own index only');
        return id === x.S.id ? 'sacc[jt][l]' : 'dpacc[jt][l]';
      }
      if (reduced.has(id)) return reduced.get(id);
      const n = N[id];
      if (!ctx.row && rowTier(id) && n.op !== 'input' && n.op !== 'const') return em.value(id, ROW, rowLines);
      if (n.op === 'broadcast' && !ctx.row && rowTier(n.inputs[0])) {
        const src = N[n.inputs[0]];
        if (src.op !== 'input' && src.op !== 'const') return em.value(src.id, ROW, rowLines);
      }
      return undefined;
    },
    load(k, ctx, lines) {
      if (k < 4) throw new Error('attention-grad body: Q, K, V and dO are read by the products only');
      if (ctx.key.startsWith('e')) {
        const ck = `${k}|${ctx.idx}`;
        if (!caches.has(ck)) {
          const c = `C${caches.size}`;
          caches.set(ck, c);
          cacheFill.push(`float ${c}[${NT}][4];`, `#pragma unroll
for (int jt = 0; jt < ${NT}; ++jt) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t c = 16u * jt + 4u * q + l;
    const uint32_t e = rowBase + c;
    ${c}[jt][l] = rowOk && c < ${TK}u ? A.in[${k}][${ctx.idx}] : 0.f;
  }
}`);
        }
        return `${caches.get(ck)}[jt][l]`;
      }
      const v = `L${lines.length}_${k}`;
      lines.push(`const float ${v} = A.in[${k}][${ctx.idx}];`);
      return v;
    },
  });
  const loop = (bodyLines) => `#pragma unroll
for (int jt = 0; jt < ${NT}; ++jt) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t c = 16u * jt + 4u * q + l;
    if (rowOk && c < ${TK}u) {
      const uint32_t e = rowBase + c;
${indent(bodyLines, '      ')}
    }
  }
}`;
  const phases = [];
  reductions.forEach((rd, k) => {
    for (const key of Array.from(em.memo.keys())) if (key.startsWith('e')) em.memo.delete(key);
    const rowBefore = rowLines.length;
    const inner = [];
    const v = em.value(rd.inputs[0], elemCtx(), inner);
    const isMax = rd.op === 'max';
    const pre = rowLines.splice(rowBefore);
    phases.push(...pre,
      `float acc${k} = ${isMax ? '(-TCMI_INF)' : '0.f'};`,
      loop(inner.concat([`acc${k} = tcmi::red_${isMax ? 'max' : 'sum'}(acc${k}, ${v});`])),
      `const float red${k} = tcmi::quad16_reduce<${isMax}>(acc${k});`);
    reduced.set(rd.id, `red${k}`);
  });
  // dS and P per score, in the scores' register layout (0 past TK and for rows past TQ).
  for (const key of Array.from(em.memo.keys())) if (key.startsWith('e')) em.memo.delete(key);
  const rowBefore = rowLines.length;
  const inner = [];
  const dsv = needDs ? em.value(x.ds, elemCtx(), inner) : null;
  const pv = needP ? em.value(x.p, elemCtx(), inner) : null;
  const pre = rowLines.splice(rowBefore);
  const valLoop = `#pragma unroll
for (int jt = 0; jt < ${NT}; ++jt) {
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint32_t c = 16u * jt + 4u * q + l;
${needDs ? '    float dse = 0.f;\n' : ''}${needP ? '    float pe = 0.f;\n' : ''}    if (rowOk && c < ${TK}u) {
      const uint32_t e = rowBase + c;
${indent(inner, '      ')}
${needDs ? `      dse = ${dsv};\n` : ''}${needP ? `      pe = ${pv};\n` : ''}    }
${needDs ? '    dsr[jt][l] = dse;\n' : ''}${needP ? '    pr[jt][l] = pe;\n' : ''}  }
}`;
  const views = o.views || {};
  const sizes = o.sizes || {};
  const qv = operandView('__KERNEL___qv', views.q, batchDims, TQ, DH);
  const kv = operandView('__KERNEL___kv', views.k, batchDims, TK, DH);
  const vv = operandView('__KERNEL___vv', views.v, batchDims, TK, DV);
  const ov = operandView('__KERNEL___ov', views.o, batchDims, TQ, DV);
  if ([qv, kv, vv, ov].some((v) => v.mapped) || [views.q, views.k, views.v, views.o].some((v) => v && v.op)) {
    throw new Error('attention-grad operand read through a mapped view or a load op');
  }
  const need = (slot, dense) => (sizes[slot] !== undefined ? sizes[slot] : dense);
  if (qv.limit > need('q', batch * TQ * DH) || kv.limit > need('k', batch * TK * DH) || vv.limit > need('v', batch * TK * DV)
    || ov.limit > need('o', batch * TQ * DV)) {
    throw new Error('attention-grad operand view out of bounds');
  }
  const W = Math.ceil(TQ / 16);
  const THREADS = 64 * W;
  const joint = !!o.joint;
  const outOf = (part) => (joint ? `B.m[${GRAD_PARTS.indexOf(part)}].out` : 'A.out');
  const steps = [];
  if (want.has('dq')) {
    steps.push(`{ // dQ = dS · K: dS from the registers, K from LDS
  tcmi::f4 oacc[G::DH16];
  tcmi::attn_pv<G::NT, G::DH16, G::KS>(oacc, dsr, Ks, t16, q);
  tcmi::attn_store<${TQ}, ${DH}, G::DH16>(${outOf('dq')}, oacc, b, row, q);
}`);
  }
  if (want.has('dk')) {
    steps.push(`__syncthreads();   // K and V read: the pool takes dS and Q
tcmi::attn_rows_to_lds<G::NT, G::TS>(pool, dsr, wave, t16, q);
tcmi::attn_frags_to_lds<G::DH16, G::QS>(pool + G::QROWS * G::TS, qf, wave, t16, q);
__syncthreads();
tcmi::attn_grad_keys<G::NT, G::W, G::DH16, G::TS, G::QS, ${TK}, ${DH}>(${outOf('dk')}, pool, pool + G::QROWS * G::TS, b, wave, t16, q);`);
  }
  if (want.has('dv')) {
    steps.push(`__syncthreads();   // the pool takes P and dO
tcmi::attn_rows_to_lds<G::NT, G::TS>(pool, pr, wave, t16, q);
tcmi::attn_frags_to_lds<G::DV16, G::OS>(pool + G::QROWS * G::TS, dof, wave, t16, q);
__syncthreads();
tcmi::attn_grad_keys<G::NT, G::W, G::DV16, G::TS, G::OS, ${TK}, ${DV}>(${outOf('dv')}, pool, pool + G::QROWS * G::TS, b, wave, t16, q);`);
  }
  const needDo = needDp || want.has('dv');
  const needV = needDp;
  const sig = joint ? 'const TcmiBatch<3> B' : 'const TcmiArgs A';
  const text = `#include "tcmi_attention.h"
${qv.text}${kv.text}${vv.text}${ov.text}extern "C" __global__ void __launch_bounds__(${THREADS}) __KERNEL__(${sig}) {
${joint ? '  const TcmiPtrs& A = B.m[0];   // the three members read the same operands\n' : ''}  using G = tcmi::AttnGradTiles<${TQ}, ${TK}, ${DH}, ${DV}>;
  __shared__ __attribute__((aligned(16))) float pool[G::POOL];
  float* const Ks = pool;
  float* const Vs = pool + G::ROWS * G::KS;
  const uint32_t b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t16 = lane & 15, q = lane >> 4;
  const uint32_t row = wave * 16u + t16;   // this lane's query row
  tcmi::attn_zero_padding<${TK}, ${DH}, ${DV}, ${THREADS}>(Ks, Vs);
  using Kst = tcmi::AttnStage<${TK}, ${DH}, G::KS, ${kv.mode}, false, __KERNEL___kv, ${THREADS}>;
  tcmi::f4 kr[Kst::PER];
  Kst::load(kr, A.in[1], b);
${needV ? `  using Vst = tcmi::AttnStage<${TK}, ${DV}, G::VS, ${vv.mode}, false, __KERNEL___vv, ${THREADS}>;
  tcmi::f4 vr[Vst::PER];
  Vst::load(vr, A.in[2], b);
` : ''}  tcmi::f4 qf[G::DH16];
  tcmi::attn_q<${TQ}, ${DH}, G::DH16, ${qv.mode}, __KERNEL___qv>(qf, A.in[0], b, row, q);
${needDo ? `  tcmi::f4 dof[G::DV16];
  tcmi::attn_q<${TQ}, ${DV}, G::DV16, ${ov.mode}, __KERNEL___ov>(dof, A.in[3], b, row, q);
` : ''}  const bool rowOk = row < ${TQ}u;
  const uint32_t r = b * ${TQ}u + (rowOk ? row : 0u);   // the score row (rows past TQ compute nothing)
  const uint32_t rowBase = r * ${TK}u;
${indent(cacheFill, '  ')}
  Kst::store(kr, Ks);
${needV ? '  Vst::store(vr, Vs);\n' : ''}  __syncthreads();
  tcmi::f4 sacc[G::NT];
  tcmi::attn_scores<G::NT, G::DH16, G::KS>(sacc, qf, Ks, t16, q);
${needDp ? '  tcmi::f4 dpacc[G::NT];\n  tcmi::attn_scores<G::NT, G::DV16, G::VS>(dpacc, dof, Vs, t16, q);\n' : ''}${indent(phases, '  ')}
${needDs ? '  tcmi::f4 dsr[G::NT];\n' : ''}${needP ? '  tcmi::f4 pr[G::NT];\n' : ''}${indent(pre.concat([valLoop]), '  ')}
${indent(steps.join('\n').split('\n'), '  ')}
}
`;
  const flops = 2 * batch * TQ * TK * DH
    + (needDp ? 2 * batch * TQ * TK * DV : 0)
    + (want.has('dq') ? 2 * batch * TQ * TK * DH : 0) + (want.has('dk') ? 2 * batch * TQ * TK * DH : 0)
    + (want.has('dv') ? 2 * batch * TQ * TK * DV : 0);
  return { text, grid: [1, batch, 1], block: [THREADS, 1, 1], params, flops, modes: [qv.mode, kv.mode, vv.mode, ov.mode] };
}

/**
 * One part of an attention-grad node (the part its output is), and, in `joint`, the
 * kernel forming all three of its body's parts in one launch: the perf lowering runs the
 * three nodes sharing a body as one batched launch of it (lower.js batchPlan).
 */
function attentionGradKernel(b, output, opts) {
  const part = gradPart(b, output);
  const one = attnGradText(b, [part], opts);
  const k = kernelText('attng', one.text);
  const all = attnGradText(b, GRAD_PARTS, Object.assign({}, opts, { joint: true }));
  const j = kernelText('attnj', all.text);
  const joint = { name: j.name, source: j.source, grid: all.grid, block: all.block, lds: 0, flops: all.flops, parts: GRAD_PARTS };
  // Work per part: its product, and dP (which only dQ and dK read) counted with dQ; the
  // recomputed scores are not the graph's work.
  const [batch, TQ, DH, TK, DV] = one.params;
  const flops = 2 * batch * TQ * TK * (part === 'dq' ? DH + DV : part === 'dk' ? DH : DV);
  return { name: k.name, source: k.source, params: Uint32Array.from(one.params), grid: one.grid, block: one.block, lds: 0,
    workspace: 0, flops, part, joint, modes: one.modes };
}

// ---- batched launches ----------------------------------------------------------------

// Members of one batched launch at most: its argument block (TcmiBatch, 80 bytes
// a member) stays well inside the 4 KiB a launch's arguments may take.
const MAX_BATCH = 32;
// Kernel families generated here: each reads its launch only through A.in /
// A.out / A.ws, and its z index only in its own text (the headers never read
// blockIdx.z or gridDim.z). `_red`: a split-K matmul's second kernel.
const BATCHABLE = /^(tcmi_(ew|row|mm|mmred|colred|colfin|attn)_[0-9a-f]+)(_red)?$/;
const MAX_GRID_Z = 65535;

/** Whether kernel `k` may run as a member of a batched launch of `count` members. */
function batchable(k, count) {
  return BATCHABLE.test(k.name) && !k.needsPad && k.grid[2] * (count || 2) <= MAX_GRID_Z;
}

/**
 * One launch of kernel `k` over `count` independent sets of buffers: the member
 * grid repeated `count` times along z, the body run with A bound to member
 * blockIdx.z / Z of a TcmiBatch argument block (Z: the member grid's z extent)
 * and blockIdx.z % Z as its own z index. Identical launches (same text: same
 * sizes, same operand views) of independent nodes become one dispatch, so a step
 * of many small launches (a parameter update per tensor, the three projections
 * of an attention layer and their weight gradients) fills the chip with one
 * launch's workgroups instead of paying a launch's ramp and drain each.
 */
/** The statement that opens a kernel whose workgroups take XCD-grouped places. */
const XCD_GROUPED = 'const tcmi::Wg wg = tcmi::xcd_grouped();';

/**
 * The family of kernel `k` for batching: its text with its operand view structs taken out
 * and its own name blanked. Launches of one family differ at most in how their matmul
 * operands are addressed (a mapped view here, a plain one there); their sizes, tiling,
 * epilogue and code are the same, so they can share one dispatch.
 */
function batchFamily(k) {
  // Elementwise kernels, and rowwise kernels that reduce within wavefronts (no LDS), of
  // one grid and workgroup size, whatever their bodies: each member runs its own (every
  // size baked into its text), so independent launches share one dispatch and one ramp
  // and drain.
  if (/^tcmi_ew_[0-9a-f]+$/.test(k.name) && !k.lds && !k.ldsStatic) return `ew@${k.grid.join(',')}/${k.block.join(',')}`;
  if (/^tcmi_row_[0-9a-f]+$/.test(k.name) && !k.lds && !k.ldsStatic && !/__shared__/.test(k.source)) {
    return `row@${k.grid.join(',')}/${k.block.join(',')}`;
  }
  // Matmul tiles take their LDS from a pool shared by instantiations of one size
  // (tcmi::lds_pool); other kernels' views would each add their own LDS: one text a family.
  if (!/^tcmi_mm_[0-9a-f]+$/.test(k.name)) return `${k.name}@${k.grid.join(',')}/${k.block.join(',')}/${k.lds}`;
  if (k.pool !== undefined) {
    // Products whose kernels differ in anything else (operand load modes, tiling,
    // epilogue) run their own bodies too: one grid and workgroup size, one LDS pool
    // size (so the batch takes no more LDS than a member), and the same workgroup
    // places (XCD-grouped or not, which decides how a member's z index is read).
    return `mm@${k.pool}@${k.source.includes(XCD_GROUPED) ? 'xcd' : ''}@${k.grid.join(',')}/${k.block.join(',')}/${k.lds}`;
  }
  const views = new RegExp(`struct ${k.name}_(?:av|bv|qv|kv|vv) \\{[\\s\\S]*?\\n\\};\\n`, 'g');
  return `${k.source.replace(views, '').split(k.name).join('@')}@${k.grid.join(',')}/${k.block.join(',')}/${k.lds}`;
}

/**
 * The batched kernel of `members` (the member launches' kernels at one position, or one
 * kernel repeated `count` times): one dispatch of `count` member grids along z, member
 * blockIdx.z / Z taking its argument block and blockIdx.z % Z as its own z index. Members
 * of one family whose texts differ (their operand views) each run their own body: a
 * switch on the member index picks it, uniformly per workgroup.
 */
function batchedKernel(members, count) {
  const ks = Array.isArray(members) ? members : new Array(count).fill(members);
  const k = ks[0];
  count = ks.length;
  if (!batchable(k, count)) throw new Error(`kernel ${k.name} cannot be batched ${count} times`);
  if (!(Number.isInteger(count) && count >= 2 && count <= MAX_BATCH)) throw new Error(`batch of ${count} launches (2..${MAX_BATCH})`);
  const family = batchFamily(k);
  const [, base, , suffix] = k.name.match(BATCHABLE);
  const variants = [];
  const variantOf = ks.map((m) => {
    if (m.name !== k.name && batchFamily(m) !== family) throw new Error(`kernels ${k.name} and ${m.name} are not of one family`);
    let v = variants.findIndex((x) => x.name === m.name);
    if (v < 0) { v = variants.length; variants.push(m); }
    return v;
  });
  const Z = k.grid[2];
  const parts = variants.map((m) => {
    const sig = `${m.name}(const TcmiArgs A) {`;
    if (m.source.split(sig).length !== 2) throw new Error(`kernel ${m.name}: no single entry point to batch`);
    if (/gridDim\.z/.test(m.source)) throw new Error(`kernel ${m.name} reads gridDim.z`);
    const [head, body] = m.source.split(sig);
    return { m, head, body };
  });
  // A member taking an XCD-grouped place: the place is taken over the whole batched
  // grid, and its z index chooses the member as blockIdx.z does otherwise.
  const grouped = parts[0].body.includes(`  ${XCD_GROUPED}\n`);
  const z = grouped ? 'wg.z' : 'blockIdx.z';
  const ownZ = (t) => t.split(z).join(`(${z} % ${Z}u)`);
  const strip = (body) => (grouped ? body.replace(`  ${XCD_GROUPED}\n`, '') : body);
  const entry = `__KERNEL__${suffix || ''}(const TcmiBatch<${count}> B) {\n${grouped ? `  ${XCD_GROUPED}\n` : ''}  const TcmiPtrs& A = B.m[${z} / ${Z}u];`;
  let text;
  if (variants.length === 1) {
    text = (ownZ(parts[0].head) + entry + ownZ(strip(parts[0].body))).split(base).join('__KERNEL__');
  } else {
    // Every variant's structs (named for its own kernel), then one entry point whose
    // switch runs the member's own body.
    const decl = parts[0].head.slice(parts[0].head.lastIndexOf('extern "C"'));
    const lines = (p) => p.head.slice(0, p.head.lastIndexOf('extern "C"')).split('\n');
    const includes = lines(parts[0]).filter((l) => l.startsWith('#include')).join('\n');
    // Each variant's structs renamed for the batched kernel (v0_, v1_, ...): the members'
    // own kernels may share its module.
    const own = (t, v) => t.split(`${parts[v].m.name}_`).join(`__KERNEL___v${v}_`);
    const structs = parts.map((p, v) => own(lines(p).filter((l) => !l.startsWith('#include')).join('\n'), v));
    const cases = parts.map((p, v) => {
      const labels = variantOf.map((x, i) => (x === v ? `    case ${i}u:` : null)).filter(Boolean).join('\n');
      const stmts = own(ownZ(strip(p.body)), v).replace(/\}\s*$/, '').split('\n').map((l) => (l ? `  ${l}` : l)).join('\n');
      return `${labels} {\n${stmts.replace(/\s+$/, '')}\n      break;\n    }`;
    });
    text = `${includes}\n${structs.join('')}${decl}${entry}\n  switch (${z} / ${Z}u) {\n${cases.join('\n')}\n  }\n}\n`;
  }
  const b = kernelText(`b${k.name.split('_')[1]}`, text);
  return { name: b.name + (suffix || ''), source: b.source, grid: [k.grid[0], k.grid[1], Z * count], block: k.block.slice(), lds: k.lds,
    members: count, variants: variants.length > 1 ? variantOf.map((v) => variants[v].name) : undefined };
}

// ---- ragged batches -----------------------------------------------------------------

// Members of a ragged batch: kernels of at most this many workgroups each (launches that
// fill less than two workgroups per CU, whose cost is mostly the dispatch), and at most
// this many bytes of static LDS over all members.
const RAGGED_MAX_BLOCKS = 512;
const RAGGED_MAX_LDS = 65536;
const LDS_TYPE_BYTES = { float: 4, 'tcmi::f4': 16 };

/** Bytes of the static LDS arrays a kernel text declares itself, or null if not known. */
function textLds(source) {
  let bytes = 0;
  const re = /__shared__\s+(?:__attribute__\(\(aligned\(\d+\)\)\)\s+)?([\w:]+)\s+\w+((?:\[\d+\])+);/g;
  const all = (source.match(/__shared__/g) || []).length;
  let found = 0;
  for (let m = re.exec(source); m; m = re.exec(source)) {
    if (!LDS_TYPE_BYTES[m[1]]) return null;
    bytes += LDS_TYPE_BYTES[m[1]] * m[2].slice(1, -1).split('][').reduce((q, d) => q * Number(d), 1);
    found++;
  }
  return found === all ? bytes : null;
}

/**
 * Whether kernel `k` may join a ragged batch: a one-kernel launch's kernel of the
 * batchable kinds (no split-K second pass), with no dynamic LDS, static LDS of a known
 * size, workgroups placed by blockIdx (not XCD-grouped), one entry point, and at most
 * RAGGED_MAX_BLOCKS workgroups.
 */
function raggable(k) {
  const m = k.name.match(BATCHABLE);
  if (!m || m[3] || k.needsPad || k.lds || k.ldsStatic || k.joint) return false;
  if (k.block[1] !== 1 || k.block[2] !== 1 || k.grid[0] * k.grid[1] * k.grid[2] > RAGGED_MAX_BLOCKS) return false;
  if (k.source.includes(XCD_GROUPED) || textLds(k.source) === null) return false;
  return k.source.split(`${k.name}(const TcmiArgs A) {`).length === 2;
}

/** Whether kernels `ks` may share one ragged batch: one workgroup size, LDS within bounds. */
function raggedFits(ks) {
  if (!(ks.length >= 1 && ks.length <= MAX_BATCH) || !ks.every(raggable)) return false;
  if (!ks.every((k) => k.block[0] === ks[0].block[0])) return false;
  // Matmul tiles share one pool per size (tcmi::lds_pool); each member's own arrays add up.
  const pools = new Set(ks.filter((k) => k.pool !== undefined).map((k) => k.pool));
  const lds = Array.from(pools).reduce((q, f) => q + 4 * f, 0) + ks.reduce((q, k) => q + textLds(k.source), 0);
  return lds <= RAGGED_MAX_LDS;
}

/**
 * A ragged batch: independent launches of small kernels whose grids differ (a product's
 * tile grid, a row reduction's, an elementwise chain's) in one dispatch of their summed
 * workgroups along x. Workgroup L runs member m, the one whose range [start_m, start_m +
 * |grid_m|) holds L, uniformly per workgroup: its own body, with `A` bound to member m's
 * argument block and the names blockIdx and gridDim shadowed in its scope by its own
 * place (l % gx, (l / gx) % gy, l / (gx·gy)), l = L − start_m, and its own grid, so the
 * body runs as it does in its own launch (kernel texts read their places and grids
 * only through those names: a matmul passes its place to tcmi_gemm.h). One workgroup
 * size for all; their static LDS adds up (raggedFits).
 */
function raggedKernel(ks) {
  if (!(ks.length >= 2 && raggedFits(ks))) throw new Error(`kernels ${ks.map((k) => k.name).join(', ')} cannot share a ragged batch`);
  const variants = [];
  const variantOf = ks.map((k) => {
    let v = variants.findIndex((x) => x.name === k.name);
    if (v < 0) { v = variants.length; variants.push(k); }
    return v;
  });
  const parts = variants.map((k) => {
    const [head, body] = k.source.split(`${k.name}(const TcmiArgs A) {`);
    return { k, head: head.slice(0, head.lastIndexOf('extern "C"')), body };
  });
  const includes = Array.from(new Set([].concat(...parts.map((p) => p.head.split('\n').filter((l) => l.startsWith('#include'))))));
  // Each variant's structs renamed for the batched kernel (v0_, v1_, ...).
  const own = (t, v) => t.split(`${parts[v].k.name}_`).join(`__KERNEL___v${v}_`);
  const structs = parts.map((p, v) => own(p.head.split('\n').filter((l) => !l.startsWith('#include')).join('\n'), v));
  let at = 0;
  const branches = ks.map((k, m) => {
    const [gx, gy, gz] = k.grid, count = gx * gy * gz, v = variantOf[m];
    const stmts = own(parts[v].body, v).replace(/\}\s*$/, '').split('\n').map((l) => (l ? `  ${l}` : l)).join('\n').replace(/\s+$/, '');
    const text = `  ${m ? '} else ' : ''}if (tcmi_wg_ < ${at + count}u) {   // member ${m}: workgroups [${at}, ${at + count}), its grid ${gx} x ${gy} x ${gz}
    const uint32_t tcmi_l_ = tcmi_wg_ - ${at}u;
    const TcmiPtrs& A = B.m[${m}];
    const uint3 gridDim = make_uint3(${gx}u, ${gy}u, ${gz}u);
    const uint3 blockIdx = make_uint3(tcmi_l_ % ${gx}u, (tcmi_l_ / ${gx}u) % ${gy}u, tcmi_l_ / ${gx * gy}u);
${stmts}`;
    at += count;
    return text;
  });
  const threads = ks[0].block[0];
  const text = `${includes.join('\n')}${includes.length ? '\n' : ''}${structs.join('')}extern "C" __global__ void __launch_bounds__(${threads}) __KERNEL__(const TcmiBatch<${ks.length}> B) {
  const uint32_t tcmi_wg_ = blockIdx.x;
${branches.join('\n')}
  }
}
`;
  const b = kernelText('rb', text);
  return { name: b.name, source: b.source, grid: [at, 1, 1], block: [threads, 1, 1], lds: 0, members: ks.length, ragged: ks.map((k) => k.name) };
}

module.exports = { elementwiseKernel, rowwiseKernel, colreduceKernels, gemmKernel, gemmTiling, attentionKernel, attentionGradKernel,
  gradPart, GRAD_PARTS, classifyGather, gatherStrides,
  literal, fnv, Emitter, ParamOverflow, WG, MAX_P, MAX_IN, MAX_BATCH, batchable, batchedKernel, batchFamily,
  raggable, raggedFits, raggedKernel, textLds, RAGGED_MAX_BLOCKS, RAGGED_MAX_LDS, COLRED_ONE_PASS };
