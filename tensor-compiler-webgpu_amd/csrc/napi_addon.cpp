// Node-API binding of the C ABI in include/tcmi.h: the thin addon the
// JavaScript host (tensor-compiler-webgpu_amd/js/src/mi355x/) calls instead of
// WebGPU. Each function unpacks its JavaScript arguments, calls one tcmi_*
// entry point, and turns a non-zero status into a thrown Error carrying
// tcmi_last_error(), as the reference's runner turns WebGPU error scopes into
// thrown Errors (src/gpu/runtime.js:110-115 in abho7/tensor-compiler-webgpu).
//
// Handles (device addresses, module/function/event/graph ids) cross into
// JavaScript as Numbers; addresses on Linux fit in 48 bits, and every handle
// is checked to be an exact integer below 2^53.
//
// Compiled with g++ against Node's headers only (node_api.h); the symbols
// resolve against the running node binary when the addon is loaded.

#include <node_api.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/tcmi.h"

namespace {

napi_value throw_status(napi_env env, int rc, const char* what) {
  std::string msg = std::string(what) + " failed (" + std::to_string(rc) + "): " + tcmi_last_error();
  napi_value code, message, err;
  napi_create_string_utf8(env, std::to_string(rc).c_str(), NAPI_AUTO_LENGTH, &code);
  napi_create_string_utf8(env, msg.c_str(), NAPI_AUTO_LENGTH, &message);
  napi_create_error(env, code, message, &err);
  napi_throw(env, err);
  return nullptr;
}

napi_value throw_type(napi_env env, const char* msg) {
  napi_throw_type_error(env, nullptr, msg);
  return nullptr;
}

#define CHECK(call, what)                          \
  do {                                             \
    int rc_ = (call);                              \
    if (rc_ != 0) return throw_status(env, rc_, what); \
  } while (0)

struct Args {
  napi_env env;
  size_t argc = 12;
  napi_value argv[12];
  bool ok = true;
  Args(napi_env e, napi_callback_info info) : env(e) {
    napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr);
  }
  bool number(size_t i, double* out) {
    napi_valuetype t;
    if (i >= argc || napi_typeof(env, argv[i], &t) != napi_ok || t != napi_number) return false;
    return napi_get_value_double(env, argv[i], out) == napi_ok;
  }
  bool u64(size_t i, uint64_t* out) {
    double d;
    if (!number(i, &d)) return false;
    if (!(d >= 0) || d > 9007199254740991.0 || std::floor(d) != d) return false;
    *out = static_cast<uint64_t>(d);
    return true;
  }
  bool u32(size_t i, uint32_t* out) {
    uint64_t v;
    if (!u64(i, &v) || v > 0xffffffffull) return false;
    *out = static_cast<uint32_t>(v);
    return true;
  }
  bool str(size_t i, std::string* out) {
    napi_valuetype t;
    if (i >= argc || napi_typeof(env, argv[i], &t) != napi_ok) return false;
    if (t == napi_null || t == napi_undefined) { out->clear(); return true; }
    if (t != napi_string) return false;
    size_t len = 0;
    napi_get_value_string_utf8(env, argv[i], nullptr, 0, &len);
    out->resize(len + 1);
    napi_get_value_string_utf8(env, argv[i], &(*out)[0], len + 1, &len);
    out->resize(len);
    return true;
  }
  // Any TypedArray or Buffer: its bytes.
  bool bytes(size_t i, void** data, size_t* length) { return i < argc && typed_bytes(env, argv[i], data, length); }
  static bool typed_bytes(napi_env env, napi_value v, void** data, size_t* length) {
    bool is = false;
    napi_is_typedarray(env, v, &is);
    if (is) {
      napi_typedarray_type type;
      size_t n;
      napi_value ab;
      size_t off;
      if (napi_get_typedarray_info(env, v, &type, &n, data, &ab, &off) != napi_ok) return false;
      size_t el = 1;
      switch (type) {
        case napi_int16_array: case napi_uint16_array: el = 2; break;
        case napi_int32_array: case napi_uint32_array: case napi_float32_array: el = 4; break;
        case napi_float64_array: el = 8; break;
        default:
          if (type == napi_bigint64_array || type == napi_biguint64_array) el = 8;
          break;
      }
      *length = n * el;
      return true;
    }
    napi_is_buffer(env, v, &is);
    if (is) return napi_get_buffer_info(env, v, data, length) == napi_ok;
    return false;
  }
  // A TypedArray of exactly `want`: its data and element count.
  bool typed(size_t i, napi_typedarray_type want, void** data, size_t* count) {
    bool is = false;
    if (i >= argc || napi_is_typedarray(env, argv[i], &is) != napi_ok || !is) return false;
    napi_typedarray_type type;
    napi_value ab;
    size_t off;
    if (napi_get_typedarray_info(env, argv[i], &type, count, data, &ab, &off) != napi_ok) return false;
    return type == want;
  }
  // An array of three unsigned 32-bit numbers.
  bool dim3(size_t i, uint32_t out[3]) {
    bool is = false;
    if (i >= argc || napi_is_array(env, argv[i], &is) != napi_ok || !is) return false;
    for (uint32_t k = 0; k < 3; k++) {
      napi_value v;
      double d;
      if (napi_get_element(env, argv[i], k, &v) != napi_ok) return false;
      if (napi_get_value_double(env, v, &d) != napi_ok || !(d >= 0) || d > 4294967295.0 || std::floor(d) != d) return false;
      out[k] = static_cast<uint32_t>(d);
    }
    return true;
  }
};

napi_value num(napi_env env, double v) {
  napi_value r;
  napi_create_double(env, v, &r);
  return r;
}

napi_value str(napi_env env, const char* s) {
  napi_value r;
  napi_create_string_utf8(env, s, NAPI_AUTO_LENGTH, &r);
  return r;
}

napi_value undef(napi_env env) {
  napi_value r;
  napi_get_undefined(env, &r);
  return r;
}

void set(napi_env env, napi_value obj, const char* key, napi_value v) { napi_set_named_property(env, obj, key, v); }

// ---- device ------------------------------------------------------------------

napi_value Init(napi_env env, napi_callback_info) {
  CHECK(tcmi_init(), "tcmi_init");
  return undef(env);
}

napi_value Info(napi_env env, napi_callback_info) {
  tcmi_device_info d;
  CHECK(tcmi_device_info_get(&d), "tcmi_device_info_get");
  napi_value o;
  napi_create_object(env, &o);
  set(env, o, "name", str(env, d.name));
  set(env, o, "arch", str(env, d.arch));
  set(env, o, "computeUnits", num(env, d.compute_units));
  set(env, o, "clockKHz", num(env, d.clock_khz));
  set(env, o, "memoryClockKHz", num(env, d.memory_clock_khz));
  set(env, o, "memoryBusWidth", num(env, d.memory_bus_width));
  set(env, o, "totalMemory", num(env, static_cast<double>(d.total_memory)));
  set(env, o, "l2Bytes", num(env, d.l2_bytes));
  set(env, o, "ldsBytesPerBlock", num(env, d.lds_bytes_per_block));
  set(env, o, "warpSize", num(env, d.warp_size));
  set(env, o, "maxThreadsPerBlock", num(env, d.max_threads_per_block));
  return o;
}

napi_value Lost(napi_env env, napi_callback_info) {
  napi_value r;
  napi_get_boolean(env, tcmi_lost() != 0, &r);
  return r;
}

napi_value Version(napi_env env, napi_callback_info) { return str(env, tcmi_version()); }
napi_value CompileOptions(napi_env env, napi_callback_info) { return str(env, tcmi_compile_options()); }

// ---- memory ------------------------------------------------------------------

napi_value Malloc(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t bytes, h;
  if (!a.u64(0, &bytes)) return throw_type(env, "malloc(bytes)");
  CHECK(tcmi_malloc(bytes, &h), "tcmi_malloc");
  return num(env, static_cast<double>(h));
}

napi_value Free(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t h;
  if (!a.u64(0, &h)) return throw_type(env, "free(handle)");
  CHECK(tcmi_free(h), "tcmi_free");
  return undef(env);
}

napi_value H2D(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t h, off;
  void* data;
  size_t n;
  if (!a.u64(0, &h) || !a.u64(1, &off) || !a.bytes(2, &data, &n)) return throw_type(env, "h2d(handle, offset, typedArray)");
  CHECK(tcmi_h2d(h, off, data, n), "tcmi_h2d");
  return undef(env);
}

napi_value D2H(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t h, off;
  void* data;
  size_t n;
  if (!a.u64(0, &h) || !a.u64(1, &off) || !a.bytes(2, &data, &n)) return throw_type(env, "d2h(handle, offset, typedArray)");
  CHECK(tcmi_d2h(data, h, off, n), "tcmi_d2h");
  return undef(env);
}

napi_value D2D(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t dst, doff, src, soff, bytes;
  if (!a.u64(0, &dst) || !a.u64(1, &doff) || !a.u64(2, &src) || !a.u64(3, &soff) || !a.u64(4, &bytes))
    return throw_type(env, "d2d(dst, dstOffset, src, srcOffset, bytes)");
  CHECK(tcmi_d2d(dst, doff, src, soff, bytes), "tcmi_d2d");
  return undef(env);
}

napi_value Fill32(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t h, off, count;
  uint32_t v;
  if (!a.u64(0, &h) || !a.u64(1, &off) || !a.u32(2, &v) || !a.u64(3, &count))
    return throw_type(env, "fill32(handle, offset, value, count)");
  CHECK(tcmi_fill32(h, off, v, count), "tcmi_fill32");
  return undef(env);
}

napi_value CountNot32(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t h, off, count, bad = 0;
  uint32_t v;
  if (!a.u64(0, &h) || !a.u64(1, &off) || !a.u32(2, &v) || !a.u64(3, &count))
    return throw_type(env, "countNot32(handle, offset, value, count)");
  CHECK(tcmi_count_not32(h, off, v, count, &bad), "tcmi_count_not32");
  return num(env, static_cast<double>(bad));
}

// ---- kernels -------------------------------------------------------------------

napi_value SetCacheDir(napi_env env, napi_callback_info info) {
  Args a(env, info);
  std::string s;
  if (!a.str(0, &s)) return throw_type(env, "setCacheDir(dir)");
  CHECK(tcmi_set_cache_dir(s.c_str()), "tcmi_set_cache_dir");
  return undef(env);
}

napi_value SetIncludeDir(napi_env env, napi_callback_info info) {
  Args a(env, info);
  std::string s;
  if (!a.str(0, &s)) return throw_type(env, "setIncludeDir(dir)");
  CHECK(tcmi_set_include_dir(s.c_str()), "tcmi_set_include_dir");
  return undef(env);
}

napi_value Compile(napi_env env, napi_callback_info info) {
  Args a(env, info);
  std::string src, opts;
  uint64_t m;
  if (!a.str(0, &src) || !a.str(1, &opts)) return throw_type(env, "compile(source, options)");
  CHECK(tcmi_module_compile(src.c_str(), opts.c_str(), &m), "tcmi_module_compile");
  return num(env, static_cast<double>(m));
}

napi_value Precompile(napi_env env, napi_callback_info info) {
  Args a(env, info);
  std::string src, opts, arch;
  if (!a.str(0, &src) || !a.str(1, &opts) || !a.str(2, &arch)) return throw_type(env, "precompile(source, options, arch)");
  CHECK(tcmi_precompile(src.c_str(), opts.c_str(), arch.c_str()), "tcmi_precompile");
  return undef(env);
}

napi_value Function(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t m, f;
  std::string name;
  if (!a.u64(0, &m) || !a.str(1, &name)) return throw_type(env, "function(module, name)");
  CHECK(tcmi_module_function(m, name.c_str(), &f), "tcmi_module_function");
  return num(env, static_cast<double>(f));
}

napi_value Unload(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t m;
  if (!a.u64(0, &m)) return throw_type(env, "unload(module)");
  CHECK(tcmi_module_unload(m), "tcmi_module_unload");
  return undef(env);
}

// launch(fn, grid[3], block[3], lds, argBytes)
napi_value Launch(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t f;
  uint32_t grid[3], block[3], lds;
  void* data = nullptr;
  size_t n = 0;
  if (!a.u64(0, &f) || !a.dim3(1, grid) || !a.dim3(2, block) || !a.u32(3, &lds) || !a.bytes(4, &data, &n))
    return throw_type(env, "launch(fn, grid, block, lds, args)");
  CHECK(tcmi_launch(f, grid, block, lds, data, n), "tcmi_launch");
  return undef(env);
}

// A device or function handle held in a double: a whole number in [0, 2^53).
bool handle_ok(double h) { return h >= 0 && h <= 9007199254740991.0 && std::floor(h) == h; }

// Function handles of a Float64Array, each checked before the cast.
bool handles(const double* F, size_t count, std::vector<uint64_t>& out) {
  out.resize(count);
  for (size_t i = 0; i < count; i++) {
    if (!handle_ok(F[i])) return false;
    out[i] = static_cast<uint64_t>(F[i]);
  }
  return true;
}

// launchMany(fns: Float64Array, dims: Uint32Array (7 per launch: grid xyz, block xyz, lds),
//            args: Uint8Array, offsets: Uint32Array (n + 1)): one native call per launch sequence.
napi_value LaunchMany(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void *fns, *dims, *args, *offs;
  size_t count, nd, na, no;
  if (!a.typed(0, napi_float64_array, &fns, &count) || !a.typed(1, napi_uint32_array, &dims, &nd) ||
      !a.bytes(2, &args, &na) || !a.typed(3, napi_uint32_array, &offs, &no))
    return throw_type(env, "launchMany(fns: Float64Array, dims: Uint32Array, args, offsets: Uint32Array)");
  if (nd != count * 7 || no != count + 1) return throw_type(env, "launchMany: array lengths disagree");
  std::vector<uint64_t> F;
  if (!handles(static_cast<const double*>(fns), count, F)) return throw_type(env, "launchMany: bad function handle");
  const uint32_t* D = static_cast<const uint32_t*>(dims);
  const uint32_t* O = static_cast<const uint32_t*>(offs);
  const uint8_t* A = static_cast<const uint8_t*>(args);
  for (size_t i = 0; i < count; i++)
    if (O[i] > O[i + 1] || O[i + 1] > na) return throw_type(env, "launchMany: bad argument offsets");
  for (size_t i = 0; i < count; i++)
    CHECK(tcmi_launch(F[i], D + 7 * i, D + 7 * i + 3, D[7 * i + 6], A + O[i], O[i + 1] - O[i]), "tcmi_launch");
  return undef(env);
}

// launchDag(fns: Float64Array, dims: Uint32Array, args, offsets: Uint32Array, streams,
//           streamOf: Uint8Array, recordEvent: Int32Array, waitBegin: Uint32Array (n + 1),
//           waits: Uint32Array): a launch list over several streams.
napi_value LaunchDag(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void *fns, *dims, *args, *offs, *sof, *rec, *wb, *ws;
  size_t count, nd, na, no, ns, nr, nwb, nw;
  uint32_t streams;
  if (!a.typed(0, napi_float64_array, &fns, &count) || !a.typed(1, napi_uint32_array, &dims, &nd) ||
      !a.bytes(2, &args, &na) || !a.typed(3, napi_uint32_array, &offs, &no) || !a.u32(4, &streams) ||
      !a.typed(5, napi_uint8_array, &sof, &ns) || !a.typed(6, napi_int32_array, &rec, &nr) ||
      !a.typed(7, napi_uint32_array, &wb, &nwb) || !a.typed(8, napi_uint32_array, &ws, &nw))
    return throw_type(env, "launchDag(fns: Float64Array, dims: Uint32Array, args, offsets: Uint32Array, streams, "
                           "streamOf: Uint8Array, recordEvent: Int32Array, waitBegin: Uint32Array, waits: Uint32Array)");
  if (nd != count * 7 || no != count + 1 || ns != count || nr != count || nwb != count + 1)
    return throw_type(env, "launchDag: array lengths disagree");
  const uint32_t* O = static_cast<const uint32_t*>(offs);
  const uint32_t* WB = static_cast<const uint32_t*>(wb);
  if (O[count] > na || WB[count] > nw) return throw_type(env, "launchDag: offsets past the arrays");
  std::vector<uint64_t> F;
  if (!handles(static_cast<const double*>(fns), count, F)) return throw_type(env, "launchDag: bad function handle");
  CHECK(tcmi_launch_dag(static_cast<uint32_t>(count), F.data(), static_cast<const uint32_t*>(dims),
                        static_cast<const uint8_t*>(args), O, streams, static_cast<const uint8_t*>(sof),
                        static_cast<const int32_t*>(rec), WB, static_cast<const uint32_t*>(ws)),
        "tcmi_launch_dag");
  return undef(env);
}

// graphStep(dsts: Float64Array, srcs: TypedArray[], graph, outSrc, out: TypedArray):
// one training step in one native call (uploads, graph replay, result readback, wait).
napi_value GraphStep(napi_env env, napi_callback_info info) {
  Args a(env, info);
  void *dsts, *out;
  size_t nd, nout;
  uint64_t graph, out_src;
  bool is_array = false;
  if (!a.bytes(0, &dsts, &nd) || a.argc < 2 || napi_is_array(env, a.argv[1], &is_array) != napi_ok || !is_array ||
      !a.u64(2, &graph) || !a.u64(3, &out_src) || !a.bytes(4, &out, &nout))
    return throw_type(env, "graphStep(dsts, srcs, graph, outSrc, out)");
  // The destinations are device handles held as doubles: a Float64Array, nothing else.
  napi_typedarray_type dtype;
  size_t dlen, doff;
  void* ddata;
  napi_value dab;
  if (napi_get_typedarray_info(env, a.argv[0], &dtype, &dlen, &ddata, &dab, &doff) != napi_ok || dtype != napi_float64_array)
    return throw_type(env, "graphStep: destinations must be a Float64Array of handles");
  uint32_t count = 0;
  napi_get_array_length(env, a.argv[1], &count);
  if (nd != count * 8) return throw_type(env, "graphStep: one destination per source");
  std::vector<uint64_t> dst(count), bytes(count);
  std::vector<const void*> src(count);
  for (uint32_t i = 0; i < count; ++i) {
    double h = static_cast<const double*>(dsts)[i];
    if (!handle_ok(h)) return throw_type(env, "graphStep: bad destination handle");
    dst[i] = static_cast<uint64_t>(h);
    napi_value el;
    void* data;
    size_t n;
    if (napi_get_element(env, a.argv[1], i, &el) != napi_ok || !Args::typed_bytes(env, el, &data, &n))
      return throw_type(env, "graphStep: every source must be a TypedArray");
    src[i] = data;
    bytes[i] = n;
  }
  CHECK(tcmi_graph_step(count, dst.data(), src.data(), bytes.data(), graph, out_src, out, nout), "tcmi_graph_step");
  return undef(env);
}

napi_value DagReserve(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint32_t n;
  if (!a.u32(0, &n)) return throw_type(env, "dagReserve(events)");
  CHECK(tcmi_dag_reserve(n), "tcmi_dag_reserve");
  return undef(env);
}

napi_value Sync(napi_env env, napi_callback_info) {
  CHECK(tcmi_sync(), "tcmi_sync");
  return undef(env);
}

// ---- events and captured sequences ---------------------------------------------------

napi_value EventCreate(napi_env env, napi_callback_info) {
  uint64_t e;
  CHECK(tcmi_event_create(&e), "tcmi_event_create");
  return num(env, static_cast<double>(e));
}

napi_value EventRecord(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t e;
  if (!a.u64(0, &e)) return throw_type(env, "eventRecord(event)");
  CHECK(tcmi_event_record(e), "tcmi_event_record");
  return undef(env);
}

napi_value EventElapsed(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t s, e;
  float ms = 0;
  if (!a.u64(0, &s) || !a.u64(1, &e)) return throw_type(env, "eventElapsed(start, end)");
  CHECK(tcmi_event_elapsed(s, e, &ms), "tcmi_event_elapsed");
  return num(env, ms);
}

napi_value EventDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t e;
  if (!a.u64(0, &e)) return throw_type(env, "eventDestroy(event)");
  CHECK(tcmi_event_destroy(e), "tcmi_event_destroy");
  return undef(env);
}

napi_value CaptureBegin(napi_env env, napi_callback_info) {
  CHECK(tcmi_capture_begin(), "tcmi_capture_begin");
  return undef(env);
}

napi_value CaptureEnd(napi_env env, napi_callback_info) {
  uint64_t g;
  CHECK(tcmi_capture_end(&g), "tcmi_capture_end");
  return num(env, static_cast<double>(g));
}

napi_value GraphLaunch(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t g;
  if (!a.u64(0, &g)) return throw_type(env, "graphLaunch(graph)");
  CHECK(tcmi_graph_launch(g), "tcmi_graph_launch");
  return undef(env);
}

napi_value GraphDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t g;
  if (!a.u64(0, &g)) return throw_type(env, "graphDestroy(graph)");
  CHECK(tcmi_graph_destroy(g), "tcmi_graph_destroy");
  return undef(env);
}

napi_value CeilingCopy(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t dst, src, bytes;
  uint32_t blocks;
  if (!a.u64(0, &dst) || !a.u64(1, &src) || !a.u64(2, &bytes) || !a.u32(3, &blocks))
    return throw_type(env, "ceilingCopy(dst, src, bytes, blocks)");
  CHECK(tcmi_ceiling_copy(dst, src, bytes, blocks), "tcmi_ceiling_copy");
  return undef(env);
}

napi_value CeilingRead(napi_env env, napi_callback_info info) {
  Args a(env, info);
  uint64_t dst, src, bytes;
  uint32_t blocks;
  if (!a.u64(0, &dst) || !a.u64(1, &src) || !a.u64(2, &bytes) || !a.u32(3, &blocks))
    return throw_type(env, "ceilingRead(dst, src, bytes, blocks)");
  CHECK(tcmi_ceiling_read(dst, src, bytes, blocks), "tcmi_ceiling_read");
  return undef(env);
}

// counters(): { malloc, free, module, h2d, d2h, event, graph } since the library loaded.
napi_value Counters(napi_env env, napi_callback_info) {
  uint64_t c[TCMI_COUNTERS];
  CHECK(tcmi_counters(c, TCMI_COUNTERS), "tcmi_counters");
  static const char* names[TCMI_COUNTERS] = {"malloc", "free", "module", "h2d", "d2h", "event", "graph"};
  napi_value o;
  napi_create_object(env, &o);
  for (int k = 0; k < TCMI_COUNTERS; ++k) napi_set_named_property(env, o, names[k], num(env, static_cast<double>(c[k])));
  return o;
}

napi_value Register(napi_env env, napi_value exports) {
  struct {
    const char* name;
    napi_callback cb;
  } fns[] = {
      {"init", Init}, {"info", Info}, {"lost", Lost}, {"version", Version}, {"compileOptions", CompileOptions},
      {"malloc", Malloc}, {"free", Free}, {"h2d", H2D}, {"d2h", D2H}, {"d2d", D2D}, {"fill32", Fill32},
      {"countNot32", CountNot32}, {"setCacheDir", SetCacheDir}, {"setIncludeDir", SetIncludeDir},
      {"compile", Compile}, {"precompile", Precompile}, {"function", Function}, {"unload", Unload},
      {"launch", Launch}, {"launchMany", LaunchMany}, {"launchDag", LaunchDag}, {"dagReserve", DagReserve},
      {"sync", Sync}, {"eventCreate", EventCreate},
      {"eventRecord", EventRecord}, {"eventElapsed", EventElapsed}, {"eventDestroy", EventDestroy},
      {"captureBegin", CaptureBegin}, {"captureEnd", CaptureEnd}, {"graphLaunch", GraphLaunch}, {"graphStep", GraphStep},
      {"graphDestroy", GraphDestroy}, {"ceilingCopy", CeilingCopy}, {"ceilingRead", CeilingRead},
      {"counters", Counters},
  };
  for (auto& f : fns) {
    napi_value fn;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn);
    napi_set_named_property(env, exports, f.name, fn);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Register)
