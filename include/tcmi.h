/*
 * tcmi.h — the C ABI of the MI355X (gfx950) execution backend for the
 * tensor-compiler's fused graphs.
 *
 * This is the boundary a host binding (the Node N-API addon in
 * tensor-compiler-webgpu_amd/csrc/napi_addon.cpp, or Python ctypes) calls.
 * Every entry point is extern "C", takes plain pointers, sizes and opaque
 * 64-bit handles, and returns a status: 0 on success, otherwise a HIP error
 * code or one of the TCMI_E_* codes below, with a message readable through
 * tcmi_last_error(). Nothing here allocates on behalf of the caller except
 * tcmi_malloc, the module loader and the event/graph constructors.
 *
 * Each entry point names the WebGPU call of the reference's runner it takes
 * the place of (paths are into abho7/tensor-compiler-webgpu):
 *   src/gpu/runtime.js:17-25    GpuRunner.create (requestAdapter/requestDevice)
 *   src/gpu/runtime.js:36-42    GpuRunner.info
 *   src/gpu/runtime.js:44-52    GpuRunner.pipeline (createShaderModule + createComputePipeline)
 *   src/gpu/runtime.js:68-83    createBuffer + queue.writeBuffer (+ canary fill)
 *   src/gpu/runtime.js:86-101   per-launch bind group + dispatchWorkgroups
 *   src/gpu/runtime.js:103-125  copyBufferToBuffer + mapAsync readback
 *   src/gpu/runtime.js:23,61    device.lost (sticky)
 *   src/fusion/trainer-fused.js:72  device-to-device feedback copies
 *   src/fusion/bench.js:124-153 timestamp queries around a pass
 *
 * Threading: calls are made from one host thread; all work is issued in order
 * on one HIP stream per process, created at tcmi_init with default priority.
 */
#ifndef TCMI_H
#define TCMI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes besides hipError_t values (which are all below 10000). */
#define TCMI_OK 0
#define TCMI_E_INVALID 10001      /* bad argument: unknown handle, out-of-range copy, bad launch shape */
#define TCMI_E_COMPILE 10002      /* hiprtc rejected a kernel source; the log is in tcmi_last_error() */
#define TCMI_E_LOST 10003         /* a fatal device error happened earlier; the device is unusable */
#define TCMI_E_NOT_INIT 10004     /* tcmi_init has not succeeded */
#define TCMI_E_IO 10005           /* kernel cache file could not be read or written */

typedef struct tcmi_device_info {
  char name[256];          /* marketing name, e.g. "AMD Instinct MI355X" */
  char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;   /* multiProcessorCount */
  int32_t clock_khz;       /* peak shader clock */
  int32_t memory_clock_khz;
  int32_t memory_bus_width;
  uint64_t total_memory;   /* bytes of HBM */
  int32_t l2_bytes;
  int32_t lds_bytes_per_block;
  int32_t warp_size;       /* 64 on CDNA */
  int32_t max_threads_per_block;
} tcmi_device_info;

/* --- device (runtime.js:17-42) --------------------------------------------- */

/* Select device 0, create the stream. Idempotent. */
int tcmi_init(void);
int tcmi_device_info_get(tcmi_device_info* out);
/* 1 once a fatal device error was seen (runtime.js:23 device.lost). */
int tcmi_lost(void);
/* Message of the last failing call on this thread ("" if none). */
const char* tcmi_last_error(void);
/* Library version string, and the hiprtc options every kernel is compiled with. */
const char* tcmi_version(void);
const char* tcmi_compile_options(void);

/* --- memory (runtime.js:68-83,103-125; trainer-fused.js:72) ----------------- */

/* Device allocation of `bytes`; the handle is the device address, 256-byte
 * aligned. Allocations of 1 MiB or more start at one of 16 staggered offsets
 * (multiples of 4352 bytes) past their hipMalloc base, so that the operands of a
 * streaming kernel do not meet the memory channels in step. Every copy below is
 * checked against the allocation's size before it is issued. */
int tcmi_malloc(uint64_t bytes, uint64_t* handle);
int tcmi_free(uint64_t handle);
/* Size in bytes of a live allocation (TCMI_E_INVALID if unknown). */
int tcmi_size(uint64_t handle, uint64_t* bytes);
/* Synchronous host->device and device->host copies (stream-ordered, then waited). */
int tcmi_h2d(uint64_t dst, uint64_t dst_offset, const void* src, uint64_t bytes);
int tcmi_d2h(void* dst, uint64_t src, uint64_t src_offset, uint64_t bytes);
/* Asynchronous device->device copy on the library stream. */
int tcmi_d2d(uint64_t dst, uint64_t dst_offset, uint64_t src, uint64_t src_offset, uint64_t bytes);
/* Fill `count` 32-bit words with `value` (canaries: runtime.js:12,64-66). Asynchronous. */
int tcmi_fill32(uint64_t dst, uint64_t offset, uint32_t value, uint64_t count);
/* Count the 32-bit words of [offset, offset + 4*count) that differ from `value`. Synchronous. */
int tcmi_count_not32(uint64_t src, uint64_t offset, uint32_t value, uint64_t count, uint64_t* mismatches);

/* --- kernels (runtime.js:44-52) --------------------------------------------- */

/* Directory for compiled code objects, keyed by a hash of (source, options, arch, compiler). */
int tcmi_set_cache_dir(const char* dir);
/* Directory searched for #include "..." by kernel sources (the skeleton headers). */
int tcmi_set_include_dir(const char* dir);
/* Compile `source` with hiprtc for the device's arch (or load it from the cache)
 * and load it as a module. `extra_options` may be NULL. */
int tcmi_module_compile(const char* source, const char* extra_options, uint64_t* module);
/* Compile only, for `arch` (e.g. "gfx950"), into the cache; needs no GPU. Used at build time. */
int tcmi_precompile(const char* source, const char* extra_options, const char* arch);
int tcmi_module_function(uint64_t module, const char* name, uint64_t* function);
int tcmi_module_unload(uint64_t module);
/* Register (kernel arguments are read but not written) and VGPR/SGPR/LDS use of a function. */
int tcmi_function_attrs(uint64_t function, int32_t* vgprs, int32_t* sgprs, int32_t* lds_bytes, int32_t* max_threads);

/* --- launches (runtime.js:86-101) -------------------------------------------- */

/* Enqueue `function` on the library stream. `args` is the packed kernel
 * argument block (HIP_LAUNCH_PARAM_BUFFER_POINTER layout), `args_bytes` its size.
 * The grid and block are checked against the device limits first. */
int tcmi_launch(uint64_t function, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes,
                const void* args, uint64_t args_bytes);
/* Wait for all work on the library stream; reports (and latches) asynchronous faults. */
int tcmi_sync(void);

/* --- a launch that allocates nothing ---------------------------------------------
 * No counterpart in the reference. For callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid it):
 * tcmi_launch with the kernel's workspace (split-K partial sums, column-sum partials)
 * taken from a fixed device array the library holds on each GPU from tcmi_init until
 * the process ends, instead of a tcmi_malloc'd buffer. The 8 bytes at `scratch_offset`
 * of the argument block (the workspace pointer, at byte 72 of the TcmiArgs layout) are
 * replaced by that array's address before the launch; `scratch_bytes` is the workspace
 * the launch's kernels use, at most TCMI_SCRATCH_BYTES (else TCMI_E_INVALID, nothing
 * enqueued). The library cannot see what the kernels write: a `scratch_bytes` below the
 * launch's real workspace is undefined behaviour (the kernels write past the array), so
 * callers take it from the lowering's launch record (`workspace`), as the Python binding's
 * launch_list_with_scratch does. Nothing is cleared: the kernels this library generates write every
 * workspace element before they read it. Every call on one GPU shares the array and
 * it keeps the last call's contents, so launches that use it must not overlap: they
 * do not when issued on the library stream (in order), as these are. */
#define TCMI_SCRATCH_BYTES (64ull << 20)
int tcmi_launch_scratch(uint64_t function, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes,
                        const void* args, uint64_t args_bytes, uint64_t scratch_offset, uint64_t scratch_bytes);

/* --- launch graphs over several streams ----------------------------------------
 * No counterpart in the reference, whose launches go to one in-order WebGPU queue
 * (runtime.js:86-101); here independent launches of a launch list may overlap.
 * The scheduler (js/src/mi355x/schedule.js) assigns each launch a stream and the
 * events it must wait for. */

#define TCMI_MAX_STREAMS 4

/* Make at least `events` event slots for tcmi_launch_dag (do it before a capture). */
int tcmi_dag_reserve(uint32_t events);
/* Enqueue `count` launches (functions, dims: 7 u32 per launch = grid xyz, block xyz,
 * dynamic LDS; args/offsets: packed argument blocks, offsets[count + 1]) over
 * `streams` (1..TCMI_MAX_STREAMS) in-order streams of default priority: launch i
 * goes on stream stream_of[i] (0 = the library stream) after waiting for the event
 * slots waits[wait_begin[i] .. wait_begin[i + 1]), and records slot record_event[i]
 * after it (-1: none). The side streams first wait for all work already on the
 * library stream, and the library stream waits for every side stream at the end,
 * so the whole sequence is ordered against other work like one launch list.
 * Everything is checked before anything is enqueued. With streams > 1 it is refused
 * (TCMI_E_INVALID) while the library stream is being captured: capture over several
 * streams is switched off; with one stream it is captured like any launch list. */
int tcmi_launch_dag(uint32_t count, const uint64_t* functions, const uint32_t* dims, const uint8_t* args,
                    const uint32_t* offsets, uint32_t streams, const uint8_t* stream_of, const int32_t* record_event,
                    const uint32_t* wait_begin, const uint32_t* waits);

/* --- timing (bench.js:124-153) ----------------------------------------------- */

int tcmi_event_create(uint64_t* event);
/* Record on the library stream. */
int tcmi_event_record(uint64_t event);
/* Milliseconds between two recorded events (waits for `end`). */
int tcmi_event_elapsed(uint64_t start, uint64_t end, float* ms);
int tcmi_event_destroy(uint64_t event);

/* --- captured launch sequences (trainer-fused.js:59-81: one submit per step) --- */

/* Begin capturing everything enqueued on the library stream into a HIP graph. */
int tcmi_capture_begin(void);
/* End the capture and instantiate it. */
int tcmi_capture_end(uint64_t* graph);
/* Replay a captured graph on the library stream. */
int tcmi_graph_launch(uint64_t graph);
/* One training step in one call, as FusedTrainer.train does it with one queue
 * submit (trainer-fused.js:59-81: write the batch, submit, read the loss back):
 * `count` host->device copies of bytes[i] from src[i] to the allocation dst[i]
 * (offset 0) on the library stream, small ones staged through pinned host
 * memory, then the replay of `graph`, then `out_bytes` from the device address
 * `out_src` into host `out`, then a wait for all of it. Everything is checked
 * before anything is enqueued; the sources may be reused when it returns. */
int tcmi_graph_step(uint32_t count, const uint64_t* dst, const void* const* src, const uint64_t* bytes, uint64_t graph,
                    uint64_t out_src, void* out, uint64_t out_bytes);
int tcmi_graph_destroy(uint64_t graph);

/* --- counters (src/fusion/bench.js:41-47: every object-creating call and every write
 * is counted, and the timed region must create none; DESIGN.md:1153-1162 there) ------ */

/* Indices into the array tcmi_counters fills. Each counts successful calls since the
 * library loaded: device allocations, frees, module loads (compiled or from the cache),
 * host->device copies (tcmi_h2d and each upload of tcmi_graph_step), device->host
 * copies, event creations, graph instantiations. */
#define TCMI_COUNT_MALLOC 0
#define TCMI_COUNT_FREE 1
#define TCMI_COUNT_MODULE 2
#define TCMI_COUNT_H2D 3
#define TCMI_COUNT_D2H 4
#define TCMI_COUNT_EVENT 5
#define TCMI_COUNT_GRAPH 6
#define TCMI_COUNTERS 7
/* Copy min(n, TCMI_COUNTERS) counters into out; works before tcmi_init. */
int tcmi_counters(uint64_t* out, uint32_t n);

/* --- built-in measurement kernels (workloads.js:312-345 ceilingPrograms) ----- */

/* dst[i] = src[i] over `bytes` (a multiple of 16), grid-strided, `blocks` x 256 threads. */
int tcmi_ceiling_copy(uint64_t dst, uint64_t src, uint64_t bytes, uint32_t blocks);
/* XOR-fold of `bytes` of src into dst[blocks*256] (a pure read). */
int tcmi_ceiling_read(uint64_t dst, uint64_t src, uint64_t bytes, uint32_t blocks);

#ifdef __cplusplus
}
#endif

#endif /* TCMI_H */
