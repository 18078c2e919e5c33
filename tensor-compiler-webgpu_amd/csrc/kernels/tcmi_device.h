// Device-side skeletons of the MI355X (gfx950) backend, included by every
// kernel source the lowering generates (tensor-compiler-webgpu_amd/js/src/mi355x/codegen.js)
// and compiled by hiprtc at run time.
//
// The lowering writes, per launch, only the straight-line body of a fused
// node (the ops of the fusion group, kept in registers) and the load of each
// operand; everything that decides how the chip is used lives here:
//   * the argument block every kernel takes (TcmiArgs);
//   * the per-op arithmetic, shared by fused and unfused kernels so that the
//     two round identically op by op;
//   * operand index maps for broadcast/transpose loads;
//   * wave- and block-level reductions for the rowwise kernels;
//   * the fp32 MFMA matmul with a fused epilogue (tcmi_gemm.h).
//
// Targets CDNA4: 64-lane wavefronts, 256-thread workgroups, 128-bit loads.

#pragma once

// hiprtc provides the HIP device environment (and the fixed-width integer
// types) itself; a full hipcc build includes it.
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <stdint.h>
#else
typedef unsigned int uint32_t;
typedef int int32_t;
typedef unsigned long long uint64_t;
#endif

#define TCMI_INF __builtin_inff()

#define TCMI_MAX_IN 8
#define TCMI_MAX_P 48

// The one kernel argument: operand pointers, the output, an optional
// workspace, and a u32 block P that carries the launch's sizes and index maps
// for inspection (kernels have them as constants of their text and never read P).
struct TcmiArgs {
  const float* in[TCMI_MAX_IN];
  float* out;
  float* ws;
  uint32_t P[TCMI_MAX_P];
};

// A batched launch of one kernel over N independent launches of it (same
// sizes, different buffers): the member kernel's grid repeated N times along z,
// its body run with A bound to member blockIdx.z / Z (Z: the member grid's z
// extent) and blockIdx.z % Z in place of its own z index. Kernel texts read z
// only in their own text, never in these headers, so the rewrite is complete.
struct TcmiPtrs {
  const float* in[TCMI_MAX_IN];
  float* out;
  float* ws;
};
template <int N>
struct TcmiBatch {
  TcmiPtrs m[N];
};

namespace tcmi {

// A native 4-wide float vector (128-bit loads and stores, non-temporal stores).
typedef float f4 __attribute__((ext_vector_type(4)));

// ---- arithmetic (the per-op semantics of the float32 kernels) --------------------
//
// Each op must stay inside the error budget the reference registered for it
// (src/gpu/bounds.js:25-55 in abho7/tensor-compiler-webgpu): exp within
// (3 + 2|x|) ulp, log within 3 ulp or 2^-21 absolute, tanh within 1e-5
// absolute, division within 2.5 ulp, sqrt within 4.5 ulp; results that would
// be subnormal may be flushed to zero.

__device__ __forceinline__ float op_add(float a, float b) { return a + b; }
__device__ __forceinline__ float op_sub(float a, float b) { return a - b; }
__device__ __forceinline__ float op_mul(float a, float b) { return a * b; }
// a / b as a · (1/b) with the hardware reciprocal (1 ulp): at most 1.5 ulp in
// all, inside the 2.5 ulp budget, in 2 instructions instead of the ~10 of a
// correctly rounded division. Where 1/b leaves the normal range (|b| outside
// [2^-126, 2^126]) the budget itself gives no bound (bounds.js:29-33).
__device__ __forceinline__ float op_div(float a, float b) { return a * __builtin_amdgcn_rcpf(b); }
__device__ __forceinline__ float op_neg(float a) { return -a; }
// exp(x) = 2^(x·log2 e) on the transcendental unit: the product's rounding
// contributes |x|·2^-24 relative, the unit about 1 ulp — inside (3 + 2|x|) ulp.
__device__ __forceinline__ float op_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
// log(x) = log2(x)·ln 2 on the transcendental unit; subnormal inputs are
// scaled into the normal range first so they keep their exponent.
__device__ __forceinline__ float op_log(float x) {
  const bool tiny = x < 1.17549435e-38f;
  const float s = tiny ? x * 16777216.0f : x;  // 2^24
  const float l = __builtin_amdgcn_logf(s) * 0.69314718055994531f;
  return tiny ? l - 16.635532333438687f : l;    // 24·ln 2
}
__device__ __forceinline__ float op_relu(float x) { return x > 0.0f ? x : 0.0f; }
__device__ __forceinline__ float op_step(float x) { return x > 0.0f ? 1.0f : 0.0f; }
// tanh(clamp(x, -20, 20)) as the reference's kernels clamp it; at |x| >= 20
// tanh is 1 in float32, so the clamp loses nothing. Computed as
// sign(x)·(1 - 2·rcp(e^{2|x|} + 1)): absolute error a few 2^-24, far inside 1e-5.
__device__ __forceinline__ float op_tanh(float x) {
  const float c = fminf(fmaxf(x, -20.0f), 20.0f);
  const float e = op_exp(2.0f * fabsf(c));
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return copysignf(t, c);
}
__device__ __forceinline__ float op_sqrt(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ float op_copy(float x) { return x; }

// The reductions' combine steps. max keeps the interpreter's `v > acc ? v : acc`
// (src/interp.js:45): a NaN never replaces the running value.
__device__ __forceinline__ float red_sum(float acc, float v) { return acc + v; }
__device__ __forceinline__ float red_max(float acc, float v) { return v > acc ? v : acc; }

__device__ __forceinline__ float f32_bits(uint32_t b) { return __uint_as_float(b); }

__device__ __forceinline__ float lane4(const float4& v, int l) {
  return l == 0 ? v.x : l == 1 ? v.y : l == 2 ? v.z : v.w;
}

// ---- operand index maps -----------------------------------------------------------
//
// A load through a broadcast or transpose reads its source at an index
// computed from the output's flat index. The lowering classifies each such
// load and writes the index as an expression of constants (it knows every
// shape): `(i / inner) % extent` for any broadcast whose kept axes are one
// contiguous run of the output's axes (row vectors, columns, scalars), and a
// sum over axes of `((i / outStride_d) % extent_d) · srcStride_d` otherwise.
// Each map is proved in bounds by the lowering before the kernel is emitted.

// ---- reductions across a workgroup ---------------------------------------------------

template <bool IsMax>
__device__ __forceinline__ float combine(float a, float b) {
  return IsMax ? red_max(a, b) : red_sum(a, b);
}

// Reduce within the 64 lanes of a wavefront (butterfly; every lane gets the result).
template <bool IsMax>
__device__ __forceinline__ float wave_reduce(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = combine<IsMax>(v, __shfl_xor(v, off, 64));
  return v;
}

// Reduce within aligned groups of L lanes (L = 16, 32 or 64) of a wavefront:
// butterfly over the group, then every lane takes the group's first lane's
// value, so all lanes of a group hold the same bits.
template <bool IsMax, int L>
__device__ __forceinline__ float group_reduce(float v) {
  static_assert(L == 16 || L == 32 || L == 64, "group width");
#pragma unroll
  for (int off = L / 2; off >= 1; off >>= 1) v = combine<IsMax>(v, __shfl_xor(v, off, L));
  return __shfl(v, 0, L);
}

// Reduce across the four lanes t, t + 16, t + 32, t + 48 of a wavefront: the
// lane groups of a 16 x 16 matrix-core tile that together hold one row of it.
// Every one of the four takes lane t's result, so all hold the same bits.
template <bool IsMax>
__device__ __forceinline__ float quad16_reduce(float v) {
  v = combine<IsMax>(v, __shfl_xor(v, 16, 64));
  v = combine<IsMax>(v, __shfl_xor(v, 32, 64));
  return __shfl(v, static_cast<int>(threadIdx.x & 15u), 64);
}

// Reduce over a workgroup of THREADS (a multiple of 64); every thread gets the
// result. `scratch` holds THREADS/64 floats of LDS; it is reused across calls,
// hence the barrier before returning.
template <bool IsMax, int THREADS>
__device__ __forceinline__ float block_reduce(float v, float* scratch) {
  v = wave_reduce<IsMax>(v);
  if (THREADS == 64) return v;
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int w = 1; w < THREADS / 64; w++) r = combine<IsMax>(r, scratch[w]);
  __syncthreads();
  return r;
}

}  // namespace tcmi
