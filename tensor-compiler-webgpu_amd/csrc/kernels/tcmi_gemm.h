// fp32 matmul on CDNA4 matrix cores with a fused epilogue.
//
// C[b] = A[b] · B[b] (A: [M, K], B: [K, N]), then out[i] = Epi(A, i, C[b][row][col])
// with i = (b·M + row)·N + col: the epilogue is the fused body of a
// matmul-epilogue group (bias broadcast, activation, residual), applied while
// the accumulator is still in registers.
//
// Operands are strided views: element (b, r, c) of an operand is at
// V::batch(b) + r·V::SR + c·V::SC of its buffer, so a transposed operand
// (autodiff's transpose(W) and transpose(X), attention's transposed keys, a
// head split) is read in place instead of being materialised first. A mapped view
// (V::MAPPED) places the element at V::batch(b) + V::row(r) + V::col(c) instead: a
// chain of transposes and reshapes (attention's heads merged back into rows) makes
// the row or column index step over several strides. The load
// path per operand (MODE) follows its layout:
//   MODE_C  c contiguous (SC = 1): 128-bit loads along c (the row-major case)
//   MODE_R  r contiguous (SR = 1): 128-bit loads along r (the transposed case)
//   MODE_S  anything else: one 32-bit load per element
// (for A, r is the output row and c the K index; for B, r is K and c the
// output column). The LDS tile keeps the layout of the loads, so every
// 128-bit load is one 128-bit LDS store, and the reads adapt instead:
//   A row-major  As[row][k]: a lane's 4 k values in one ds_read_b128
//   A k-major    As[k][row]: 4 ds_read_b32 (MODE_R)
//   B k-major    Bs[k][col]: one ds_read_b32 per k
//   B col-major  Bs[col][k]: a lane's 4 k values in one ds_read_b128 (MODE_R)
// Every tile's row stride is padded by 4 floats, which puts the four lane
// groups q of a read (or the 16 lanes of a 128-bit read) on disjoint banks.
// (Storing a transposed tile in the other layout would scatter each 128-bit
// load into four 32-bit LDS writes that collide on the same banks; measured
// on the MI355X, that stalled LDS for a third of the kernel's time.)
//
// Tiling: a workgroup of 2 x WN wavefronts (WN = 2: 256 threads, WN = 4: 512)
// owns a BM x BN tile of C; each wavefront owns (TM·16) x (TN·16) of it as TM x TN
// accumulators of v_mfma_f32_16x16x4f32 (D 16x16 += A 16x4 · B 4x16). K is
// walked BK (16, 32 or 64) at a time through two LDS buffers: the global loads
// of the next slice are in flight while the current one feeds the matrix
// cores, and one barrier per slice separates the two. A deeper slice gives the
// matrix cores more work per round trip to memory, which is what a long-K,
// few-tile matmul (a weight gradient) needs when there is one workgroup per CU.
//
// Operand layout per lane of a 16x16x4 MFMA (lane = 16·q + t, t in 0..15):
//   A value: row t, k-group q;  B value: column t, k-group q;
//   D: column t, rows 4q .. 4q+3 (one per accumulator register).
// The kernel passes the B value as the MFMA's first operand and the A value as
// its second, so each 16 x 16 accumulator holds its output tile transposed:
// lane (t, q) has row t, columns 4q .. 4q+3 — four consecutive outputs.
// Within each 16-wide part of a slice, lane group q supplies k = 4q + s at step
// s, so a lane's four A values of a part are contiguous in LDS (one ds_read_b128);
// both operands use the same k for the same (q, s), so the product is exact
// in what it sums, in an order the float32 budget already covers (any order
// of K terms, gamma(K)). The order depends on neither BK, the tile size nor
// the operands' layouts (k ascends 16 at a time whatever the slice depth): a
// view and a materialised copy of the same operand give the same bits.

#pragma once

#include "tcmi_device.h"

namespace tcmi {

enum { MODE_C = 0, MODE_R = 1, MODE_S = 2 };

// The contiguous row-major view of a [batch, R, C] operand.
template <uint32_t R, uint32_t C>
struct DenseView {
  static constexpr size_t SR = C, SC = 1;
  static __device__ __forceinline__ size_t batch(uint32_t b) { return (size_t)b * R * C; }
};

// One LDS array of FLOATS floats per size: every caller asking for the same size gets the
// same array.
template <int FLOATS>
__device__ __forceinline__ float* lds_pool() {
  __shared__ __attribute__((aligned(16))) float pool[FLOATS];
  return pool;
}

// A view's row and column offsets: r·SR and c·SC, or, for a mapped view (MAPPED: an
// operand read through a chain of transposes and reshapes, whose row or column index
// steps over several strides), its own row(r) and col(c).
template <class V>
__device__ constexpr auto mapped_view(int) -> decltype(V::MAPPED, bool()) { return true; }
template <class V>
__device__ constexpr bool mapped_view(long) { return false; }
template <class V>
__device__ __forceinline__ size_t vrow(uint32_t r) {
  if constexpr (mapped_view<V>(0)) return V::row(r);
  else return (size_t)r * V::SR;
}
template <class V>
__device__ __forceinline__ size_t vcol(uint32_t c) {
  if constexpr (mapped_view<V>(0)) return V::col(c);
  else return (size_t)c * V::SC;
}

// The op a view applies to each element it loads: V::OP 1 is relu (tcmi::op_relu, the
// op a relu kernel runs, so the same bits as reading that kernel's output); a view
// without OP loads elements as they are. Applied as a staged slice is stored to LDS,
// not as it is loaded: the slice's global loads stay in flight while the previous
// slice is computed (an op right after the load would wait for it).
template <class V>
__device__ constexpr auto view_op(int) -> decltype(V::OP, int()) { return V::OP; }
template <class V>
__device__ constexpr int view_op(long) { return 0; }
template <class V>
__device__ __forceinline__ float vop(float x) {
  if constexpr (view_op<V>(0) == 1) return op_relu(x);
  else return x;
}
template <class V>
__device__ __forceinline__ float4 vop(float4 x) {
  if constexpr (view_op<V>(0) == 1) return make_float4(op_relu(x.x), op_relu(x.y), op_relu(x.z), op_relu(x.w));
  else return x;
}

// A workgroup's (x, y, z) place in its launch's grid.
struct Wg {
  uint32_t x, y, z;
};

// Workgroups grouped by XCD for split-K launches. The G = gridDim.x * gridDim.y tiles
// of one z index (one K chunk of one product) read the same A and B panels; the
// hardware hands a launch's workgroups to the 8 XCDs in turn by linear id L, so L
// runs on XCD L % 8, and consecutive tiles would land on 8 different L2 caches.
// Here z index q = L % 8 + 8 * (L / (8 * G)) and tile t = (L / 8) % G: every tile of
// one z index runs on one XCD. A bijection of [0, G * gridDim.z) when gridDim.z is a
// multiple of 8 (launch order kept otherwise), so every (tile, z) is computed once,
// by the same code: only which workgroup computes it changes, not the result.
__device__ __forceinline__ Wg xcd_grouped() {
  const uint32_t gx = gridDim.x, gy = gridDim.y, nz = gridDim.z, G = gx * gy;
  if (nz % 8u != 0u) return {blockIdx.x, blockIdx.y, blockIdx.z};
  const uint32_t L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const uint32_t rest = L / 8u, t = rest % G;
  return {t % gx, t / gx, L % 8u + 8u * (rest / G)};
}

// Sizes are compile-time constants of the generated kernel (batch, M, K, N, and
// for SPLIT the number of K chunks and their length, a multiple of 16). The
// workgroup's z index `zid` enumerates batches, or for SPLIT (batch, chunk)
// pairs, and each SPLIT workgroup stores its raw
// partial tile to the workspace at ((chunk·batch + b)·M + row)·N + col; a
// second kernel (gemm_splitk_reduce) sums the chunks in order and applies the
// epilogue. MODE_C needs C % 4 == 0 and MODE_R needs R % 4 == 0 (R, C: the
// operand's extents), and both need every other stride a multiple of 4, so a
// 128-bit load is aligned and either wholly inside the operand or wholly out.
template <int TM, int TN, int BK, int PF, int AMODE, int BMODE, bool SPLIT, class AV, class BV, class Epi, int WN = 2,
          bool PRIO = false, int KW = 1, class Args = TcmiArgs>
__device__ __forceinline__ void gemm_f32(const Args& A, const float* __restrict__ a_ptr,
                                         const float* __restrict__ b_ptr, const uint32_t batch, const uint32_t M,
                                         const uint32_t K, const uint32_t N, const uint32_t chunks,
                                         const uint32_t chunkK, const uint32_t zid, const uint32_t tx,
                                         const uint32_t ty) {
  // KW groups of 2 x WN wavefronts; in each group a wavefront owns (TM·16) x (TN·16)
  // of the BM x BN tile, and group g sums its own part of K (see below).
  static_assert(KW == 1 || KW == 2 || KW == 4, "K groups");
  constexpr int THREADS = 64 * 2 * WN;   // threads of one K group
  constexpr int BM = 2 * TM * 16;
  constexpr int BN = WN * TN * 16;
  static_assert(BK == 16 || BK == 32 || BK == 64, "slice depth");
  static_assert(PF == 1 || PF == 2, "prefetch depth");
  constexpr bool A_KMAJOR = AMODE == MODE_R;   // As[k][row] instead of As[row][k]
  constexpr bool B_NMAJOR = BMODE == MODE_R;   // Bs[col][k] instead of Bs[k][col]
  constexpr int AS = A_KMAJOR ? BM + 4 : BK + 4;   // padded row stride of the A tile
  constexpr int BS = B_NMAJOR ? BK + 4 : BN + 4;   // padded row stride of the B tile
  // The tiles (and the K groups' hand-over area) live in one LDS pool of this size: two
  // instantiations of the same size in one kernel (members of one batched launch whose
  // operand views differ) share it instead of adding up.
  constexpr int A_TILE = (A_KMAJOR ? BK : BM) * AS, B_TILE = (B_NMAJOR ? BN : BK) * BS;
  constexpr int TILES = KW * 2 * (A_TILE + B_TILE);
  float* const pool = lds_pool<TILES + (KW > 1 ? (KW - 1) * THREADS * TM * TN * 4 : 0)>();
  float (*As_)[2][A_TILE] = reinterpret_cast<float (*)[2][A_TILE]>(pool);
  float (*Bs_)[2][B_TILE] = reinterpret_cast<float (*)[2][B_TILE]>(pool + KW * 2 * A_TILE);

  // zid: the workgroup's z index within this launch (blockIdx.z, or its part
  // below the member index in a batched launch); (tx, ty): its output tile's column
  // and row (blockIdx.x and .y, or their XCD-grouped places).
  const uint32_t kz = SPLIT ? zid % chunks : 0u;
  const uint32_t bz = SPLIT ? zid / chunks : zid;
  const uint32_t kbeg0 = SPLIT ? kz * chunkK : 0u;
  const uint32_t kend0 = SPLIT ? min(K, kbeg0 + chunkK) : K;
  // K groups (KW > 1, for few-tile products: more wavefronts in flight per CU): group g
  // sums K range [kbeg0 + g·sub, kbeg0 + (g+1)·sub) of this workgroup's range, every
  // group the same number of slices (a short last range is zero-filled, so every
  // barrier is reached by all), and the groups' sums are added in order g = 0, 1, ...
  // after the loop. The split depends on (M, N, K, KW) alone, as everything else here.
  const int kg = KW == 1 ? 0 : static_cast<int>(threadIdx.x) / THREADS;
  const uint32_t sub = KW == 1 ? kend0 - kbeg0 : ((kend0 - kbeg0 + KW * BK - 1) / (KW * BK)) * BK;
  const uint32_t kbeg = kbeg0 + kg * sub;
  const uint32_t kend = min(kend0, kbeg + sub);
  float (*As)[A_TILE] = As_[kg];
  float (*Bs)[B_TILE] = Bs_[kg];
  const uint32_t m0 = ty * BM, n0 = tx * BN;
  const float* __restrict__ Ab = a_ptr + AV::batch(bz);
  const float* __restrict__ Bb = b_ptr + BV::batch(bz);

  const int tid = KW == 1 ? static_cast<int>(threadIdx.x) : static_cast<int>(threadIdx.x) % THREADS;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int t16 = lane & 15, q = lane >> 4;

  // Per-thread staging registers for one K slice.
  constexpr int A_VEC = (BM * BK / 4 + THREADS - 1) / THREADS;   // float4 loads per thread
  constexpr int B_VEC = (BK * BN / 4 + THREADS - 1) / THREADS;
  constexpr int A_SC = (BM * BK + THREADS - 1) / THREADS;        // scalar loads per thread
  constexpr int B_SC = (BK * BN + THREADS - 1) / THREADS;
  constexpr bool VA = AMODE != MODE_S, VB = BMODE != MODE_S;
  // Staging registers for a slice in flight: one set, or two for PF = 2 (the
  // global loads of slice k + 2 are issued while slice k is computed, so each
  // load has two slices' compute to arrive before it is stored to LDS).
  struct Stage {
    float4 ra[VA ? A_VEC : 1];
    float4 rb[VB ? B_VEC : 1];
    float sa[VA ? 1 : A_SC];
    float sb[VB ? 1 : B_SC];
  };
  Stage st0, st1;

  auto load_slice = [&](Stage& S, uint32_t k0) {
    float4* ra = S.ra;
    float4* rb = S.rb;
    float* sa = S.sa;
    float* sb = S.sb;
    if (AMODE == MODE_C) {
#pragma unroll
      for (int v = 0; v < A_VEC; ++v) {
        const int t = tid + v * THREADS;
        const uint32_t row = t / (BK / 4), kk = (t % (BK / 4)) * 4;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < BM * BK / 4 && m0 + row < M && k0 + kk < kend)
          x = *reinterpret_cast<const float4*>(Ab + vrow<AV>(m0 + row) + vcol<AV>(k0 + kk));
        ra[v] = x;
      }
    } else if (AMODE == MODE_R) {
#pragma unroll
      for (int v = 0; v < A_VEC; ++v) {
        const int t = tid + v * THREADS;
        const uint32_t kk = t / (BM / 4), row = (t % (BM / 4)) * 4;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < BM * BK / 4 && m0 + row < M && k0 + kk < kend)
          x = *reinterpret_cast<const float4*>(Ab + vcol<AV>(k0 + kk) + vrow<AV>(m0 + row));
        ra[v] = x;
      }
    } else {
#pragma unroll
      for (int v = 0; v < A_SC; ++v) {
        const int t = tid + v * THREADS;
        const uint32_t row = t / BK, kk = t % BK;
        float x = 0.f;
        if (t < BM * BK && m0 + row < M && k0 + kk < kend) x = Ab[vrow<AV>(m0 + row) + vcol<AV>(k0 + kk)];
        sa[v] = x;
      }
    }
    if (BMODE == MODE_C) {
#pragma unroll
      for (int v = 0; v < B_VEC; ++v) {
        const int t = tid + v * THREADS;
        const uint32_t kk = t / (BN / 4), c = (t % (BN / 4)) * 4;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < BK * BN / 4 && k0 + kk < kend && n0 + c < N)
          x = *reinterpret_cast<const float4*>(Bb + vrow<BV>(k0 + kk) + vcol<BV>(n0 + c));
        rb[v] = x;
      }
    } else if (BMODE == MODE_R) {
#pragma unroll
      for (int v = 0; v < B_VEC; ++v) {
        const int t = tid + v * THREADS;
        const uint32_t c = t / (BK / 4), kk = (t % (BK / 4)) * 4;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < BK * BN / 4 && k0 + kk < kend && n0 + c < N)
          x = *reinterpret_cast<const float4*>(Bb + vcol<BV>(n0 + c) + vrow<BV>(k0 + kk));
        rb[v] = x;
      }
    } else {
#pragma unroll
      for (int v = 0; v < B_SC; ++v) {
        const int t = tid + v * THREADS;
        const uint32_t kk = t / BN, c = t % BN;
        float x = 0.f;
        if (t < BK * BN && k0 + kk < kend && n0 + c < N) x = Bb[vrow<BV>(k0 + kk) + vcol<BV>(n0 + c)];
        sb[v] = x;
      }
    }
  };

  auto store_slice = [&](const Stage& S, int buf) {
    const float4* ra = S.ra;
    const float4* rb = S.rb;
    const float* sa = S.sa;
    const float* sb = S.sb;
    if (AMODE == MODE_C) {
#pragma unroll
      for (int v = 0; v < A_VEC; ++v) {
        const int t = tid + v * THREADS;
        if (t < BM * BK / 4) {
          const int row = t / (BK / 4), kk = (t % (BK / 4)) * 4;
          *reinterpret_cast<float4*>(&As[buf][row * AS + kk]) = vop<AV>(ra[v]);
        }
      }
    } else if (AMODE == MODE_R) {
#pragma unroll
      for (int v = 0; v < A_VEC; ++v) {
        const int t = tid + v * THREADS;
        if (t < BM * BK / 4) {
          const int kk = t / (BM / 4), row = (t % (BM / 4)) * 4;
          *reinterpret_cast<float4*>(&As[buf][kk * AS + row]) = vop<AV>(ra[v]);
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < A_SC; ++v) {
        const int t = tid + v * THREADS;
        if (t < BM * BK) As[buf][(t / BK) * AS + (t % BK)] = vop<AV>(sa[v]);
      }
    }
    if (BMODE == MODE_C) {
#pragma unroll
      for (int v = 0; v < B_VEC; ++v) {
        const int t = tid + v * THREADS;
        if (t < BK * BN / 4) {
          const int kk = t / (BN / 4), c = (t % (BN / 4)) * 4;
          *reinterpret_cast<float4*>(&Bs[buf][kk * BS + c]) = vop<BV>(rb[v]);
        }
      }
    } else if (BMODE == MODE_R) {
#pragma unroll
      for (int v = 0; v < B_VEC; ++v) {
        const int t = tid + v * THREADS;
        if (t < BK * BN / 4) {
          const int c = t / (BK / 4), kk = (t % (BK / 4)) * 4;
          *reinterpret_cast<float4*>(&Bs[buf][c * BS + kk]) = vop<BV>(rb[v]);
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < B_SC; ++v) {
        const int t = tid + v * THREADS;
        if (t < BK * BN) Bs[buf][(t / BN) * BS + (t % BN)] = vop<BV>(sb[v]);
      }
    }
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  // One K slice from LDS buffer `cur` into the accumulators. The MFMA takes the
  // B value as its first operand and the A value as its second, so it computes
  // the tile transposed: lane (t16, q) holds row t16, columns 4q .. 4q+3 of each
  // 16 x 16 output tile — four consecutive outputs, stored with one 128-bit write.
  auto compute = [&](const int cur) {
    // PRIO: a wavefront in its MFMA phase is issued ahead of wavefronts loading or storing.
    if (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int g = 0; g < BK / 16; ++g) {
      // A values of this lane for every row tile: k = 16g + 4q .. 16g + 4q + 3 of the slice.
      float4 av[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * TM * 16 + i * 16 + t16;
        if (A_KMAJOR) {
          const float* a = &As[cur][(16 * g + 4 * q) * AS + row];
          av[i] = make_float4(a[0], a[AS], a[2 * AS], a[3 * AS]);
        } else {
          av[i] = *reinterpret_cast<const float4*>(&As[cur][row * AS + 16 * g + 4 * q]);
        }
      }
      // B values of a column-major tile: the same 4 k values of each column tile at once.
      float4 bq[B_NMAJOR ? TN : 1];
      if (B_NMAJOR) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bq[j] = *reinterpret_cast<const float4*>(&Bs[cur][(wn * TN * 16 + j * 16 + t16) * BS + 16 * g + 4 * q]);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float bv[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bv[j] = B_NMAJOR ? lane4(bq[j], s) : Bs[cur][(16 * g + 4 * q + s) * BS + wn * TN * 16 + j * 16 + t16];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const float a = lane4(av[i], s);
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[j], a, acc[i][j], 0, 0, 0);
        }
      }
    }
    if (PRIO) __builtin_amdgcn_s_setprio(0);
  };

  const uint32_t slices = KW == 1 ? (kend - kbeg + BK - 1) / BK : sub / BK;
  load_slice(st0, kbeg);
  store_slice(st0, 0);
  if (PF == 2 && slices > 1) load_slice(st1, kbeg + BK);
  __syncthreads();
  if (PF == 1) {
    for (uint32_t ks = 0; ks < slices; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < slices) load_slice(st0, kbeg + (ks + 1) * BK);
      compute(cur);
      if (ks + 1 < slices) store_slice(st0, cur ^ 1);
      __syncthreads();
    }
  } else {
    // Slice s travels in set s & 1 and is computed from LDS buffer s & 1; the loop
    // is unrolled by two so that every set and buffer index is a constant.
    for (uint32_t ks = 0; ks < slices; ks += 2) {
      if (ks + 2 < slices) load_slice(st0, kbeg + (ks + 2) * BK);
      compute(0);
      if (ks + 1 < slices) store_slice(st1, 1);
      __syncthreads();
      if (ks + 1 >= slices) break;
      if (ks + 3 < slices) load_slice(st1, kbeg + (ks + 3) * BK);
      compute(1);
      if (ks + 2 < slices) store_slice(st0, 0);
      __syncthreads();
    }
  }

  if constexpr (KW > 1) {
    // Groups 1 .. KW-1 hand their sums to group 0 through LDS, which adds them in
    // group order; group 0 alone stores (no barrier follows).
    f4 (*red)[THREADS][TM * TN] = reinterpret_cast<f4 (*)[THREADS][TM * TN]>(pool + TILES);
    if (kg > 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) red[kg - 1][tid][i * TN + j] = acc[i][j];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KW; ++g)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] += red[g - 1][tid][i * TN + j];
  }

  // Store: lane (t16, q) of tile (i, j) holds row t16, columns 4q .. 4q+3.
  constexpr bool VOUT = true;
  if (SPLIT) {
    float* __restrict__ part = A.ws + (size_t)(kz * batch + bz) * M * N;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const uint32_t row = m0 + wm * TM * 16 + i * 16 + t16;
        const uint32_t col0 = n0 + wn * TN * 16 + j * 16 + 4 * q;
        if (row >= M) continue;
        if (N % 4 == 0 && VOUT) {
          if (col0 < N) *reinterpret_cast<f4*>(part + (size_t)row * N + col0) = acc[i][j];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (col0 + r < N) part[(size_t)row * N + col0 + r] = acc[i][j][r];
        }
      }
    return;
  }
  // Epilogue: the fused body on each accumulator element, then the store.
  const Epi epi;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint32_t row = m0 + wm * TM * 16 + i * 16 + t16;
      const uint32_t col0 = n0 + wn * TN * 16 + j * 16 + 4 * q;
      if (row >= M) continue;
      const uint32_t o = (bz * M + row) * N + col0;
      if (N % 4 == 0 && VOUT) {
        if (col0 < N) {
          f4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = epi(A, o + r, acc[i][j][r]);
          *reinterpret_cast<f4*>(A.out + o) = v;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col0 + r < N) A.out[o + r] = epi(A, o + r, acc[i][j][r]);
      }
    }
  }
}

// Output element j of a split-K matmul's product: its chunks' partial sums from the
// workspace, added in chunk order — the value gemm_splitk_reduce forms for j itself.
// An epilogue that reads the product at another element's index (a recomputed
// broadcast or transpose of it) reads it here.
template <class Args>
__device__ __forceinline__ float gemm_product_at(const Args& A, uint32_t j, uint32_t total, uint32_t chunks) {
  float acc = A.ws[j];
  for (uint32_t c = 1; c < chunks; ++c) acc += A.ws[(size_t)c * total + j];
  return acc;
}

// The second half of a split-K matmul: out[i] = Epi(A, i, Σ_chunk ws[chunk·total + i]),
// the chunks summed in order; `total` = batch·M·N. Four outputs per thread when N % 4 == 0.
template <bool VEC, class Epi, class Args>
__device__ __forceinline__ void gemm_splitk_reduce(const Args& A, uint32_t total, uint32_t chunks) {
  const Epi epi;
  const uint32_t stride = gridDim.x * blockDim.x;
  if (VEC) {
    const uint32_t nv = total >> 2;
    const f4* __restrict__ ws = reinterpret_cast<const f4*>(A.ws);
    for (uint32_t v = blockIdx.x * blockDim.x + threadIdx.x; v < nv; v += stride) {
      f4 acc = ws[v];
      for (uint32_t c = 1; c < chunks; ++c) acc += ws[(size_t)c * nv + v];
      f4 o;
#pragma unroll
      for (int l = 0; l < 4; ++l) o[l] = epi(A, 4 * v + l, acc[l]);
      reinterpret_cast<f4*>(A.out)[v] = o;
    }
  } else {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
      float acc = A.ws[i];
      for (uint32_t c = 1; c < chunks; ++c) acc += A.ws[(size_t)c * total + i];
      A.out[i] = epi(A, i, acc);
    }
  }
}

}  // namespace tcmi
