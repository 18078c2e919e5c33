// Fused attention on CDNA4 matrix cores: out = P · V, P = body(Q · Kᵀ), one
// kernel instead of three launches (scores matmul, rowwise softmax, P·V).
//
// Q [batch, TQ, DH], Kt [batch, DH, TK] and V [batch, TK, DV] are strided views
// of their buffers (tcmi_gemm.h's MODE_C / MODE_R / MODE_S), so the head split
// and the transposed keys are read in place. `body` is the generated score
// transformation and row reduction (scale, mask, the softmax composite, or any
// rowwise body the fusion pass grew): it runs on the scores while they are in
// registers, and its result feeds the second product without leaving them.
//
// A workgroup of W wavefronts (W = TQ / 16 rounded up, at most 8) owns one batch
// index and 16·W query rows, 16 per wavefront. The batch index's whole K and V
// are staged once in LDS (padded rows, every 128-bit access on disjoint banks)
// and shared by the W wavefronts, so up to 128 queries read them from memory once.
// Per wavefront, with lane = 16·q + t (t in 0..15) of a 16x16x4 MFMA:
//   scores  sacc[jt] += mfma(K value, Q value): the transposed-accumulator form
//           of tcmi_gemm.h, so lane (t, q) holds S[row t][key 16·jt + 4q + r],
//           r = 0..3 (one row's keys spread over the four lanes t + 16q);
//   body    per element on those registers; a row reduction is the lane's own
//           partial over its keys, then quad16_reduce across the four lanes;
//   output  oacc[jn] += mfma(V value, P value): lane (t, q)'s P values for key
//           part g are exactly the MFMA's A operand for k = 16g + 4q + s, so P
//           goes from the score registers into the second product directly.
// Both products walk their k index 16 at a time, s inner (the order of
// tcmi_gemm.h), so the scores equal a tcmi_gemm.h product's bit for bit.

#pragma once

#include "tcmi_gemm.h"

namespace tcmi {

// Padded LDS geometry of the key and value tiles.
template <int TK, int DH, int DV>
struct AttnTiles {
  static constexpr int NT = (TK + 15) / 16;    // key tiles of 16 (the scores' columns, P·V's k parts)
  static constexpr int DH16 = (DH + 15) / 16;  // parts of 16 of the scores' k (head size)
  static constexpr int DV16 = (DV + 15) / 16;  // output column tiles
  static constexpr int ROWS = NT * 16;         // key rows staged (zero past TK)
  static constexpr int KS = DH16 * 16 + 4;     // row stride of Ks[key][d]
  static constexpr int VS = DV16 * 16 + 4;     // row stride of Vs[key][d]
};

// Staging of one operand tile (K as Ks[key][d], V as Vs[key][d]) through
// registers: load() issues every global load of this thread's share at once
// (128-bit where the layout allows) into `r`, store() writes `r` to LDS.
// Splitting the two lets the V loads fly while the scores are computed. The
// registers are native 4-vectors, which the compiler keeps in VGPRs (an array
// of the HIP float4 struct, live across the scores, was placed in scratch).
// View V_ element (b, r, c) is at V_::batch(b) + r·SR + c·SC; the tile's LDS
// row is `key`, its column `d`: for K (Kt's view) key = c and d = r, for V
// key = r and d = c.
template <int KEYS, int D, int STRIDE, int MODE, bool KEY_IS_C, class V_, int THREADS>
struct AttnStage {
  // 128-bit along d (one 128-bit LDS store), along the keys (four 32-bit stores), or per element.
  static constexpr bool ALONG_D = MODE != MODE_S && ((MODE == MODE_R) == KEY_IS_C);
  static constexpr int VEC = MODE != MODE_S ? 4 : 1;
  static constexpr int TOTAL = KEYS * D / VEC;
  static constexpr int PER = (TOTAL + THREADS - 1) / THREADS;

  static __device__ __forceinline__ void load(f4 (&r)[PER], const float* __restrict__ base, uint32_t b) {
    const float* __restrict__ p = base + V_::batch(b);
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int t = threadIdx.x + v * THREADS;
      if (TOTAL % THREADS != 0 && t >= TOTAL) continue;
      if (MODE == MODE_S) {
        const int key = t / D, d = t % D;
        r[v][0] = KEY_IS_C ? p[(size_t)d * V_::SR + (size_t)key * V_::SC] : p[(size_t)key * V_::SR + (size_t)d * V_::SC];
      } else if (ALONG_D) {
        const int key = t / (D / 4), d = (t % (D / 4)) * 4;
        r[v] = *reinterpret_cast<const f4*>(p + (size_t)key * (KEY_IS_C ? V_::SC : V_::SR) + d);
      } else {
        const int d = t / (KEYS / 4), key = (t % (KEYS / 4)) * 4;
        r[v] = *reinterpret_cast<const f4*>(p + (size_t)d * (KEY_IS_C ? V_::SR : V_::SC) + key);
      }
    }
  }

  static __device__ __forceinline__ void store(const f4 (&r)[PER], float* tile) {
#pragma unroll
    for (int v = 0; v < PER; ++v) {
      const int t = threadIdx.x + v * THREADS;
      if (TOTAL % THREADS != 0 && t >= TOTAL) continue;
      if (MODE == MODE_S) {
        tile[(t / D) * STRIDE + t % D] = r[v][0];
      } else if (ALONG_D) {
        const int key = t / (D / 4), d = (t % (D / 4)) * 4;
        *reinterpret_cast<f4*>(&tile[key * STRIDE + d]) = r[v];
      } else {
        const int d = t / (KEYS / 4), key = (t % (KEYS / 4)) * 4;
        tile[(key + 0) * STRIDE + d] = r[v][0];
        tile[(key + 1) * STRIDE + d] = r[v][1];
        tile[(key + 2) * STRIDE + d] = r[v][2];
        tile[(key + 3) * STRIDE + d] = r[v][3];
      }
    }
  }
};

// Zero the padding of the key and value tiles (keys past TK, d past the head sizes),
// which the products read; a barrier follows before any tile is written.
template <int TK, int DH, int DV, int THREADS>
__device__ __forceinline__ void attn_zero_padding(float* Ks, float* Vs) {
  using G = AttnTiles<TK, DH, DV>;
  const int tid = threadIdx.x;
  if (TK % 16 != 0 || DH % 16 != 0) {
    for (int t = tid; t < G::ROWS * G::KS; t += THREADS) Ks[t] = 0.f;
  }
  if (TK % 16 != 0 || DV % 16 != 0) {
    for (int t = tid; t < G::ROWS * G::VS; t += THREADS) Vs[t] = 0.f;
  }
  if (TK % 16 != 0 || DH % 16 != 0 || DV % 16 != 0) __syncthreads();
}

// This lane's Q values: qf[g][s] = Q[b][row][16g + 4q + s] (0 past DH, or when row >= TQ).
template <int TQ, int DH, int DH16, int QMODE, class QV>
__device__ __forceinline__ void attn_q(f4 (&qf)[DH16], const float* __restrict__ qp, uint32_t b, uint32_t row,
                                       int q) {
  const float* __restrict__ qb = qp + QV::batch(b);
#pragma unroll
  for (int g = 0; g < DH16; ++g) {
    f4 x = f4{0.f, 0.f, 0.f, 0.f};
    const int d0 = 16 * g + 4 * q;
    if (row < TQ) {
      if (QMODE == MODE_C && DH % 4 == 0) {
        if (d0 < DH) {
          const float4 v = *reinterpret_cast<const float4*>(qb + (size_t)row * QV::SR + d0);
          x = f4{v.x, v.y, v.z, v.w};
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (d0 + s < DH) x[s] = qb[(size_t)row * QV::SR + (size_t)(d0 + s) * QV::SC];
      }
    }
    qf[g] = x;
  }
}

// Scores: sacc[jt] = Σ_d K[16jt + ·][d] ⊗ Q[·][d] as 16x16 tiles, transposed accumulator.
template <int NT, int DH16, int KS>
__device__ __forceinline__ void attn_scores(f4 (&sacc)[NT], const f4 (&qf)[DH16], const float* Ks, int t16, int q) {
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) sacc[jt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int g = 0; g < DH16; ++g) {
    float4 kq[NT];
#pragma unroll
    for (int jt = 0; jt < NT; ++jt)
      kq[jt] = *reinterpret_cast<const float4*>(&Ks[(16 * jt + t16) * KS + 16 * g + 4 * q]);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int jt = 0; jt < NT; ++jt)
        sacc[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(lane4(kq[jt], s), qf[g][s], sacc[jt], 0, 0, 0);
  }
}

// Output: oacc[jn] = Σ_key V[key][16jn + ·] ⊗ P[·][key], P in the scores' register layout.
template <int NT, int DV16, int VS>
__device__ __forceinline__ void attn_pv(f4 (&oacc)[DV16], const f4 (&p)[NT], const float* Vs, int t16, int q) {
#pragma unroll
  for (int jn = 0; jn < DV16; ++jn) oacc[jn] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int g = 0; g < NT; ++g)
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int jn = 0; jn < DV16; ++jn)
        oacc[jn] = __builtin_amdgcn_mfma_f32_16x16x4f32(Vs[(16 * g + 4 * q + s) * VS + 16 * jn + t16], p[g][s],
                                                        oacc[jn], 0, 0, 0);
}

// Store: lane (t, q) of column tile jn holds out[b][row][16jn + 4q .. 16jn + 4q + 3].
template <int TQ, int DV, int DV16>
__device__ __forceinline__ void attn_store(float* __restrict__ out, const f4 (&oacc)[DV16], uint32_t b, uint32_t row,
                                           int q) {
  if (row >= TQ) return;
  float* __restrict__ o = out + ((size_t)b * TQ + row) * DV;
#pragma unroll
  for (int jn = 0; jn < DV16; ++jn) {
    const int c0 = 16 * jn + 4 * q;
    if (DV % 4 == 0) {
      if (c0 < DV) *reinterpret_cast<f4*>(o + c0) = oacc[jn];
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (c0 + r < DV) o[c0 + r] = oacc[jn][r];
    }
  }
}

// ---- the gradient (fusion/attention.js, fuseAttentionTraining) --------------------------
//
// dQ = dS·K, dK = dSᵀ·Q and dV = Pᵀ·dO of one attention, with the scores S = Q·Kᵀ, P and
// dP = dO·Vᵀ recomputed: one workgroup per batch index holds all TQ query rows (16 per
// wavefront, W wavefronts) and all TK keys. K and V are staged in LDS; each wavefront
// forms its rows' S and dP in registers (attn_scores), the generated body turns them into
// dS and P there, and dQ takes dS as the A operand of its product with K straight from
// the registers (attn_pv). dK and dV sum over the queries, which the wavefronts hold one
// row per lane: dS (then P) is written to LDS as a [query][key] tile beside Q (then dO),
// and each wavefront forms the rows of 16 keys at a time, reading the tile down its
// columns. Every product walks its k index in the order of tcmi_gemm.h (16 at a time, 4
// per MFMA step), so each output is computed the same way whichever others a kernel forms.

template <int TQ, int TK, int DH, int DV>
struct AttnGradTiles {
  static constexpr int W = (TQ + 15) / 16;        // wavefronts: one per 16 query rows
  static constexpr int NT = (TK + 15) / 16;       // key tiles of 16
  static constexpr int DH16 = (DH + 15) / 16;
  static constexpr int DV16 = (DV + 15) / 16;
  static constexpr int ROWS = NT * 16;            // keys staged (zero past TK)
  static constexpr int QROWS = W * 16;            // query rows staged (zero past TQ)
  static constexpr int KS = DH16 * 16 + 4;        // Ks[key][d]
  static constexpr int VS = DV16 * 16 + 4;        // Vs[key][d]
  static constexpr int TS = ROWS + 4;             // Ts[query][key]: dS, then P
  static constexpr int QS = DH16 * 16 + 4;        // Qs[query][d]
  static constexpr int OS = DV16 * 16 + 4;        // Os[query][d] (dO)
  static constexpr int PHASE1 = ROWS * KS + ROWS * VS;
  static constexpr int PHASE2 = QROWS * TS + QROWS * QS;
  static constexpr int PHASE3 = QROWS * TS + QROWS * OS;
  static constexpr int POOL = PHASE1 > PHASE2 ? (PHASE1 > PHASE3 ? PHASE1 : PHASE3) : (PHASE2 > PHASE3 ? PHASE2 : PHASE3);
  static_assert(W >= 1 && W <= 8, "the gradient kernel holds at most 128 query rows");
};

// Registers in the scores' layout (lane (t, q): row 16·wave + t, keys 16jt + 4q .. +3)
// written to a [row][key] tile of row stride TS.
template <int NT, int TS>
__device__ __forceinline__ void attn_rows_to_lds(float* tile, const f4 (&v)[NT], int wave, int t16, int q) {
  float* row = tile + (16 * wave + t16) * TS + 4 * q;
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) *reinterpret_cast<f4*>(row + 16 * jt) = v[jt];
}

// A lane's operand fragments (row 16·wave + t, columns 16g + 4q .. +3) written to a
// [row][column] tile of row stride S.
template <int D16, int S>
__device__ __forceinline__ void attn_frags_to_lds(float* tile, const f4 (&v)[D16], int wave, int t16, int q) {
  float* row = tile + (16 * wave + t16) * S + 4 * q;
#pragma unroll
  for (int g = 0; g < D16; ++g) *reinterpret_cast<f4*>(row + 16 * g) = v[g];
}

// out[b][key][d] = Σ_query T[query][key] · X[query][d] for the key tiles of this wavefront
// (kt = wave, wave + W, ...): the A operand read down T's columns (lane (t, q) at step s:
// T[16g + 4q + s][16kt + t]), the B operand along X's rows, the queries 16 at a time.
template <int NT, int W, int D16, int TS, int XS, int TK, int D>
__device__ __forceinline__ void attn_grad_keys(float* __restrict__ out, const float* T, const float* X, uint32_t b,
                                               int wave, int t16, int q) {
  for (int kt = wave; kt < NT; kt += W) {
    f4 acc[D16];
#pragma unroll
    for (int jn = 0; jn < D16; ++jn) acc[jn] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < W; ++g) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int qr = 16 * g + 4 * q + s;
        const float a = T[qr * TS + 16 * kt + t16];
#pragma unroll
        for (int jn = 0; jn < D16; ++jn)
          acc[jn] = __builtin_amdgcn_mfma_f32_16x16x4f32(X[qr * XS + 16 * jn + t16], a, acc[jn], 0, 0, 0);
      }
    }
    const int key = 16 * kt + t16;
    if (key < TK) {
      float* __restrict__ o = out + ((size_t)b * TK + key) * D;
#pragma unroll
      for (int jn = 0; jn < D16; ++jn) {
        const int c0 = 16 * jn + 4 * q;
        if (D % 4 == 0) {
          if (c0 < D) *reinterpret_cast<f4*>(o + c0) = acc[jn];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (c0 + r < D) o[c0 + r] = acc[jn][r];
        }
      }
    }
  }
}

}  // namespace tcmi
