// Wave-level Polar-Express (Newton-Schulz with the Polar-Express coefficients)
// on one D x E matrix (D <= E, both multiples of 32) held in registers.
//
// Semantics: atlas_jax/memory_layer.py:43-71 / kernels/triton_pe.py:26-69,
// wide branch: X <- X / (sqrt(sum X^2 + eps) * 1.01 + 1e-6), then per step
//   A = X X^T,  B = b A + c A^2,  X <- a X + B X.
// Tall inputs are handled by the caller passing X^T (PE(X)^T = PE(X^T) since
// (X X^T)^j X = X (X^T X)^j).
//
// Per step on the matrix cores:
//   A  = X X^T       each 32-column block of X passes once through the wave's
//                    private LDS scratch (written in C-layout order, read back
//                    row-contiguous), since the Gram contracts over columns;
//   B  = A (c A + b I)   one product of the symmetric A with N = cA + bI, both
//                    taken straight from A's C-layout tiles (A and N commute
//                    and are symmetric, so no transpose is needed);
//   X <- a X + B X   X's own C-layout tiles are the B operand; a X stays fp32.
// X lives in arch VGPRs; A and B are MFMA accumulators only touched by VALU
// when converted to operands, so they can sit in the accumulator registers.
#pragma once

#include "atlas_common.hpp"

namespace atlas {

// Row stride (elements) of the per-wave scratch used for the Gram transpose.
template <class M>
struct Scr {
  static constexpr int SP = (sizeof(typename M::elem) == 2) ? 40 : 33;
  template <int D>
  static constexpr int elems() { return D * SP; }
};

template <class M, int TI, int TJ>
__device__ __forceinline__ void scr_put_cols(const f32x16 (&X)[TI][TJ], int J,
                                             typename M::elem* scr) {
  constexpr int SP = Scr<M>::SP;
  const int c = lane_id() & 31, h = lane_id() >> 5;
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      scr[(32 * I + crow(r, h)) * SP + c] = M::to_elem(X[I][J][r]);
}

template <class M, int D, int E>
__device__ __forceinline__ void polar_express_wave(f32x16 (&X)[D / 32][E / 32], int ns,
                                                   float norm_eps,
                                                   typename M::elem* scr) {
  constexpr int TI = D / 32, TJ = E / 32, KPT = M::KPT;
  constexpr int SP = Scr<M>::SP;
  using frag = typename M::frag;
  const int c = lane_id() & 31, h = lane_id() >> 5;

  float ss = 0.f;
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J)
#pragma unroll
      for (int r = 0; r < 16; ++r) ss += X[I][J][r] * X[I][J][r];
  ss = wave_sum(ss);
  const float inv = 1.f / (sqrtf(ss + norm_eps) * 1.01f + 1e-6f);
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J) X[I][J] *= inv;

  for (int st = 0; st < ns; ++st) {
    const float pa = kPE[st][0], pb = kPE[st][1], pc = kPE[st][2];

    // ---- Gram A = X X^T -------------------------------------------------
    f32x16 A[TI][TI];
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = zero16();
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      scr_put_cols<M, TI, TJ>(X, J, scr);
#pragma unroll
      for (int kb = 0; kb < KPT; ++kb) {
        frag fr[TI];
#pragma unroll
        for (int I = 0; I < TI; ++I) fr[I] = M::ld_contig(scr + (32 * I + c) * SP, kb, h);
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = M::mma(fr[I], fr[I2], A[I][I2]);
      }
    }

    // ---- B = A (c A + b I) ------------------------------------------------
    // Af[K][I] = tile (K, I) of A as operand; Nf likewise for N = cA + bI,
    // formed in fp32 (the coefficients stay exact) before conversion.
    frag Af[TI][TI][KPT], Nf[TI][TI][KPT];
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        const f32x16 t = A[K][I];
        f32x16 nt = t * pc;
        if (K == I) {
#pragma unroll
          for (int r = 0; r < 16; ++r) nt[r] += (crow(r, h) == c) ? pb : 0.f;
        }
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) {
          Af[K][I][kb] = M::from_c(t, kb);
          Nf[K][I][kb] = M::from_c(nt, kb);
        }
      }
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = zero16();
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int kb = 0; kb < KPT; ++kb)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2)
            A[I][I2] = M::mma(Af[K][I][kb], Nf[K][I2][kb], A[I][I2]);
    // A now holds B; its operand form reuses Af
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) Af[K][I][kb] = M::from_c(A[K][I], kb);

    // ---- X <- a X + B X ---------------------------------------------------
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      frag xf[TI][KPT];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) xf[K][kb] = M::from_c(X[K][J], kb);
#pragma unroll
      for (int I = 0; I < TI; ++I) X[I][J] *= pa;
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb)
#pragma unroll
          for (int I = 0; I < TI; ++I)
            X[I][J] = M::mma(Af[K][I][kb], xf[K][kb], X[I][J]);
    }
  }
}

}  // namespace atlas
