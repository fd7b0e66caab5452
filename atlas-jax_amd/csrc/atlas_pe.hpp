// Wave-level Polar-Express (Newton-Schulz with the Polar-Express coefficients)
// on one D x E matrix (D <= E, both multiples of 32) held in registers.
//
// Semantics: atlas_jax/memory_layer.py:43-71 / kernels/triton_pe.py:26-69,
// wide branch: X <- X / (sqrt(sum X^2 + eps) * 1.01 + 1e-6), then per step
//   A = X X^T,  B = b A + c A^2,  X <- a X + B X.
// Tall inputs are handled by the caller passing X^T (PE(X)^T = PE(X^T) since
// (X X^T)^j X = X (X^T X)^j).
//
// X lives in registers as 32x32 MFMA C-layout tiles (fp32 master copy).
// fp16 matrix-core path (ModeF16), per step:
//   X^T  one MFMA per 32x16 block against the identity: a C-layout tile used
//        as the A operand supplies its transpose, so (X tile)^T * I lands in
//        C layout with the contraction index of the Gram (the columns of X)
//        along its rows -- the Gram then takes both operands straight from
//        registers, with no LDS round trip;
//   A  = X X^T;
//   B  = c A^2 + b A   accumulated onto (b/c) A in fp32 and scaled by c when
//        converted, so the b A term is never rounded to fp16 (A and A^2 are
//        symmetric: their C-layout tiles serve as operands as they are);
//   X <- a X + B X     computed as X' = a X (fp32, while the B products run)
//        then X' + (B/a) X', with X''s own C-layout tiles as the B operand.
// fp32 path (ModeF32): the Gram passes each 32-column block of X through the
// wave's private LDS scratch instead.
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

// Keeps the scheduler from hoisting the next column block's conversions above
// the current block's products (which would raise register pressure past the
// arch VGPR file).
#define PE_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// fp16 matrix-core Polar-Express (see the header comment); no LDS.
template <int D, int E>
__device__ __forceinline__ void polar_express_wave_f16(f32x16 (&X)[D / 32][E / 32], int ns, float norm_eps) {
  constexpr int TI = D / 32, TJ = E / 32;
  using M = ModeF16;
  using frag = M::frag;
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

  // identity B operand (same k assignment as a C-layout tile's fragments)
  frag idf[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) idf[kb] = M::identity(kb, c, h);

  for (int st = 0; st < ns; ++st) {
    const float pa = kPE[st][0], pb = kPE[st][1], pc = kPE[st][2];

    // ---- Gram A = X X^T over the column blocks J -------------------------
    f32x16 A[TI][TI];
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = zero16();
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      frag th[TI][2];   // (X[I][J])^T in fp16, as operand fragments
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        f32x16 t = zero16();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) t = M::mma(M::from_c(X[I][J], kb), idf[kb], t);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) th[I][kb] = M::from_c(t, kb);
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = M::mma(th[I][kb], th[I2][kb], A[I][I2]);
      PE_SCHED_FENCE();
    }

    // ---- B = c A^2 + b A ---------------------------------------------------
    frag af[TI][TI][2];
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) af[K][I][kb] = M::from_c(A[K][I], kb);
    const float bc = pb / pc;
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) A[I][I2] *= bc;
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = M::mma(af[K][I][kb], af[K][I2][kb], A[I][I2]);
    // X <- a X while those products run; then X + (B/a) X equals the step's
    // a X + B X, with the operand taken from the scaled X.
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J) X[I][J] *= pa;
    // A now holds B / c; its operand form (times c / a) reuses af
    const float ca = pc / pa;
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        const f32x16 t = A[K][I] * ca;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) af[K][I][kb] = M::from_c(t, kb);
      }

    // ---- X <- X + (B / a) X ------------------------------------------------
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      frag xf[TI][2];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) xf[K][kb] = M::from_c(X[K][J], kb);
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int I = 0; I < TI; ++I) X[I][J] = M::mma(af[K][I][kb], xf[K][kb], X[I][J]);
      PE_SCHED_FENCE();
    }
  }
}

template <class M, int D, int E>
__device__ __forceinline__ void polar_express_wave(f32x16 (&X)[D / 32][E / 32], int ns,
                                                   float norm_eps,
                                                   typename M::elem* scr) {
  if constexpr (sizeof(typename M::elem) == 2) {
    (void)scr;
    polar_express_wave_f16<D, E>(X, ns, norm_eps);
    return;
  }
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
