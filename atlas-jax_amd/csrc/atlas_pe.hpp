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

// Polar-Express in three pieces so that one matrix can also be split by
// columns over two waves (polar_express_pair): the Frobenius sum of squares,
// the Gram of the wave's own columns, and one step's update from the full
// Gram.
template <class M, int D, int E>
struct PEWave {
  static constexpr int TI = D / 32, TJ = E / 32, KPT = M::KPT;
  using frag = typename M::frag;
  using elem = typename M::elem;
  static constexpr bool F16 = sizeof(elem) == 2;

  __device__ __forceinline__ static float sumsq(const f32x16 (&X)[TI][TJ]) {
    float ss = 0.f;
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int r = 0; r < 16; ++r) ss += X[I][J][r] * X[I][J][r];
    return wave_sum(ss);
  }

  __device__ __forceinline__ static void scale(f32x16 (&X)[TI][TJ], float s) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J) X[I][J] *= s;
  }

  // A = X X^T over this wave's columns.  fp16: each 32-column block is
  // transposed on the matrix core ((X tile)^T * I); fp32: through the wave's
  // LDS scratch.
  __device__ __forceinline__ static void gram(const f32x16 (&X)[TI][TJ], f32x16 (&A)[TI][TI], elem* scr) {
    const int c = lane_id() & 31, h = lane_id() >> 5;
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = zero16();
    if constexpr (F16) {
      (void)scr;
      frag idf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) idf[kb] = M::identity(kb, c, h);
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
    } else {
      constexpr int SP = Scr<M>::SP;
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
    }
  }

  // X <- a X + (b A + c A^2) X for step st, from the full Gram A (consumed).
  __device__ __forceinline__ static void apply(f32x16 (&X)[TI][TJ], f32x16 (&A)[TI][TI], int st) {
    const int c = lane_id() & 31, h = lane_id() >> 5;
    if constexpr (F16) {
      const float pa = kPEd[st][0], bc = kPEd[st][1], ca = kPEd[st][2];
      // B = c A^2 + b A accumulated onto (b/c) A in fp32; X <- a X while those
      // products run; then X + (B/a) X with X's own tiles as the B operand.
      frag af[TI][TI][2];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) af[K][I][kb] = M::from_c(A[K][I], kb);
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
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J) X[I][J] *= pa;
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int I = 0; I < TI; ++I) {
          const f32x16 t = A[K][I] * ca;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) af[K][I][kb] = M::from_c(t, kb);
        }
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
    } else {
      const float pa = kPE[st][0], pb = kPE[st][1], pc = kPE[st][2];
      // B = A (c A + b I): A and N = cA + bI formed in fp32, both symmetric
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
            for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = M::mma(Af[K][I][kb], Nf[K][I2][kb], A[I][I2]);
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) Af[K][I][kb] = M::from_c(A[K][I], kb);
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
            for (int I = 0; I < TI; ++I) X[I][J] = M::mma(Af[K][I][kb], xf[K][kb], X[I][J]);
      }
    }
  }
};

// fp16 Gram with its operands transposed through LDS (gfx950 transposing
// reads) instead of on the matrix cores.  One wave, one D x E matrix (D <= E)
// in registers as 32x32 C-layout tiles: for each 32-column block J, X[:, J]
// goes to LDS in fp16 as rows e (row stride SP halves) and comes back as
// operand fragments with d along the lanes and e along the registers, so that
// A += X_J X_J^T takes both operands straight from those reads.  The step's
// update is PEWave::apply.  xs holds two blocks of 32 x SP halves per wave
// (block J uses half J % 2).
template <int D, int E>
struct PEWaveT {
  using M = ModeF16;
  using frag = f16x8;
  static constexpr int TI = D / 32, TJ = E / 32;
  static constexpr int SP = D + 12;                // LDS row stride (halves): 16-byte aligned rows at an odd 8-byte offset keep the staging writes free of bank conflicts
  static constexpr int BLOCK = 32 * SP;            // halves per staged block
  static constexpr int ELEMS = 2 * BLOCK;          // halves per wave

  // Per-lane offsets (halves) of the staging accesses: writes at wr_off()
  // + compile-time offsets, transposing reads at rd_off() + compile-time
  // offsets.  Callers pass them through opaque() so that the compiler forms
  // the addresses where they are used instead of keeping them live across
  // enclosing loops.
  __device__ __forceinline__ static int wr_off() { return (lane_id() & 31) * SP + 4 * (lane_id() >> 5); }
  __device__ __forceinline__ static int rd_off() {
    const int l = lane_id(), j = l & 15;
    return (8 * (l >> 5) + (j >> 2)) * SP + 16 * ((l >> 4) & 1) + 4 * (j & 3);
  }
  __device__ __forceinline__ static int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
  }

  // block J of X as fp16 rows e: lane (c, h) writes rows d = 32I + 8q + 4h + 0..3 of column c
  __device__ __forceinline__ static void put_block(const f32x16 (&X)[TI][TJ], int J, _Float16* buf, int wo) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f16x4*>(buf + wo + 32 * I + 8 * q) =
            f16x4{(_Float16)X[I][J][4 * q], (_Float16)X[I][J][4 * q + 1], (_Float16)X[I][J][4 * q + 2],
                  (_Float16)X[I][J][4 * q + 3]};
  }
  __device__ __forceinline__ static void put_block(const f32x16 (&X)[TI][TJ], int J, _Float16* buf) {
    put_block(X, J, buf, wr_off());
  }
  // Gram operand fragment (I, kb) of a staged block: lane l holds
  // X[32I + l % 32][16kb + 8(l / 32) + v], v = 0..7 (two transposing reads)
  __device__ __forceinline__ static frag get_tr(const _Float16* buf, int I, int kb, int ro) {
    const _Float16* p = buf + ro + 16 * kb * SP + 32 * I;
    const f16x4 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 4 * SP);
    return frag{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  __device__ __forceinline__ static frag get_tr(const _Float16* buf, int I, int kb) { return get_tr(buf, I, kb, rd_off()); }

  __device__ __forceinline__ static void gram(const f32x16 (&X)[TI][TJ], f32x16 (&A)[TI][TI], _Float16* xs) {
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      _Float16* buf = xs + (J & 1) * BLOCK;
      put_block(X, J, buf);
      frag th[TI][2];
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) th[I][kb] = get_tr(buf, I, kb);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2)
            A[I][I2] = M::mma(th[I][kb], th[I2][kb], (J == 0 && kb == 0) ? zero16() : A[I][I2]);
    }
  }

  // X_s <- X_s + rho (kappa G + G^2) X_s for step st (kPEt), from the Gram G
  // of X_s (consumed).  G and G^2 are symmetric: their C tiles serve as
  // operands as they are; X_s's own tiles are the B operand of the last
  // product, whose accumulator starts from X_s.
  __device__ __forceinline__ static void apply_scaled(f32x16 (&X)[TI][TJ], f32x16 (&A)[TI][TI], int st) {
    const float kap = kPEt[st][0], rho = kPEt[st][1];
    frag af[TI][TI][2];
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) af[K][I][kb] = M::from_c(A[K][I], kb);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) A[I][I2] *= kap;
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2) A[I][I2] = M::mma(af[K][I][kb], af[K][I2][kb], A[I][I2]);
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        const f32x16 t = A[K][I] * rho;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) af[K][I][kb] = M::from_c(t, kb);
      }
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      frag xf[TI][2];
#pragma unroll
      for (int K = 0; K < TI; ++K) {
        // converted again rather than kept from the Gram's staging (holding
        // all of X in fp16 across the step exceeds the register file)
        asm volatile("" : "+v"(X[K][J]));
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) xf[K][kb] = M::from_c(X[K][J], kb);
      }
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int I = 0; I < TI; ++I) X[I][J] = M::mma(af[K][I][kb], xf[K][kb], X[I][J]);
    }
    // One scheduling region for the whole update, each MFMA followed by two
    // VALU instructions: the conversions and scalings then issue in the
    // shadow of the matrix-core work instead of between dependent groups
    // (measured 9 % less Polar-Express time than block-wise scheduling).
#pragma unroll
    for (int i = 0; i < TI * TI * 4 + TI * TI * 2 * TJ; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // 2 VALU
    }
  }

  __device__ __forceinline__ static void read_block(frag (&th)[TI][2], const _Float16* buf, int ro) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) th[I][kb] = get_tr(buf, I, kb, ro);
  }

  // ---- symmetric step (D = 64): upper tiles only ---------------------------
  // G and kappa G + G^2 are symmetric, so only their tiles (0,0), (0,1) and
  // (1,1) are formed (24 instead of 32 Gram products and 12 instead of 16 for
  // G^2 per step).  The operand fragments of tile (1,0) -- lane = column d0
  // of block 0, k = rows d1 of block 1 in the C-layout k-slot order -- are
  // the transpose of tile (0,1): it is written to the staging area as fp16
  // rows d1 (as put_block writes X) and read back with transposing reads
  // whose row offsets follow the k-slot order (lo rows 16kb + 4h + 0..3, hi
  // rows +8) instead of the contiguous order of get_tr.  Fewer matrix-core
  // products per step draw less power: at one wave per SIMD the step takes
  // the same cycles, at a higher sustained clock.
  __device__ __forceinline__ static int rd_off_ks() {
    const int l = lane_id(), j = l & 15;
    return (4 * (l >> 5) + (j >> 2)) * SP + 16 * ((l >> 4) & 1) + 4 * (j & 3);
  }
  __device__ __forceinline__ static frag get_tr_ks(const _Float16* buf, int kb, int ro) {
    const _Float16* p = buf + ro + 16 * kb * SP;
    const f16x4 lo = lds_read_tr16(p), hi = lds_read_tr16(p + 8 * SP);
    return frag{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  // fp16(s * t) for C-layout tile t as rows = its columns: buf[c][crow(r, h)]
  __device__ __forceinline__ static void put_tile(const f32x16& t, float s, _Float16* buf, int wo) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f16x4*>(buf + wo + 8 * q) =
          f16x4{(_Float16)(t[4 * q] * s), (_Float16)(t[4 * q + 1] * s), (_Float16)(t[4 * q + 2] * s),
                (_Float16)(t[4 * q + 3] * s)};
  }

  // Gram of X: with TI == 2 only the tiles (I, I2 >= I) (A[1][0] is left
  // unset); otherwise as gram.  NB staging blocks at xs: with NB == 1 every
  // column block goes through the same one (block J + 1's writes are ordered
  // after block J's reads: they may alias, and LDS operations of one wave
  // complete in order).
  template <int NB = 2>
  __device__ __forceinline__ static void gram_sym(const f32x16 (&X)[TI][TJ], f32x16 (&A)[TI][TI], _Float16* xs) {
    static_assert(NB == 1 || NB == 2, "one or two staging blocks");
    if constexpr (TI != 2) {
      static_assert(NB == 2, "the generic Gram double-buffers its staging");
      gram(X, A, xs);
    } else {
#pragma unroll
      for (int J = 0; J < TJ; ++J) {
        _Float16* buf = xs + (NB == 2 ? (J & 1) * BLOCK : 0);
        put_block(X, J, buf);
        frag th[TI][2];
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) th[I][kb] = get_tr(buf, I, kb);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int I = 0; I < TI; ++I)
#pragma unroll
            for (int I2 = I; I2 < TI; ++I2)
              A[I][I2] = M::mma(th[I][kb], th[I2][kb], (J == 0 && kb == 0) ? zero16() : A[I][I2]);
      }
    }
  }

  // apply_scaled from the upper tiles of G (gram_sym); xs is the staging area
  // of NB blocks (free once the Gram's reads have been issued: LDS
  // operations of one wave complete in order).
  template <int NB = 2>
  __device__ __forceinline__ static void apply_sym(f32x16 (&X)[TI][TJ], f32x16 (&A)[TI][TI], int st, _Float16* xs) {
    if constexpr (TI != 2) {
      apply_scaled(X, A, st);
    } else {
      const float kap = kPEt[st][0], rho = kPEt[st][1];
      const int wo = opaque(wr_off()), ro = opaque(rd_off_ks());
      frag af[TI][TI][2];
      put_tile(A[0][1], 1.f, xs, wo);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        af[0][0][kb] = M::from_c(A[0][0], kb);
        af[0][1][kb] = M::from_c(A[0][1], kb);
        af[1][1][kb] = M::from_c(A[1][1], kb);
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) af[1][0][kb] = get_tr_ks(xs, kb, ro);
      A[0][0] *= kap;
      A[0][1] *= kap;
      A[1][1] *= kap;
      // the products without the transposed fragments first
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        A[0][0] = M::mma(af[0][0][kb], af[0][0][kb], A[0][0]);
        A[0][1] = M::mma(af[0][0][kb], af[0][1][kb], A[0][1]);
        A[1][1] = M::mma(af[0][1][kb], af[0][1][kb], A[1][1]);
        A[1][1] = M::mma(af[1][1][kb], af[1][1][kb], A[1][1]);
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        A[0][0] = M::mma(af[1][0][kb], af[1][0][kb], A[0][0]);
        A[0][1] = M::mma(af[1][0][kb], af[1][1][kb], A[0][1]);
      }
      // rho (kappa G + G^2): tile (1,0) through the other staging block (the
      // same one with NB == 1: these writes are ordered after the reads above)
      _Float16* xs2 = xs + (NB == 2 ? BLOCK : 0);
      put_tile(A[0][1], rho, xs2, wo);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const f32x16 t00 = A[0][0] * rho, t01 = A[0][1] * rho, t11 = A[1][1] * rho;
        af[0][0][kb] = M::from_c(t00, kb);
        af[0][1][kb] = M::from_c(t01, kb);
        af[1][1][kb] = M::from_c(t11, kb);
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) af[1][0][kb] = get_tr_ks(xs2, kb, ro);
#pragma unroll
      for (int J = 0; J < TJ; ++J) {
        frag xf[TI][2];
#pragma unroll
        for (int K = 0; K < TI; ++K) {
          asm volatile("" : "+v"(X[K][J]));
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) xf[K][kb] = M::from_c(X[K][J], kb);
        }
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int I = 0; I < TI; ++I) X[I][J] = M::mma(af[K][I][kb], xf[K][kb], X[I][J]);
      }
      // one scheduling region, each MFMA followed by two VALU instructions
      // (as apply_scaled)
#pragma unroll
      for (int i = 0; i < 12 + TI * TI * 2 * TJ; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // 2 VALU
      }
    }
  }
};

// One matrix per wave (fp16 operands), the Gram's operands transposed through
// the wave's LDS staging area xs (PEWaveT<D, E>::ELEMS halves).  The iterate
// is carried scaled (X_s = X / tau, kPEt), which saves the a X multiply of
// every step.  Returns the factor that turns X into PolarExpress(X)
// (PE = X * returned value).
template <int D, int E>
__device__ __forceinline__ float polar_express_wave_t(f32x16 (&X)[D / 32][E / 32], int ns, float norm_eps,
                                                      _Float16* xs) {
  using P = PEWaveT<D, E>;
  using W = PEWave<ModeF16, D, E>;
  const float ss = W::sumsq(X);
  W::scale(X, 32.f / (sqrtf(ss + norm_eps) * 1.01f + 1e-6f));   // X_s = X_0 / tau_0
  for (int st = 0; st < ns; ++st) {
    f32x16 A[D / 32][D / 32];
    P::gram_sym(X, A, xs);
    P::apply_sym(X, A, st, xs);
  }
  return kPEtau[ns];
}

// One matrix per wave.
template <class M, int D, int E>
__device__ __forceinline__ void polar_express_wave(f32x16 (&X)[D / 32][E / 32], int ns, float norm_eps,
                                                   typename M::elem* scr) {
  using P = PEWave<M, D, E>;
  const float ss = P::sumsq(X);
  P::scale(X, 1.f / (sqrtf(ss + norm_eps) * 1.01f + 1e-6f));
  for (int st = 0; st < ns; ++st) {
    f32x16 A[D / 32][D / 32];
    P::gram(X, A, scr);
    P::apply(X, A, st);
  }
}

// One D x 2EH matrix split by columns over a pair of waves of the same
// workgroup (each holds EH columns, `half` = 0 or 1).  The sum of squares and
// every Gram are combined through LDS, in one of two ways:
//   SEQ == false: `mine` and `other` are this wave's and the partner's
//     slots; both waves write their partial Gram and read the other's.  With
//     fp16 operands (ModeF16) the slots hold D*D halves: the partials are
//     rounded to fp16 and both waves form fp16(mine) + fp16(other) in fp32
//     (the Gram's fp16 operands already round X; this rounding is of the
//     same size and halves the exchange's LDS traffic and footprint).  With
//     fp32 operands the slots hold D*D floats and the waves form other + mine
//     / mine + other.  Either way both halves get the same values and stay
//     consistent.
//   SEQ == true: `mine` is one D*D-float slot shared by the pair (half the
//     LDS): half 0 writes its partial, half 1 adds it to its own and writes
//     the sum back, half 0 reads the sum.
// Every wave of the workgroup must call this with the same ns (it contains
// __syncthreads).
template <class M, int D, int EH, bool SEQ = false>
__device__ __forceinline__ float polar_express_pair(f32x16 (&X)[D / 32][EH / 32], int ns, float norm_eps,
                                                    typename M::elem* scr, float* mine, const float* other,
                                                    int half) {
  // fp16: the iterate is carried scaled (X_s = X / tau, kPEt; the update is
  // PEWaveT::apply_scaled) and the Gram's operands are transposed on the
  // matrix cores (scr unused); the return value turns X into PolarExpress(X)
  // (1 for fp32, which updates X itself and uses scr for the Gram).
  using P = PEWave<M, D, EH>;
  using PT = PEWaveT<D, EH>;
  constexpr bool F16 = sizeof(typename M::elem) == 2;
  constexpr int TI = D / 32;
  const int lane = lane_id();
  float ss = P::sumsq(X);
  if constexpr (SEQ) {
    if (lane == 0) mine[half] = ss;
    __syncthreads();
    ss = mine[0] + mine[1];
  } else {
    if (lane == 0) mine[0] = ss;
    __syncthreads();
    ss += other[0];
  }
  __syncthreads();
  P::scale(X, (F16 ? 32.f : 1.f) / (sqrtf(ss + norm_eps) * 1.01f + 1e-6f));
  // Gram tiles in LDS as 16-byte quads: registers 4q..4q+3 of tile (I, I2)
  // for this lane at quad ((I*TI + I2)*4 + q)*64 + lane
  auto put = [&](const f32x16 (&A)[TI][TI], float* dst) {
    f32x4* d4 = reinterpret_cast<f32x4*>(dst);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          d4[((I * TI + I2) * 4 + q) * WAVE + lane] =
              f32x4{A[I][I2][4 * q], A[I][I2][4 * q + 1], A[I][I2][4 * q + 2], A[I][I2][4 * q + 3]};
  };
  // fp16 exchange: registers 4q..4q+3 of tile (I, I2) as 8 bytes at
  // ((I*TI + I2)*4 + q)*64 + lane; put16 also rounds the wave's own tiles to
  // the values the partner reads, add16 adds the partner's
  auto put16 = [&](f32x16 (&A)[TI][TI], float* dst) {
    f16x4* d4 = reinterpret_cast<f16x4*>(dst);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f16x4 v = f16x4{(_Float16)A[I][I2][4 * q], (_Float16)A[I][I2][4 * q + 1],
                                (_Float16)A[I][I2][4 * q + 2], (_Float16)A[I][I2][4 * q + 3]};
          d4[((I * TI + I2) * 4 + q) * WAVE + lane] = v;
#pragma unroll
          for (int u = 0; u < 4; ++u) A[I][I2][4 * q + u] = (float)v[u];
        }
  };
  auto add16 = [&](const float* src, f32x16 (&A)[TI][TI]) {
    const f16x4* s4 = reinterpret_cast<const f16x4*>(src);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f16x4 v = s4[((I * TI + I2) * 4 + q) * WAVE + lane];
#pragma unroll
          for (int u = 0; u < 4; ++u) A[I][I2][4 * q + u] += (float)v[u];
        }
  };
  // A += (or =) the quads at src, one tile at a time
  auto add_from = [&](const float* src, f32x16 (&A)[TI][TI], bool assign) {
    const f32x4* s4 = reinterpret_cast<const f32x4*>(src);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = s4[((I * TI + I2) * 4 + q) * WAVE + lane];
#pragma unroll
          for (int u = 0; u < 4; ++u) A[I][I2][4 * q + u] = assign ? v[u] : A[I][I2][4 * q + u] + v[u];
        }
  };
  for (int st = 0; st < ns; ++st) {
    f32x16 A[TI][TI];
    P::gram(X, A, scr);
    if constexpr (SEQ) {
      if (half == 0) put(A, mine);
      __syncthreads();
      if (half == 1) {
        add_from(mine, A, false);
        put(A, mine);
      }
      __syncthreads();
      if (half == 0) add_from(mine, A, true);
    } else if constexpr (F16) {
      put16(A, mine);
      __syncthreads();
      add16(other, A);
      __syncthreads();
    } else {
      put(A, mine);
      __syncthreads();
      add_from(other, A, false);
      __syncthreads();
    }
    if constexpr (F16) PT::apply_scaled(X, A, st);
    else P::apply(X, A, st);
  }
  return F16 ? kPEtau[ns] : 1.f;
}

// Halves of one wave's exchange slot in polar_express_pair_sym: the three
// upper 32 x 32 Gram tiles in fp16.
constexpr int kPairXSlot = 3 * 4 * WAVE * 4;

// polar_express_pair for fp16 operands at D = 64, on the symmetric step of
// PEWaveT: each wave forms the upper tiles (0,0), (0,1), (1,1) of its partial
// Gram from its columns staged through LDS with transposing reads (no
// identity products), the pair adds the three tiles through LDS as
// fp16(mine) + fp16(other), and each wave applies apply_sym to its columns.
// Per step and wave 68 matrix-core products instead of 96 (16 of which
// transposed the Gram's operands), and one barrier per exchange instead of
// two:
//   * each wave has two slot sets, mine0 / mine0 + set_stride (floats; the
//     partner's at other0 / other0 + set_stride), of kPairXSlot halves each;
//     exchange number k (xk counts them across calls, so consecutive calls of
//     the same pair keep alternating) writes set k & 1, passes the barrier and
//     reads the partner's set k & 1;
//   * before a wave writes set k & 1 the partner has finished reading it: that
//     read (exchange k - 2) came before the partner's barrier k - 1;
//   * between barrier k - 1 and its write of exchange k a wave stages its
//     Gram and transposed blocks in its own set k & 1, which the partner is
//     not reading then (it reads set (k - 1) & 1); the exchange's writes come
//     after the staging reads (they may alias, and LDS operations of one wave
//     complete in order).
// Every wave of the workgroup must call this with the same ns and the same
// number of times (it contains __syncthreads).
template <int D, int EH>
__device__ __forceinline__ float polar_express_pair_sym(f32x16 (&X)[D / 32][EH / 32], int ns, float norm_eps,
                                                        float* mine0, const float* other0, int set_stride,
                                                        int& xk) {
  using P = PEWave<ModeF16, D, EH>;
  using PT = PEWaveT<D, EH>;
  constexpr int TI = D / 32;
  static_assert(TI == 2, "the symmetric pair step is written for D = 64");
  static_assert(PT::BLOCK <= kPairXSlot, "a staging block fits an exchange slot");
  const int lane = lane_id();
  auto mine = [&](int k) { return mine0 + (k & 1) * set_stride; };
  auto other = [&](int k) { return other0 + (k & 1) * set_stride; };
  float ss = P::sumsq(X);
  if (lane == 0) mine(xk)[0] = ss;
  __syncthreads();
  ss += other(xk)[0];
  ++xk;
  P::scale(X, 32.f / (sqrtf(ss + norm_eps) * 1.01f + 1e-6f));
  // tiles (0,0), (0,1), (1,1) as slots 0, 1, 2: registers 4q..4q+3 of slot u
  // as 8 bytes at (u*4 + q)*64 + lane
  for (int st = 0; st < ns; ++st) {
    f32x16 A[TI][TI];
    PT::template gram_sym<1>(X, A, reinterpret_cast<_Float16*>(mine(xk)));
    f16x4* m4 = reinterpret_cast<f16x4*>(mine(xk));
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      f32x16& t = (u == 0) ? A[0][0] : (u == 1) ? A[0][1] : A[1][1];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f16x4 v = f16x4{(_Float16)t[4 * q], (_Float16)t[4 * q + 1], (_Float16)t[4 * q + 2],
                              (_Float16)t[4 * q + 3]};
        m4[(u * 4 + q) * WAVE + lane] = v;
#pragma unroll
        for (int k = 0; k < 4; ++k) t[4 * q + k] = (float)v[k];
      }
    }
    __syncthreads();
    const f16x4* o4 = reinterpret_cast<const f16x4*>(other(xk));
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      f32x16& t = (u == 0) ? A[0][0] : (u == 1) ? A[0][1] : A[1][1];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f16x4 v = o4[(u * 4 + q) * WAVE + lane];
#pragma unroll
        for (int k = 0; k < 4; ++k) t[4 * q + k] += (float)v[k];
      }
    }
    ++xk;
    PT::template apply_sym<1>(X, A, st, reinterpret_cast<_Float16*>(mine(xk)));
  }
  return kPEtau[ns];
}

}  // namespace atlas
