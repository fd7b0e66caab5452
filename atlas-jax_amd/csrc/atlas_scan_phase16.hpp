// fp16 phase kernel of the chunk scan (memories with E <= 128).
//
// Same work as phase_kernel (atlas_scan_kernels.hpp) for one (stream, slice):
// build S_t for each of the slice's tokens, Polar-Express it, and accumulate
// the slice-local parts of the memory scan (L_j = sum_s a(s->end_j) P_s) and
// of the read-out (hloc / yloc).  What differs is where things live:
//   - the Polar-Express Gram operands and the W1 read-out's P1 rows are
//     transposed through a per-wave LDS staging area (transposing LDS reads)
//     instead of on the matrix cores;
//   - the per-wave partial of L_j and the read-out partials accumulate in the
//     accumulation registers (AGPRs) through MFMAs with an AGPR accumulator,
//     L_j as a(s->end) I * bf16(P_s) (identity A operand carrying the
//     weight; bf16 for fp32's exponent range: when the momentum is below the
//     normalisation's 1e-6, P and with it W_end are tiny, and fp16 would
//     flush them), so they neither occupy the arch VGPRs that Polar-Express
//     needs nor synchronise the waves per token; the four waves' partials are
//     summed in a fixed order in the epilogue (bitwise reproducible).
// Semantics and outputs are those of phase_kernel (atlas_jax/memory_layer.py
// :496-597 split by the chunk algebra described there).
#pragma once

#include "atlas_scan_kernels.hpp"

namespace atlas {

template <int D, int E>
struct Phase16Layout {
  using PT = PEWaveT<D, E>;
  static constexpr int PADE = 8;                   // row padding (halves)
  static constexpr int SPD = D + 4;                // Sp row stride (floats)
  static constexpr int QSP = D + PADE;             // query rows (MAT 2)
  static constexpr int GSP = E + PADE;             // g rows (MAT 1)
  int csp;                                         // token-row stride of Ut/Vt/ctil
  size_t o_ctil, o_small, o_Ut, o_Vt, o_Sp, o_QG, o_xs, total;

  __host__ __device__ Phase16Layout(int cs, int ts) {
    const int npad = ((cs + 15) / 16) * 16;
    csp = npad + PADE;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t r = o; o += (bytes + 15) & ~size_t(15); return r; };
    o_ctil = take((size_t)ts * csp * 2);
    o_small = take((size_t)(4 * TS_MAX + ts * ts + NSL_MAX * ts + 16) * sizeof(float));
    const size_t big0 = o;
    o_Ut = take((size_t)D * csp * 2);
    o_Vt = take((size_t)E * csp * 2);
    o_Sp = take((size_t)E * SPD * sizeof(float));
    o_QG = take((size_t)32 * (QSP > GSP ? QSP : GSP) * 2);
    o_xs = take((size_t)NW * PT::ELEMS * 2);
    // epilogue (reuses [big0, end)): one D*E fp32 slot per wave for L_j,
    // later one read-out slot (up to 4 tiles) per wave
    const size_t epi = big0 + (size_t)NW * D * E * sizeof(float);
    total = o > epi ? o : epi;
  }
};

template <int D, int E, int MAT>
__global__ void __launch_bounds__(NTHREADS)
__attribute__((amdgpu_waves_per_eu(1, 1)))
phase16_kernel(ScanArgs p) {
  using M = ModeF16;
  using frag = f16x8;
  using PT = PEWaveT<D, E>;
  constexpr int TI = D / 32, TJ = E / 32, KPT = 2;
  using LY = Phase16Layout<D, E>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const LY L(p.cs, p.ts);

  const int lb = xcd_block();
  const int stream = lb / p.nsl, j = lb % p.nsl;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, wv = wave_id();
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, n = tok0 + ts;
  const long long sDE = (long long)stream * D * E;

  _Float16* ctil = reinterpret_cast<_Float16*>(smem + L.o_ctil);
  float* sm = reinterpret_cast<float*>(smem + L.o_small);
  float* mrow = sm;
  float* thp = sm + TS_MAX;
  float* Apre = sm + 2 * TS_MAX;
  float* ass = sm + 4 * TS_MAX;       // [s][t'] = a(s -> t') within the slice
  float* ait = ass + ts * ts;         // [i][t'] = a(e_i -> t'), i < j
  float* red4 = ait + NSL_MAX * ts;
  _Float16* Ut = reinterpret_cast<_Float16*>(smem + L.o_Ut);
  _Float16* Vt = reinterpret_cast<_Float16*>(smem + L.o_Vt);
  float* Sp = reinterpret_cast<float*>(smem + L.o_Sp);
  _Float16* Qs = reinterpret_cast<_Float16*>(smem + L.o_QG);   // MAT 2: queries
  _Float16* Gs = Qs;                                           // MAT 1: g = gelu(h)
  _Float16* xs = reinterpret_cast<_Float16*>(smem + L.o_xs) + wv * PT::ELEMS;

  // ---- staging: every global load is issued before any of them is used ----
  const long long tb = chunk_table(p, stream, p.chunk);
  float inv_uv;              // undoes the operand scaling of the momentum products
  f32x4 wraw[TI][KPT][2];    // MAT 1: read-out init W1 rows (fp32, loaded with the staging)
  f32x4 hraw[4];             // MAT 1: hloc rows of the slice
  // MAT 1 without the slice prefix (at most four slices, so at most three
  // earlier ones): the rows of L2_i (E-tile wv, i < j) for the cross-slice
  // read-out terms, loaded with the staging (fp32, converted where they are
  // used, after the staging barrier: nothing in the staging waits for them)
  constexpr int NXS = 3;
  f32x4 lraw[NXS][TI][KPT][2];
  {
    constexpr int CF4 = TS_MAX * CS_MAX / 4 / NTHREADS;
    constexpr int UF4 = D * CS_MAX / 4 / NTHREADS, VF4 = E * CS_MAX / 4 / NTHREADS;
    constexpr int SF4 = D * E / 4 / NTHREADS;
    const float* Usrc = (MAT == 2 ? p.kT : p.errT) + (long long)stream * D * cs;
    const float* Vsrc = (MAT == 2 ? p.chainT : p.actT) + (long long)stream * E * cs;
    const float* Sc = (MAT == 2 ? p.S2[p.cur] : p.S1[p.cur]) + sDE;
    // gate tables first: they stay in registers while the operand loads are
    // in flight (a wait for a load waits for every load issued before it)
    const float* am = p.am + tb * cs * cs;
    const bool tok_ok = tid < ts;
    const long long gq = tb * cs + tok0 + (tok_ok ? tid : 0);
    const float g_m = p.cm[gq], g_th = p.thp[gq], g_ap = p.ap[gq];
    constexpr int NAS = TS_MAX * TS_MAX / NTHREADS;
    float asv[NAS];
#pragma unroll
    for (int u = 0; u < NAS; ++u) {
      const int idx = tid + u * NTHREADS, s_ = idx / ts, t_ = idx % ts;
      asv[u] = am[idx < ts * ts ? (tok0 + t_) * cs + tok0 + s_ : 0];
    }
    const bool ait_ok = tid < j * ts;   // j * ts < cs <= NTHREADS
    const float aitv = am[ait_ok ? (tok0 + tid % ts) * cs + (tid / ts + 1) * ts - 1 : 0];
    if constexpr (MAT == 1) {
      const int Iw = (wv < TJ) ? wv : 0;
#pragma unroll
      for (int di = 0; di < NXS; ++di) {
        if (p.use_prefix || di >= j) break;
        const float* L2i = p.L2 + ((long long)stream * p.nsl + di) * D * E + (32 * Iw + c) * D + 4 * h;
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) {
            lraw[di][K][kb][0] = *reinterpret_cast<const f32x4*>(L2i + 32 * K + 16 * kb);
            lraw[di][K][kb][1] = *reinterpret_cast<const f32x4*>(L2i + 32 * K + 16 * kb + 8);
          }
      }
    }

    f32x4 cv[CF4], uv[UF4], vv[VF4], sv4[SF4];
    TokenRows<D, 32> qr;
    static_assert(TJ <= NW, "one read-out E-tile per wave");
    load_rows4<CF4>(cv, p.cmt + tb * cs * cs + (long long)tok0 * cs, ts, n, cs);
    load_rows4<UF4>(uv, Usrc, D, n, cs);
    load_rows4<VF4>(vv, Vsrc, E, n, cs);
    // chunk-start momentum: S2 ([e][d]) as quads; S1 ([d][e]) as 4x4 blocks
    // (rows d0..d0+3 at columns e0..e0+3, consecutive threads along e) that
    // are stored transposed below
    constexpr bool S4X4 = (MAT == 1) && (SF4 % 4 == 0);
    if constexpr (!S4X4) {
#pragma unroll
      for (int u = 0; u < SF4; ++u) sv4[u] = reinterpret_cast<const f32x4*>(Sc)[tid + u * NTHREADS];
    } else {
#pragma unroll
      for (int u = 0; u < SF4; ++u) {
        const int bi = tid + (u / 4) * NTHREADS, eq = bi % (E / 4), dq = bi / (E / 4);
        sv4[u] = *reinterpret_cast<const f32x4*>(Sc + (4 * dq + (u & 3)) * E + 4 * eq);
      }
    }
    qr.load(p, p.q, b, hh, tok0, ts);
    // MAT 1 read-out init operands, converted after the staging barrier: W1
    // rows d at E-block wv (contiguous k) and the slice's hloc rows (E <= 128:
    // one E-tile per wave).  (MAT 2 loads its W2 rows after the barrier: with
    // the staging registers live they would spill.)
    if constexpr (MAT == 1) {
      const int Iw = (wv < TJ) ? wv : 0;
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) {
          const float* lo = p.W1[p.cur] + sDE + (32 * K + c) * E + 32 * Iw + 16 * kb + 8 * h;
          wraw[K][kb][0] = *reinterpret_cast<const f32x4*>(lo);
          wraw[K][kb][1] = *reinterpret_cast<const f32x4*>(lo + 4);
        }
      const float* hl = p.hloc + (((long long)stream * p.nsl + j) * ts + (c < ts ? c : 0)) * E + 32 * Iw + 4 * h;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) hraw[g4] = *reinterpret_cast<const f32x4*>(hl + 8 * g4);
    }

    if (tok_ok) {
      mrow[tid] = g_m;
      thp[tid] = g_th;
      Apre[tid] = g_ap;
    }
#pragma unroll
    for (int u = 0; u < NAS; ++u) {
      const int idx = tid + u * NTHREADS;
      if (idx < ts * ts) ass[idx] = asv[u];
    }
    if (ait_ok) ait[tid] = aitv;

    store_rows4<M, CF4>(cv, ctil, ts, n, L.csp, 1.f);
    // operands power-of-two scaled into fp16 range
    float mu = maxabs4<UF4>(uv, D, n), mv = maxabs4<VF4>(vv, E, n);
    block_max2<NW>(mu, mv, red4);
    const float su = pow2_scale(mu), sv = pow2_scale(mv);
    store_rows4<M, UF4>(uv, Ut, D, n, L.csp, su);
    store_rows4<M, VF4>(vv, Vt, E, n, L.csp, sv);
    // zero the K-block tail [n, 16*ceil(n/16)) of every operand row
    const int npad = ((n + M::KB - 1) / M::KB) * M::KB;
    if (npad > n) {
      const int w = npad - n;
      for (int i = tid; i < (D + E + ts) * w; i += NTHREADS) {
        const int r = i / w, t = n + i % w;
        if (r < D) Ut[r * L.csp + t] = (_Float16)0.f;
        else if (r < D + E) Vt[(r - D) * L.csp + t] = (_Float16)0.f;
        else ctil[(r - D - E) * L.csp + t] = (_Float16)0.f;
      }
    }
    inv_uv = 1.f / (su * sv);
    // chunk-start momentum, stored [e][d]
    if constexpr (MAT == 2) {   // S2 is [e][d]
#pragma unroll
      for (int u = 0; u < SF4; ++u) {
        const int i = 4 * (tid + u * NTHREADS);
        *reinterpret_cast<f32x4*>(Sp + (i / D) * LY::SPD + (i % D)) = sv4[u];
      }
    } else if constexpr (!S4X4) {   // S1 is [d][e], few elements per thread
#pragma unroll
      for (int u = 0; u < SF4; ++u) {
        const int i = 4 * (tid + u * NTHREADS), d = i / E, e0 = i % E;
#pragma unroll
        for (int k = 0; k < 4; ++k) Sp[(e0 + k) * LY::SPD + d] = sv4[u][k];
      }
    } else {          // S1 is [d][e]: transpose each 4x4 block in registers
#pragma unroll
      for (int g = 0; g < SF4 / 4; ++g) {
        const int bi = tid + g * NTHREADS, eq = bi % (E / 4), dq = bi / (E / 4);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          *reinterpret_cast<f32x4*>(Sp + (4 * eq + k) * LY::SPD + 4 * dq) =
              f32x4{sv4[4 * g][k], sv4[4 * g + 1][k], sv4[4 * g + 2][k], sv4[4 * g + 3][k]};
      }
    }
    qr.template store<_Float16>(Qs, LY::QSP, p.io_dtype);   // MAT 1: in the g area until g replaces it
  }
  __syncthreads();
  auto wfrag = [&](int K, int kb) -> frag {
    frag f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      f[v] = (_Float16)wraw[K][kb][0][v];
      f[4 + v] = (_Float16)wraw[K][kb][1][v];
    }
    return f;
  };

  // ---- read-out partial accumulators (AGPRs) ----------------------------
  constexpr int TR = (MAT == 2) ? TJ : TI;   // tiles of the slice read-out block
  f32x16 RO[TR];
  agpr_init(RO);

  // query fragments with the C-layout k assignment (B operand, lane = t'); lc
  // is the lane's row, passed through opaque() inside the token loop so that
  // these loop-invariant LDS reads are repeated per token rather than held
  // in registers across Polar-Express
  auto load_qf = [&](int K, int kb, int lc) -> frag { return M::ld_cslot(Qs + lc * LY::QSP + 32 * K, kb, h); };
  const float wA = (c < ts) ? Apre[c] : 0.f;

  if (MAT == 2) {
    // hloc init: A_t * W2 q_t, wave w -> E-tile w (a compile-time tile index:
    // the accumulators are registers)
    const float* W2c = p.W2[p.cur] + sDE;
#pragma unroll
    for (int Ie = 0; Ie < TJ; ++Ie) {
      if (Ie != wv) continue;
      frag wf[TI][KPT];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) wf[K][kb] = M::gl_cslot(W2c + (32 * Ie + c) * D + 32 * K, kb, h);
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) agpr_mfma(RO[Ie], wf[K][kb], M::scale(load_qf(K, kb, c), wA));
    }
  } else {
    // h for the slice: hloc_j + sum_{i<j} a(end_i->t) L2_i^T q_t, then g = gelu(h)
    constexpr int QJ = 1;   // one E-tile per wave (TJ <= NW)
    f32x16 hacc[QJ];
#pragma unroll
    for (int q = 0; q < QJ; ++q) {
      const int Ie = wv + q * NW;
      if (Ie >= TJ) break;
      // cross-slice terms first (their loads do not wait for hloc's), hloc
      // added at the end
      f32x16 acc = zero16();
      if (!p.use_prefix) {
#pragma unroll
        for (int di = 0; di < NXS; ++di) {
          if (di >= j) break;
          const float wi = (c < ts) ? ait[di * ts + c] : 0.f;
#pragma unroll
          for (int K = 0; K < TI; ++K)
#pragma unroll
            for (int kb = 0; kb < KPT; ++kb) {
              frag lf;   // C-layout k of L2_i's row (gl_cslot)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                lf[v] = (_Float16)lraw[di][K][kb][0][v];
                lf[4 + v] = (_Float16)lraw[di][K][kb][1][v];
              }
              acc = M::mma(lf, M::scale(load_qf(K, kb, c), wi), acc);
            }
        }
      }
      if (p.use_prefix && j > 0) {
        const float* M2j = p.L2 + ((long long)stream * p.nsl + j) * D * E;
        frag lf[TI][KPT];
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) lf[K][kb] = M::gl_cslot(M2j + (32 * Ie + c) * D + 32 * K, kb, h);
        const float wi = (c < ts) ? ait[(j - 1) * ts + c] : 0.f;
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) acc = M::mma(lf[K][kb], M::scale(load_qf(K, kb, c), wi), acc);
      }
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[4 * g4 + u] += (c < ts) ? hraw[g4][u] : 0.f;
      hacc[q] = acc;
    }
    __syncthreads();   // queries consumed: the area takes g
#pragma unroll
    for (int q = 0; q < QJ; ++q) {
      const int Ie = wv + q * NW;
      if (Ie >= TJ) break;
      float* gout = p.g + ((long long)stream * cs + tok0 + c) * E;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        f32x4 gv;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * g4 + u, e = 32 * Ie + crow(r, h);
          gv[u] = (c < ts) ? gelu_tanh(hacc[q][r]) : 0.f;
          Gs[c * LY::GSP + e] = (_Float16)gv[u];
        }
        // rows crow(4*g4 + u, h) are four consecutive e
        if (c < ts) *reinterpret_cast<f32x4*>(gout + 32 * Ie + 8 * g4 + 4 * h) = gv;
      }
    }
    __syncthreads();
    // yloc init: A_t * W1 g_t, wave w -> E-blocks Je = w (mod NW) of the contraction
#pragma unroll
    for (int q = 0; q < QJ; ++q) {
      const int Je = wv + q * NW;
      if (Je >= TJ) break;
#pragma unroll
      for (int Id = 0; Id < TI; ++Id)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb)
          agpr_mfma(RO[Id], wfrag(Id, kb), M::scale(M::ld_contig(Gs + c * LY::GSP + 32 * Je, kb, h), wA));
    }
  }

  // ---- per-token momentum assembly, Polar-Express, partial sums ----------
  f32x16 Lw[TI][TJ];   // this wave's share of L_j (AGPRs), tiles of X's layout
#pragma unroll
  for (int I = 0; I < TI; ++I) agpr_init(Lw[I]);

  const int tpw = ts / NW;
  const int nkb = (n + M::KB - 1) / M::KB;
  for (int it = 0; it < tpw; ++it) {
    const int sl = wv * tpw + it;      // slice-local token
    const int t = tok0 + sl;           // chunk-local token
    const int lc = PT::opaque(c);      // (see load_qf)
    f32x16 X[TI][TJ];
    // Y = sum_i c~[t,i] u_i (x) v_i on the matrix cores
    const _Float16* crowp = ctil + sl * L.csp;
    auto s_block = [&](int kb, bool first) {
      const frag cf = M::ld_contig(crowp, kb, h);
      frag uf[TI];
#pragma unroll
      for (int I = 0; I < TI; ++I) uf[I] = M::ld_contig(Ut + (32 * I + lc) * L.csp, kb, h) * cf;
#pragma unroll
      for (int J = 0; J < TJ; ++J) {
        const frag vf = M::ld_contig(Vt + (32 * J + lc) * L.csp, kb, h);
#pragma unroll
        for (int I = 0; I < TI; ++I) X[I][J] = M::mma(uf[I], vf, first ? zero16() : X[I][J]);
      }
    };
    s_block(0, true);                  // nkb >= 1: every chunk has a token
    for (int kb = 1; kb < nkb; ++kb) s_block(kb, false);
    // S_t = th * S_0 + f * Y (f undoes the operand scaling)
    const float f = mrow[sl] * inv_uv;
    const float th = thp[sl];
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 sp = *reinterpret_cast<const f32x4*>(Sp + (32 * J + lc) * LY::SPD + 32 * I + 8 * q4 + 4 * h);
#pragma unroll
          for (int u = 0; u < 4; ++u) X[I][J][4 * q4 + u] = th * sp[u] + f * X[I][J][4 * q4 + u];
        }
    if (j == p.nsl - 1 && t == cs - 1) {
      // final momentum of the chunk -> next state buffer
      if (MAT == 2) {
        float* S2n = p.S2[p.cur ^ 1] + sDE;
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int J = 0; J < TJ; ++J)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
              f32x4 v4;
#pragma unroll
              for (int u = 0; u < 4; ++u) v4[u] = X[I][J][4 * q4 + u];
              *reinterpret_cast<f32x4*>(S2n + (32 * J + c) * D + 32 * I + 8 * q4 + 4 * h) = v4;
            }
      } else {
        // S1 is [d][e]: 64 single-float stores per lane.  The lane's offset is
        // formed here (opaque), so that the compiler does not hoist 64
        // per-element addresses out of the token loop into registers that
        // Polar-Express needs (they were spilled to AGPRs and reloaded in
        // every Newton-Schulz step) for a store that runs once per chunk.
        float* S1n = p.S1[p.cur ^ 1] + sDE + PT::opaque(crow(0, h) * E + c);
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int J = 0; J < TJ; ++J)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              S1n[(32 * I + 8 * (r >> 2) + (r & 3)) * E + 32 * J] = X[I][J][r];
      }
    }

    const float pscale = polar_express_wave_t<D, E>(X, p.ns, 1e-12f, xs);   // X * pscale = P

    // memory-scan partial L += a(s->end_j) P (bf16 identity A operand carrying
    // the weight) and the slice read-out partial (fp16 P fragments)
    const float aend = ass[sl * ts + ts - 1] * pscale;
    const float wt = (c < ts) ? ass[sl * ts + c] * pscale : 0.f;   // a(s->t') masked to t' >= s
    bf16x8 aid[KPT];
#pragma unroll
    for (int kb = 0; kb < KPT; ++kb) aid[kb] = M::a_identity(kb, c, h, aend);
    if (MAT == 2) {
      // hloc[e][t'] += sum_d P2[e][d] q_t'[d] w(t')  (X tiles as A operand = P2 rows e)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int K = 0; K < TI; ++K) {
          frag xf[KPT];
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) xf[kb] = M::from_c(X[K][J], kb);
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) agpr_mfma(RO[J], xf[kb], M::scale(load_qf(K, kb, lc), wt));
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) agpr_mfma_bf16(Lw[K][J], aid[kb], M::a_from_c(X[K][J], kb));
        }
    } else {
      // yloc[d][t'] += sum_e P1[d][e] g_t'[e] w(t'): block Je of P1 through the
      // staging area as fp16 rows e, transposing reads give P1[d][e] with d
      // along the lanes and e (contiguous k) along the registers
      const int wo = PT::opaque(PT::wr_off()), ro = PT::opaque(PT::rd_off());
#pragma unroll
      for (int Je = 0; Je < TJ; ++Je) {
        _Float16* buf = xs + (Je & 1) * PT::BLOCK;
        frag xf[TI][KPT];
#pragma unroll
        for (int Id = 0; Id < TI; ++Id)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) {
            xf[Id][kb] = M::from_c(X[Id][Je], kb);
            // elements 4g..4g+3 of the fragment are rows 32Id + 16kb + 8g + 4h + 0..3
#pragma unroll
            for (int g = 0; g < 2; ++g)
              *reinterpret_cast<f16x4*>(buf + wo + 32 * Id + 16 * kb + 8 * g) =
                  f16x4{xf[Id][kb][4 * g], xf[Id][kb][4 * g + 1], xf[Id][kb][4 * g + 2], xf[Id][kb][4 * g + 3]};
          }
        frag th[TI][KPT], gw[KPT];
        PT::read_block(th, buf, ro);
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) gw[kb] = M::scale(M::ld_contig(Gs + lc * LY::GSP + 32 * Je, kb, h), wt);
#pragma unroll
        for (int Id = 0; Id < TI; ++Id)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) agpr_mfma(RO[Id], th[Id][kb], gw[kb]);
#pragma unroll
        for (int Id = 0; Id < TI; ++Id)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) agpr_mfma_bf16(Lw[Id][Je], aid[kb], M::a_from_c(X[Id][Je], kb));
      }
    }
  }
  agpr_mfma_drain(RO);
#pragma unroll
  for (int I = 0; I < TI; ++I) agpr_mfma_drain(Lw[I]);

  // ---- epilogue: the four waves' partials, summed in a fixed order --------
  // Each wave stores its tiles as 16-byte quads (element 4q + u of tile tl for
  // lane ln at quad (tl * 4 + q) * 64 + ln of its slot); then every thread
  // sums quads of the four slots, ((w0 + w1) + w2) + w3, and stores them.
  __syncthreads();
  constexpr int RW = (MAT == 2) ? E : D;   // row length of hloc / yloc
  float* ro_out = (MAT == 2 ? p.hloc : p.yloc) + (((long long)stream * p.nsl + j) * ts) * RW;
  float* Lout = (MAT == 2 ? p.L2 : p.L1) + ((long long)stream * p.nsl + j) * D * E;
  f32x4* slots = reinterpret_cast<f32x4*>(smem + L.o_Ut);   // 4 x D*E floats
  constexpr int NQ = D * E / 4;                              // quads per slot (L)
  {
    f32x4* sw = slots + wv * NQ;
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sw[((I * TJ + J) * 4 + q) * WAVE + lane] =
              f32x4{Lw[I][J][4 * q], Lw[I][J][4 * q + 1], Lw[I][J][4 * q + 2], Lw[I][J][4 * q + 3]};
  }
  __syncthreads();
  for (int i = tid; i < NQ; i += NTHREADS) {
    const f32x4 v = ((slots[i] + slots[NQ + i]) + slots[2 * NQ + i]) + slots[3 * NQ + i];
    // tile (I, J) rows d = 32I + crow(4q + u, hl) = d0 + u, column e = 32J + cl
    const int tl = i / (4 * WAVE), q = (i / WAVE) & 3, ln = i & (WAVE - 1);
    const int I = tl / TJ, J = tl % TJ, cl = ln & 31, hl = ln >> 5;
    const int d0 = 32 * I + 8 * q + 4 * hl, e = 32 * J + cl;
    if (MAT == 2) {   // L2 is [e][d]
      *reinterpret_cast<f32x4*>(Lout + (long long)e * D + d0) = v;
    } else {          // L1 is [d][e]: consecutive lanes write consecutive e
#pragma unroll
      for (int u = 0; u < 4; ++u) Lout[(long long)(d0 + u) * E + e] = v[u];
    }
  }
  __syncthreads();
  constexpr int NR = TR * 4 * WAVE;                          // quads per slot (read-out)
  {
    f32x4* sw = slots + wv * NR;
#pragma unroll
    for (int q = 0; q < TR; ++q)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        sw[(q * 4 + q4) * WAVE + lane] = f32x4{RO[q][4 * q4], RO[q][4 * q4 + 1], RO[q][4 * q4 + 2], RO[q][4 * q4 + 3]};
  }
  __syncthreads();
  for (int i = tid; i < NR; i += NTHREADS) {
    // tile q rows x = 32q + crow(4 q4 + u, hl) (e or d), column t' = cl
    const int q = i / (4 * WAVE), q4 = (i / WAVE) & 3, ln = i & (WAVE - 1), cl = ln & 31, hl = ln >> 5;
    if (cl < ts) {
      const f32x4 v = ((slots[i] + slots[NR + i]) + slots[2 * NR + i]) + slots[3 * NR + i];
      *reinterpret_cast<f32x4*>(ro_out + (long long)cl * RW + 32 * q + 8 * q4 + 4 * hl) = v;
    }
  }
}

}  // namespace atlas
