// Phase kernels for wide memories (E = 256 at D = 64; the ~170M and MAG
// configurations), fp16 matrix-core operands only.
//
// Same algebra as phase_kernel (atlas_scan_kernels.hpp): per (stream, slice)
// the per-token momentum S_t, its Polar-Express P_t, the slice's memory-scan
// partial L_j = sum_s a(s->end_j) P_s and the slice read-out partials.  What
// changes is the mapping onto the workgroup, because a D x E fp32 matrix no
// longer fits one wave's registers next to the Polar-Express temporaries and
// the single-wave LDS layout exceeds 160 KiB:
//   * the four waves form two pairs; pair p takes tokens p*ts/2 .. p*ts/2 +
//     ts/2 - 1 of the slice, and within a pair wave `half` holds columns
//     [half*E/2, half*E/2 + E/2) of S_t (Polar-Express via polar_express_pair,
//     the Gram summed through LDS);
//   * the chunk-start momentum S_0, in [e][d] form for both matrices (a
//     transposed copy of S1 is kept in the workspace), is staged in LDS as
//     power-of-two scaled fp16 when the layout leaves room for it (S0L: the
//     cs = 64 shapes), else read from global memory (L2) when S_t is formed;
//     the chunk's last token, whose momentum is the carried state, always
//     takes the fp32 S_0 from global memory;
//   * each wave accumulates its share of L_j in accumulation registers
//     (AGPRs, through bf16 identity MFMAs as in phase16_kernel), and the two
//     pairs' partials are added in a fixed order in the epilogue.
#pragma once

#include "atlas_scan_kernels.hpp"

namespace atlas {

constexpr size_t WIDE_LDS_MAX = 160 * 1024;

// Runtime LDS layout of the wide phase kernels (host and device agree on it).
template <int D, int E>
struct WideLayout {
  static constexpr int EB = 2, PADE = 8;
  static constexpr int QSP = D + PADE, GSP = E + PADE;
  static constexpr int S0P = D + 4;   // S_0 row stride (halves): 8-byte aligned rows, conflict-free lane rows
  static constexpr int TI = D / 32, TJh = E / 64;
  // one wave's fp16 exchange slot (halves) of the symmetric pair step
  static constexpr int XSLOT = kPairXSlot;
  int csp;
  bool seq;   // pair Gram exchange through one fp32 slot per pair (else two fp16 slots per wave)
  bool s0l;   // S_0 staged in LDS (fp16)
  size_t o_ctil, o_small, o_Ut, o_Vt, o_Qs, o_Gs, o_xch, o_S0, total;

  __host__ __device__ WideLayout(int cs, int ts, int nsl) {
    const int npad = ((cs + 15) / 16) * 16;
    csp = npad + PADE;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t r = o; o += (bytes + 15) & ~size_t(15); return r; };
    o_ctil = take((size_t)ts * csp * EB);
    o_small = take((size_t)(ts * 4 + ts * ts + nsl * ts + 16) * sizeof(float));
    const size_t big0 = o;
    o_Ut = take((size_t)D * csp * EB);
    o_Vt = take((size_t)E * csp * EB);
    o_Qs = take((size_t)32 * QSP * EB);
    o_Gs = take((size_t)32 * GSP * EB);
    const size_t xpar = D == 64 ? (size_t)NW * 2 * XSLOT * 2 : ~size_t(0) / 2,
                 xseq = (size_t)(NW / 2) * D * D * sizeof(float);
    seq = o + xpar > WIDE_LDS_MAX;
    o_xch = take(seq ? xseq : xpar);
    const size_t s0b = (size_t)E * S0P * 2;
    s0l = !seq && o + s0b <= WIDE_LDS_MAX;
    o_S0 = s0l ? take(s0b) : 0;
    // epilogue reuse of [big0, total): the NW waves' read-out partial tiles,
    // then pair 1's memory partials
    const size_t ro = (size_t)NW * (TJh > TI ? TJh : TI) * 16 * WAVE * sizeof(float);
    const size_t lx = (size_t)2 * TI * TJh * 16 * WAVE * sizeof(float);
    const size_t need = big0 + (ro > lx ? ro : lx);
    total = o > need ? o : need;
  }
};

// SEQ and S0L must be the layout's seq and s0l for (p.cs, p.ts, p.nsl).
template <int D, int E, int MAT, bool SEQ, bool S0L>
__global__ void __launch_bounds__(NTHREADS)
__attribute__((amdgpu_waves_per_eu(1, 1)))
phase_wide_kernel(ScanArgs p) {
  using M = ModeF16;
  constexpr int EH = E / 2, TI = D / 32, TJh = EH / 32, KPT = M::KPT;
  constexpr int TJ = E / 32, NTh = TI * TJh;
  using elem = typename M::elem;
  using frag = typename M::frag;
  using LY = WideLayout<D, E>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const LY L(p.cs, p.ts, p.nsl);

  const int lb = xcd_block();
  const int stream = lb / p.nsl, j = lb % p.nsl;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, wv = wave_id();
  const int pair = wv >> 1, half = wv & 1;
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, n = tok0 + ts;
  const long long sDE = (long long)stream * D * E;

  elem* ctil = reinterpret_cast<elem*>(smem + L.o_ctil);
  float* sm = reinterpret_cast<float*>(smem + L.o_small);
  float* mrow = sm;
  float* thp = sm + p.ts;
  float* Apre = sm + 2 * p.ts;
  float* ass = sm + 4 * p.ts;
  float* ait = ass + p.ts * p.ts;
  float* red4 = ait + p.nsl * p.ts;
  elem* Ut = reinterpret_cast<elem*>(smem + L.o_Ut);
  elem* Vt = reinterpret_cast<elem*>(smem + L.o_Vt);
  elem* Qs = reinterpret_cast<elem*>(smem + L.o_Qs);
  elem* Gs = reinterpret_cast<elem*>(smem + L.o_Gs);
  float* xch = reinterpret_cast<float*>(smem + L.o_xch);
  // SEQ: one fp32 slot per pair.  Otherwise two sets of one fp16 slot per
  // wave (LY::XSLOT halves each; set s of wave w at float offset
  // (s * NW + w) * XSLOT / 2), used alternately by the pair's exchanges (xk
  // counts them, polar_express_pair_sym)
  float* mine = xch + pair * D * D;
  constexpr int XSF = LY::XSLOT / 2, XSET = NW * XSF;   // floats per slot, per set
  int xk = 0;
  _Float16* S0h = reinterpret_cast<_Float16*>(smem + L.o_S0);

  // ---- staging (as phase_kernel, without the chunk-start momentum) -------
  const long long tb = chunk_table(p, stream, p.chunk);
  {
    constexpr int CF4 = TS_MAX * CS_MAX / 4 / NTHREADS;
    constexpr int UF4 = D * CS_MAX / 4 / NTHREADS, VF4 = E * CS_MAX / 4 / NTHREADS;
    const float* Usrc = (MAT == 2 ? p.kT : p.errT) + (long long)stream * D * cs;
    const float* Vsrc = (MAT == 2 ? p.chainT : p.actT) + (long long)stream * E * cs;
    f32x4 cv[CF4], uv[UF4], vv[VF4];
    TokenRows<D, 32> qr;
    load_rows4<CF4>(cv, p.cmt + tb * cs * cs + (long long)tok0 * cs, ts, n, cs);
    load_rows4<UF4>(uv, Usrc, D, n, cs);
    load_rows4<VF4>(vv, Vsrc, E, n, cs);
    qr.load(p, p.q, b, hh, tok0, ts);

    const float* am = p.am + tb * cs * cs;
    if (tid < ts) {
      mrow[tid] = p.cm[tb * cs + tok0 + tid];
      thp[tid] = p.thp[tb * cs + tok0 + tid];
      Apre[tid] = p.ap[tb * cs + tok0 + tid];
    }
    for (int idx = tid; idx < ts * ts; idx += NTHREADS) {
      const int s_ = idx / ts, t_ = idx % ts;
      ass[idx] = am[(tok0 + t_) * cs + tok0 + s_];
    }
    for (int idx = tid; idx < j * ts; idx += NTHREADS) {
      const int i = idx / ts, t_ = idx % ts;
      ait[idx] = am[(tok0 + t_) * cs + (i + 1) * ts - 1];
    }
    store_rows4<M, CF4>(cv, ctil, ts, n, L.csp, 1.f);
    const float su = pow2_scale(block_max<NW>(maxabs4<UF4>(uv, D, n), red4));
    const float sv = pow2_scale(block_max<NW>(maxabs4<VF4>(vv, E, n), red4 + NW));
    store_rows4<M, UF4>(uv, Ut, D, n, L.csp, su);
    store_rows4<M, VF4>(vv, Vt, E, n, L.csp, sv);
    const int npad = ((n + M::KB - 1) / M::KB) * M::KB;
    if (npad > n) {
      const int w = npad - n;
      for (int i = tid; i < (D + E + ts) * w; i += NTHREADS) {
        const int r = i / w, t = n + i % w;
        if (r < D) Ut[r * L.csp + t] = M::to_elem(0.f);
        else if (r < D + E) Vt[(r - D) * L.csp + t] = M::to_elem(0.f);
        else ctil[(r - D - E) * L.csp + t] = M::to_elem(0.f);
      }
    }
    if (tid == 0) red4[2 * NW] = 1.f / (su * sv);
    qr.template store<elem>(Qs, LY::QSP, p.io_dtype);
    if constexpr (S0L) {
      // S_0 [e][d] as fp16 rows scaled by a power of two (after the operand
      // rows, whose registers are free by now)
      // Two passes of at most eight quads per thread (the maximum, then the
      // scaled stores after reloading from L2) keep the staging's register
      // peak below the file.
      const f32x4* Sg = reinterpret_cast<const f32x4*>((MAT == 2 ? p.S2[p.cur] : p.S1T[p.cur]) + sDE);
      constexpr int SF4 = D * E / 4 / NTHREADS, SB = SF4 < 8 ? SF4 : 8;
      static_assert(SF4 % SB == 0, "S_0 staging: whole batches");
      float m = 0.f;
      for (int u0 = 0; u0 < SF4; u0 += SB) {
        f32x4 s4[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) s4[u] = Sg[tid + (u0 + u) * NTHREADS];
#pragma unroll
        for (int u = 0; u < SB; ++u)
#pragma unroll
          for (int k = 0; k < 4; ++k) m = fmaxf(m, fabsf(s4[u][k]));
      }
      const float s0 = pow2_scale(block_max<NW>(m, red4 + 2 * NW + 1));
      for (int u0 = 0; u0 < SF4; u0 += SB) {
        f32x4 s4[SB];
#pragma unroll
        for (int u = 0; u < SB; ++u) s4[u] = Sg[tid + (u0 + u) * NTHREADS];
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const int i = 4 * (tid + (u0 + u) * NTHREADS), e = i / D, d = i % D;
          *reinterpret_cast<f16x4*>(S0h + e * LY::S0P + d) =
              f16x4{(_Float16)(s4[u][0] * s0), (_Float16)(s4[u][1] * s0), (_Float16)(s4[u][2] * s0),
                    (_Float16)(s4[u][3] * s0)};
        }
      }
      if (tid == 0) red4[2 * NW + 1 + NW] = 1.f / s0;
    }
  }
  __syncthreads();
  const float inv_uv = red4[2 * NW];
  const float inv_s0 = S0L ? red4[2 * NW + 1 + NW] : 1.f;

  // ---- read-out partial accumulators -----------------------------------
  // MAT 2: this wave's E-tiles half*TJh + q of h; MAT 1: the D-tiles of y
  // (partial over this wave's half of the E contraction).
  constexpr int TR = (MAT == 2) ? TJh : TI;
  f32x16 RO[TR];   // read-out partials (AGPRs)
  agpr_init(RO);
  auto load_qf = [&](int K, int kb) -> frag { return M::ld_cslot(Qs + c * LY::QSP + 32 * K, kb, h); };
  const float wA = (c < ts) ? Apre[c] : 0.f;

  if (MAT == 2) {
    // hloc init A_t * W2 q_t: the half's tiles alternate between the pairs
    const float* W2c = p.W2[p.cur] + sDE;
#pragma unroll
    for (int q = 0; q < TJh; ++q) {
      if ((q & 1) != pair) continue;
      const int Ie = half * TJh + q;
      frag wf[TI][KPT];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) wf[K][kb] = M::gl_cslot(W2c + (32 * Ie + c) * D + 32 * K, kb, h);
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) agpr_mfma(RO[q], wf[K][kb], M::scale(load_qf(K, kb), wA));
    }
  } else {
    const float* W1c = p.W1[p.cur] + sDE;
    constexpr int QJ = (TJ + NW - 1) / NW;
    frag w1f[QJ][TI][KPT];
#pragma unroll
    for (int q = 0; q < QJ; ++q) {
      const int Je = wv + q * NW;
#pragma unroll
      for (int Id = 0; Id < TI; ++Id)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb)
          w1f[q][Id][kb] = M::gl_contig(W1c + (32 * Id + c) * E + 32 * (Je < TJ ? Je : 0), kb, h);
    }
    // h for the slice: hloc_j + sum_{i<j} a(end_i->t) L2_i^T q_t, then g = gelu(h)
    const float* hl = p.hloc + (((long long)stream * p.nsl + j) * ts) * E;
#pragma unroll
    for (int q = 0; q < QJ; ++q) {
      const int Ie = wv + q * NW;
      if (Ie >= TJ) break;
      f32x16 acc;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x4 v = (c < ts) ? *reinterpret_cast<const f32x4*>(hl + (long long)c * E + 32 * Ie + 8 * g4 + 4 * h)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[4 * g4 + u] = v[u];
      }
      // earlier slices: sum_{i<j} a(e_i -> t) L2_i^T q_t, directly or as
      // a(e_{j-1} -> t) M2_j^T q_t (slice prefix in slot j of L2)
      for (int i0 = 0; !p.use_prefix && i0 < j; i0 += 4) {
        frag lf[4][TI][KPT];
#pragma unroll
        for (int di = 0; di < 4; ++di) {
          const int i = (i0 + di < j) ? i0 + di : i0;
          const float* L2i = p.L2 + ((long long)stream * p.nsl + i) * D * E;
#pragma unroll
          for (int K = 0; K < TI; ++K)
#pragma unroll
            for (int kb = 0; kb < KPT; ++kb) lf[di][K][kb] = M::gl_cslot(L2i + (32 * Ie + c) * D + 32 * K, kb, h);
        }
#pragma unroll
        for (int di = 0; di < 4; ++di) {
          if (i0 + di >= j) break;
          const float wi = (c < ts) ? ait[(i0 + di) * ts + c] : 0.f;
#pragma unroll
          for (int K = 0; K < TI; ++K)
#pragma unroll
            for (int kb = 0; kb < KPT; ++kb) acc = M::mma(lf[di][K][kb], M::scale(load_qf(K, kb), wi), acc);
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
          for (int kb = 0; kb < KPT; ++kb) acc = M::mma(lf[K][kb], M::scale(load_qf(K, kb), wi), acc);
      }
      float* gout = p.g + ((long long)stream * cs + tok0 + c) * E;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        f32x4 gv;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * g4 + u, e = 32 * Ie + crow(r, h);
          gv[u] = (c < ts) ? gelu_tanh(acc[r]) : 0.f;
          Gs[c * LY::GSP + e] = M::to_elem(gv[u]);
        }
        if (c < ts) *reinterpret_cast<f32x4*>(gout + 32 * Ie + 8 * g4 + 4 * h) = gv;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < QJ; ++q) {
      const int Je = wv + q * NW;
      if (Je >= TJ) break;
#pragma unroll
      for (int Id = 0; Id < TI; ++Id)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb)
          agpr_mfma(RO[Id], w1f[q][Id][kb], M::scale(M::ld_contig(Gs + c * LY::GSP + 32 * Je, kb, h), wA));
    }
  }

  // ---- per-token momentum, Polar-Express, memory and read-out partials ---
  const int tpp = ts / 2;
  const int nkb = (n + M::KB - 1) / M::KB;
  const float* Sc = (MAT == 2 ? p.S2[p.cur] : p.S1T[p.cur]) + sDE;
  f32x16 Lw[TI][TJh];   // this wave's share of L_j (AGPRs), tiles of X's layout
#pragma unroll
  for (int I = 0; I < TI; ++I) agpr_init(Lw[I]);
  for (int it = 0; it < tpp; ++it) {
    const int sl = pair * tpp + it;   // slice-local token
    const int t = tok0 + sl;          // chunk-local token
    f32x16 X[TI][TJh];
    const elem* crowp = ctil + sl * L.csp;
    auto s_block = [&](int kb, bool first) {
      const frag cf = M::ld_contig(crowp, kb, h);
      frag uf[TI];
#pragma unroll
      for (int I = 0; I < TI; ++I) uf[I] = M::scale_v(M::ld_contig(Ut + (32 * I + c) * L.csp, kb, h), cf);
#pragma unroll
      for (int J = 0; J < TJh; ++J) {
        const frag vf = M::ld_contig(Vt + (32 * (half * TJh + J) + c) * L.csp, kb, h);
#pragma unroll
        for (int I = 0; I < TI; ++I) X[I][J] = M::mma(uf[I], vf, first ? zero16() : X[I][J]);
      }
    };
    s_block(0, true);
    for (int kb = 1; kb < nkb; ++kb) s_block(kb, false);
    // S_t = th * S_0 + f * Y, S_0 in [e][d] form (S2, and the transposed copy
    // of S1): from the fp16 LDS copy, or from global memory with four
    // consecutive d per 16-byte load (always for the chunk's last token)
    const float f = mrow[sl] * inv_uv;
    const float th = thp[sl];
    const bool carried = j == p.nsl - 1 && t == cs - 1;
    if (S0L && !carried) {
      const float ths = th * inv_s0;
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJh; ++J)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const f16x4 sp =
                *reinterpret_cast<const f16x4*>(S0h + (32 * (half * TJh + J) + c) * LY::S0P + 32 * I + 8 * q4 + 4 * h);
#pragma unroll
            for (int u = 0; u < 4; ++u) X[I][J][4 * q4 + u] = ths * (float)sp[u] + f * X[I][J][4 * q4 + u];
          }
    } else {
      // the lane's offset formed here (opaque): per-element addresses are not
      // hoisted out of the token loop into registers Polar-Express needs
      const float* Sl = Sc + PEWaveT<D, EH>::opaque((32 * half * TJh + c) * D + 4 * h);
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJh; ++J) {
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const f32x4 sp = *reinterpret_cast<const f32x4*>(Sl + 32 * J * D + 32 * I + 8 * q4);
#pragma unroll
            for (int u = 0; u < 4; ++u) X[I][J][4 * q4 + u] = th * sp[u] + f * X[I][J][4 * q4 + u];
          }
          // with S0L this path serves one token per chunk: one tile's loads
          // at a time, so that it does not set the kernel's register peak
          if constexpr (S0L) asm volatile("" ::: "memory");
        }
    }
    if (carried) {
      // S2, and S1 in its transposed [e][d] copy (the scan's S1 result is
      // transposed back after the last chunk)
      float* Sn = (MAT == 2 ? p.S2[p.cur ^ 1] : p.S1T[p.cur ^ 1]) + sDE +
                  PEWaveT<D, EH>::opaque((32 * half * TJh + c) * D + 4 * h);
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJh; ++J)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            f32x4 v4;
#pragma unroll
            for (int u = 0; u < 4; ++u) v4[u] = X[I][J][4 * q4 + u];
            *reinterpret_cast<f32x4*>(Sn + 32 * J * D + 32 * I + 8 * q4) = v4;
          }
    }

    // one fp16 slot per wave: the symmetric step with the Gram's operands
    // staged through the slot; the shared fp32 slot (SEQ): Gram operands
    // transposed on the matrix cores
    float pscale;   // X * pscale = P
    if constexpr (SEQ) pscale = polar_express_pair<M, D, EH, true>(X, p.ns, 1e-12f, nullptr, mine, mine, half);
    else pscale = polar_express_pair_sym<D, EH>(X, p.ns, 1e-12f, xch + wv * XSF, xch + (wv ^ 1) * XSF, XSET, xk);

    const float aend = ass[sl * ts + ts - 1] * pscale;
    const float wt = (c < ts) ? ass[sl * ts + c] * pscale : 0.f;
    // memory partial += a(s->end_j) P in AGPRs: (a I) * bf16(P) on the matrix
    // cores (bf16 keeps fp32's exponent range for tiny P)
    {
      bf16x8 aid[KPT];
#pragma unroll
      for (int kb = 0; kb < KPT; ++kb) aid[kb] = M::a_identity(kb, c, h, aend);
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJh; ++J)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) agpr_mfma_bf16(Lw[I][J], aid[kb], M::a_from_c(X[I][J], kb));
    }
    if (MAT == 2) {
      // hloc[e][t'] += sum_d P2[e][d] q_t'[d] w(t') over this wave's e
#pragma unroll
      for (int J = 0; J < TJh; ++J)
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            agpr_mfma(RO[J], M::from_c(X[K][J], kb), M::scale(load_qf(K, kb), wt));
    } else if constexpr (S0L || SEQ) {
      // yloc[d][t'] += sum_{e in this half} P1[d][e] g_t'[e] w(t') (P1 rows via
      // the identity-product transpose: with S_0 in LDS this measured 4 us per
      // C3 launch faster than the staged transpose below; with the sequential
      // exchange the pair's one slot is still being read by half 0 after the
      // exchange's last barrier, so it cannot take a staged block)
      frag idf[KPT];
#pragma unroll
      for (int kb = 0; kb < KPT; ++kb) idf[kb] = M::identity(kb, c, h);
#pragma unroll
      for (int Je = 0; Je < TJh; ++Je) {
        frag gw[KPT];
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb)
          gw[kb] = M::scale(M::ld_cslot(Gs + c * LY::GSP + 32 * (half * TJh + Je), kb, h), wt);
#pragma unroll
        for (int Id = 0; Id < TI; ++Id) {
          f32x16 tt = zero16();
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) tt = M::mma(M::from_c(X[Id][Je], kb), idf[kb], tt);
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) agpr_mfma(RO[Id], M::from_c(tt, kb), gw[kb]);
        }
      }
    } else {
      // the same, with block Je of P1 staged as fp16 rows e in the wave's
      // exchange slot that the partner is not reading (the one the next
      // exchange writes, after these reads); transposing reads give P1[d][e]
      // with d along the lanes and e along the registers, as in
      // phase16_kernel's read-out (C5: 306.7 instead of 312.2 us per W1 launch)
      using PS = PEWaveT<D, EH>;
      _Float16* buf = reinterpret_cast<_Float16*>(xch + (xk & 1) * XSET + wv * XSF);
      const int wo = PS::opaque(PS::wr_off()), ro = PS::opaque(PS::rd_off());
#pragma unroll
      for (int Je = 0; Je < TJh; ++Je) {
#pragma unroll
        for (int Id = 0; Id < TI; ++Id)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) {
            const frag xf = M::from_c(X[Id][Je], kb);
            // elements 4g..4g+3 of the fragment are rows 32Id + 16kb + 8g + 4h + 0..3
#pragma unroll
            for (int g = 0; g < 2; ++g)
              *reinterpret_cast<f16x4*>(buf + wo + 32 * Id + 16 * kb + 8 * g) =
                  f16x4{xf[4 * g], xf[4 * g + 1], xf[4 * g + 2], xf[4 * g + 3]};
          }
        frag th[TI][KPT], gw[KPT];
        PS::read_block(th, buf, ro);
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb)
          gw[kb] = M::scale(M::ld_contig(Gs + c * LY::GSP + 32 * (half * TJh + Je), kb, h), wt);
#pragma unroll
        for (int Id = 0; Id < TI; ++Id)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) agpr_mfma(RO[Id], th[Id][kb], gw[kb]);
      }
    }
  }

  // ---- epilogue ----------------------------------------------------------
  agpr_mfma_drain(RO);
#pragma unroll
  for (int I = 0; I < TI; ++I) agpr_mfma_drain(Lw[I]);
  auto lw_quad = [&](int tl, int q) {
    const f32x16& t = Lw[tl / TJh][tl % TJh];
    return f32x4{t[4 * q], t[4 * q + 1], t[4 * q + 2], t[4 * q + 3]};
  };
  __syncthreads();
  constexpr int RW = (MAT == 2) ? E : D;
  float* ro_out = (MAT == 2 ? p.hloc : p.yloc) + (((long long)stream * p.nsl + j) * ts) * RW;
  float* Lout = (MAT == 2 ? p.L2 : p.L1) + ((long long)stream * p.nsl + j) * D * E;
  float* ros = reinterpret_cast<float*>(smem + L.o_Ut);
#pragma unroll
  for (int q = 0; q < TR; ++q)
#pragma unroll
    for (int r = 0; r < 16; ++r) ros[((wv * TR + q) * 16 + r) * WAVE + lane] = RO[q][r];
  __syncthreads();
  // read-out partial rows t' < ts: element (t', x) sits at register r of lane
  // t' + 32 hx with x % 32 = 8 (r / 4) + 4 hx + r % 4; summed over the waves
  // that hold its tile, in wave order
  for (int i = tid; i < ts * RW; i += NTHREADS) {
    const int tp = i / RW, x = i % RW;
    const int xt = x >> 5, xl = x & 31, hx = (xl >> 2) & 1, r = 4 * (xl >> 3) + (xl & 3);
    const int ln = tp + 32 * hx;
    float acc;
    if (MAT == 2) {
      const int hf = xt / TJh, q = xt % TJh;
      acc = ros[(((0 + hf) * TR + q) * 16 + r) * WAVE + ln] + ros[(((2 + hf) * TR + q) * 16 + r) * WAVE + ln];
    } else {
      acc = ros[((0 * TR + xt) * 16 + r) * WAVE + ln];
#pragma unroll
      for (int w = 1; w < NW; ++w) acc += ros[((w * TR + xt) * 16 + r) * WAVE + ln];
    }
    ro_out[i] = acc;
  }
  __syncthreads();
  // memory partial: pair 1's quads through LDS, pair 0 adds (pair 0 first) and
  // stores L_j in the state layout (L2 as [e][d], L1 as [d][e])
  f32x4* lx = reinterpret_cast<f32x4*>(smem + L.o_Ut);
  if (pair == 1) {
#pragma unroll
    for (int tl = 0; tl < NTh; ++tl)
#pragma unroll
      for (int q = 0; q < 4; ++q) lx[((half * NTh + tl) * 4 + q) * WAVE + lane] = lw_quad(tl, q);
  }
  __syncthreads();
  if (pair == 0) {
#pragma unroll
    for (int tl = 0; tl < NTh; ++tl)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = lw_quad(tl, q) + lx[((half * NTh + tl) * 4 + q) * WAVE + lane];
        const int d0 = 32 * (tl / TJh) + 8 * q + 4 * h, e = 32 * (half * TJh + tl % TJh) + c;
        if (MAT == 2) {
          *reinterpret_cast<f32x4*>(Lout + (long long)e * D + d0) = v;
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u) Lout[(long long)(d0 + u) * E + e] = v[u];
        }
      }
  }
}

// dst[s][c][r] = src[s][r][c] for R x C matrices (the momentum S1 into and
// out of its transposed form; 32 x 32 tiles through LDS).
// Grid: streams * (R/32) * (C/32), 256 threads.
template <int R, int C>
__global__ void __launch_bounds__(256) transpose_kernel(const float* src, float* dst) {
  __shared__ float tile[32][33];
  constexpr int TI = R / 32, TJ = C / 32;
  const int blk = blockIdx.x % (TI * TJ);
  const long long s = blockIdx.x / (TI * TJ);
  const int I = blk / TJ, J = blk % TJ;
  const float* a = src + s * R * C;
  float* o = dst + s * R * C;
  const int x = threadIdx.x & 31, y0 = threadIdx.x >> 5;
#pragma unroll
  for (int y = y0; y < 32; y += 8) tile[y][x] = a[(long long)(32 * I + y) * C + 32 * J + x];
  __syncthreads();
#pragma unroll
  for (int y = y0; y < 32; y += 8) o[(long long)(32 * J + y) * R + 32 * I + x] = tile[x][y];
}

}  // namespace atlas
