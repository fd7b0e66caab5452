// The per-chunk tail on blocks of eight waves (D = 64, E <= 128, slice
// partials summed directly): one launch holding
//   - the prep of chunk p.chunk (blocks [0, n_prep), 32 tokens each), which
//     first forms that chunk's start weights from the previous chunk's state
//     and slice partials itself,
//         W = A_end W_prev + sum_j a(e_j -> end) L_j      (memory_layer.py:566-590)
//     into LDS (the stream's first block also writes W to the state buffer
//     the next phase kernels and the next tail read), and then computes the
//     inner-gradient factors of _process_chunk_deep (memory_layer.py:505-520)
//     as prep_body does, each fp32 MFMA contraction split over the eight
//     waves (partial tiles summed in a fixed order through LDS);
//   - y of the previous chunk (the remaining blocks, two slices per block:
//     waves 0-3 and 4-7), as fin_body's read-out part.
// This replaces the W_end launch and the four-wave tail of tail_kernel: W no
// longer round-trips through memory between two kernels before the prep can
// load it, and the prep's three product chains are half as long.
#pragma once

#include "atlas_scan_kernels.hpp"

namespace atlas {

constexpr int NT8 = 512;   // threads of a tail8 block

template <int D, int E>
struct Prep8L {            // LDS layout (floats)
  static constexpr int KS = D + 4, ES = E + 4;
  static constexpr int o_K = 0;                      // K rows  [32][KS]
  static constexpr int o_V = o_K + 32 * KS;          // V rows  [32][KS]
  static constexpr int o_R = o_V + 32 * KS;          // Err rows [32][KS]
  static constexpr int o_A = o_R + 32 * KS;          // Act rows [32][ES]
  static constexpr int o_W1 = o_A + 32 * ES;         // W1 [D][ES]
  static constexpr int o_W2 = o_W1 + D * ES;         // W2 [E][KS]
  static constexpr int o_P = o_W2 + E * KS;          // partial tiles [8 waves][16][64]
  static constexpr int total = o_P + 8 * 16 * WAVE;
  static constexpr size_t bytes() { return (size_t)total * sizeof(float); }
};

template <int D, int E>
__device__ __forceinline__ void prep8_body(const ScanArgs& p, int lb) {
  static_assert(D == 64 && (E == 64 || E == 128), "prep8: D 64, E 64 or 128");
  using L = Prep8L<D, E>;
  constexpr int KS = L::KS, ES = L::ES;
  constexpr int TI = D / 32, TJ = E / 32;
  constexpr int KP = 8 / TJ;             // parts of the D contraction (H, Chain)
  constexpr int KL = D / KP / 2;         // contraction elements per lane half and part
  constexpr int NPE = 8 / TI;            // parts of the E contraction (Err)
  constexpr int EL = E / NPE / 2;
  constexpr int RP = 16 / KP, RE = 16 / NPE;   // tile rows each wave finishes
  static_assert(KL % 4 == 0 && EL % 4 == 0, "16-byte operand reads");
  extern __shared__ float lds[];
  float* Ks = lds + L::o_K;
  float* Vs = lds + L::o_V;
  float* Rs = lds + L::o_R;
  float* As = lds + L::o_A;
  float* W1s = lds + L::o_W1;
  float* W2s = lds + L::o_W2;
  float* Ps = lds + L::o_P;

  const int nblk = (p.cs + 31) / 32;
  const int stream = lb / nblk, blk = lb % nblk;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, w = wave_id();
  const int t0 = blk * 32, cs = p.cs;
  const long long sDE = (long long)stream * D * E;

  // ---- every global load in flight: token rows, then the previous chunk's
  // state, slice partials and gate weights
  const int nt = min(32, cs - t0);
  TokenRows<D, 32> kr, vr;   // (written for 256 threads: the upper half idles)
  kr.load(p, p.k, b, hh, t0, nt);
  vr.load(p, p.v, b, hh, t0, nt);
  asm volatile("" ::: "memory");
  constexpr int N4 = D * E / 4;                      // quads per matrix
  constexpr int NQ = 2 * N4 / NT8;                   // quads per thread (both matrices)
  constexpr int NSD = 4;                             // slices summed directly (<= 4)
  const int nsl = p.nsl, ts = p.ts, pc = p.cur ^ 1;  // the previous chunk's buffer
  const long long tb = chunk_table(p, stream, p.chunk - 1);
  const float* am = p.am + tb * cs * cs;
  const float Aend = p.ap[tb * cs + cs - 1];
  float aend[NSD];
#pragma unroll
  for (int s = 0; s < NSD; ++s) aend[s] = (s < nsl) ? am[(cs - 1) * cs + (s + 1) * ts - 1] : 0.f;
  f32x4 wq[NQ];
  f32x4 lq[NQ][NSD];
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = tid + u * NT8, m = i / N4, iq = i % N4;   // matrix m (0: W1, 1: W2), quad iq
    const float* Wp = (m == 0 ? p.W1[pc] : p.W2[pc]) + sDE;
    const float* Lm = (m == 0 ? p.L1 : p.L2) + (long long)stream * nsl * D * E;
    wq[u] = reinterpret_cast<const f32x4*>(Wp)[iq];
#pragma unroll
    for (int s = 0; s < NSD; ++s) lq[u][s] = reinterpret_cast<const f32x4*>(Lm)[(long long)(s < nsl ? s : 0) * N4 + iq];
  }
  // W = A_end W_prev + sum_s a(e_s -> end) L_s, the sum over s in order (as
  // fin_body forms it)
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int i = tid + u * NT8, m = i / N4, iq = i % N4;
    f32x4 a = Aend * wq[u];
#pragma unroll
    for (int s = 0; s < NSD; ++s)
      if (s < nsl) a += aend[s] * lq[u][s];
    if (m == 0) {   // W1 [d][e]
      const int d = (4 * iq) / E, e = (4 * iq) % E;
      *reinterpret_cast<f32x4*>(W1s + d * ES + e) = a;
    } else {        // W2 [e][d]
      const int e = (4 * iq) / D, d = (4 * iq) % D;
      *reinterpret_cast<f32x4*>(W2s + e * KS + d) = a;
    }
    if (blk == 0) reinterpret_cast<f32x4*>((m == 0 ? p.W1[p.cur] : p.W2[p.cur]) + sDE)[iq] = a;
  }
  kr.store(Ks, KS, p.io_dtype);
  vr.store(Vs, KS, p.io_dtype);
  __syncthreads();

  // ---- H^T [e][t] = W2 K^T: wave w takes E-tile Ie and part kp of the D
  // contraction; lane half h a contiguous half of the part
  float gp[RP];   // gelu'(H) of the rows this wave finishes
  const int Ie = w % TJ, kp = w / TJ;
  {
    f32x16 acc = zero16();
    const int k0 = kp * (D / KP) + h * KL;
#pragma unroll
    for (int j = 0; j < KL / 4; ++j) {
      const f32x4 wv = *reinterpret_cast<const f32x4*>(W2s + (32 * Ie + c) * KS + k0 + 4 * j);
      const f32x4 kv = *reinterpret_cast<const f32x4*>(Ks + c * KS + k0 + 4 * j);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = ModeF32::mma(wv[u], kv[u], acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Ps[(w * 16 + r) * WAVE + lane] = acc[r];
  }
  __syncthreads();
  // wave (Ie, kp) finishes rows r = kp * RP + rr of tile Ie: the KP partials
  // summed in part order, then the GELUs
#pragma unroll
  for (int rr = 0; rr < RP; ++rr) {
    const int r = kp * RP + rr;
    float x = 0.f;
#pragma unroll
    for (int q = 0; q < KP; ++q) x += Ps[((q * TJ + Ie) * 16 + r) * WAVE + lane];
    const int e = 32 * Ie + crow(r, h);
    As[c * ES + e] = gelu_tanh(x);
    gp[rr] = gelu_erf_prime(x);
  }
  __syncthreads();

  // ---- Err^T [d][t] = W1 Act^T + K^T - V^T: wave w takes D-tile Id and part
  // pe of the E contraction
  const int Id = w % TI, pe = w / TI;
  {
    f32x16 acc = zero16();
    const int e0 = pe * (E / NPE) + h * EL;
#pragma unroll
    for (int j = 0; j < EL / 4; ++j) {
      const f32x4 wv = *reinterpret_cast<const f32x4*>(W1s + (32 * Id + c) * ES + e0 + 4 * j);
      const f32x4 av = *reinterpret_cast<const f32x4*>(As + c * ES + e0 + 4 * j);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = ModeF32::mma(wv[u], av[u], acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Ps[(w * 16 + r) * WAVE + lane] = acc[r];
  }
  __syncthreads();
#pragma unroll
  for (int rr = 0; rr < RE; ++rr) {
    const int r = pe * RE + rr;
    float x = 0.f;
#pragma unroll
    for (int q = 0; q < NPE; ++q) x += Ps[((q * TI + Id) * 16 + r) * WAVE + lane];
    const int d = 32 * Id + crow(r, h);
    Rs[c * KS + d] = x + Ks[c * KS + d] - Vs[c * KS + d];
  }
  __syncthreads();

  // ---- K, Err and Act as token-contiguous rows, four tokens per store
  {
    float* k_out = p.kT + (long long)stream * D * cs;
    float* err_out = p.errT + (long long)stream * D * cs;
    float* act_out = p.actT + (long long)stream * E * cs;
    for (int i = tid; i < D * 8; i += NT8) {
      const int d = i / 8, t = 4 * (i % 8);
      if (t < nt) {
        f32x4 rv, kv;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          rv[u] = Rs[(t + u) * KS + d];
          kv[u] = Ks[(t + u) * KS + d];
        }
        *reinterpret_cast<f32x4*>(err_out + (long long)d * cs + t0 + t) = rv;
        *reinterpret_cast<f32x4*>(k_out + (long long)d * cs + t0 + t) = kv;
      }
    }
    for (int i = tid; i < E * 8; i += NT8) {
      const int e = i / 8, t = 4 * (i % 8);
      if (t < nt) {
        f32x4 av;
#pragma unroll
        for (int u = 0; u < 4; ++u) av[u] = As[(t + u) * ES + e];
        *reinterpret_cast<f32x4*>(act_out + (long long)e * cs + t0 + t) = av;
      }
    }
  }

  // ---- Chain^T [e][t] = (W1^T Err^T) * gelu': the same (tile, part) split
  // as H, so each wave finishes the rows whose gelu' it holds
  {
    f32x16 acc = zero16();
    const int k0 = kp * (D / KP) + h * KL;
#pragma unroll
    for (int j = 0; j < KL / 4; ++j) {
      const f32x4 rv = *reinterpret_cast<const f32x4*>(Rs + c * KS + k0 + 4 * j);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = ModeF32::mma(W1s[(k0 + 4 * j + u) * ES + 32 * Ie + c], rv[u], acc);
    }
    // the partial-tile slots were last read before the Rs barrier
#pragma unroll
    for (int r = 0; r < 16; ++r) Ps[(w * 16 + r) * WAVE + lane] = acc[r];
  }
  __syncthreads();
  float* chain_out = p.chainT + (long long)stream * E * cs;
  const int tl = t0 + c;
  if (tl < cs) {
#pragma unroll
    for (int rr = 0; rr < RP; ++rr) {
      const int r = kp * RP + rr;
      float x = 0.f;
#pragma unroll
      for (int q = 0; q < KP; ++q) x += Ps[((q * TJ + Ie) * 16 + r) * WAVE + lane];
      chain_out[(long long)(32 * Ie + crow(r, h)) * cs + tl] = x * gp[rr];
    }
  }
}

// y of slice j (waves 4 * half .. 4 * half + 3 of a tail8 block), as the
// read-out part of fin_body; `live` false for a half without a slice (it
// still takes part in the block barrier).
template <class M, int D, int E>
__device__ __forceinline__ void fin_y_half(const ScanArgs& p, int stream, int j, int half, bool live,
                                           float* part_acc, float* ait) {
  constexpr int TI = D / 32, TJ = E / 32, KPT = M::KPT;
  constexpr int NP = NW / TI;                 // waves per D-tile (E split for the read-out)
  constexpr int JP = (TJ + NP - 1) / NP;      // E-tiles per wave
  using frag = typename M::frag;
  const int b = stream / p.H, hh = stream % p.H;
  const int lane = lane_id(), c = lane & 31, h = lane >> 5, wv = wave_id() - 4 * half, tq = threadIdx.x - NTHREADS * half;
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, nsl = p.nsl;
  if (live) {
    const long long tb = chunk_table(p, stream, p.chunk);
    const float* am = p.am + tb * cs * cs;
    for (int idx = tq; idx < j * ts; idx += NTHREADS) {
      const int i = idx / ts, t = idx % ts;
      ait[idx] = am[(tok0 + t) * cs + (i + 1) * ts - 1];
    }
  }
  __syncthreads();
  const int Id = wv % TI, part = wv / TI;
  f32x16 acc = zero16();
  if (live && j > 0) {
    const float* grow = p.g + ((long long)stream * cs + tok0 + ((c < ts) ? c : 0)) * E;
    frag gf[JP][KPT];
#pragma unroll
    for (int jj = 0; jj < JP; ++jj)
#pragma unroll
      for (int kb = 0; kb < KPT; ++kb) {
        const int Je = part * JP + jj;
        gf[jj][kb] = M::gl_contig(grow + 32 * (Je < TJ ? Je : 0), kb, h);
      }
    for (int i = 0; i < j; ++i) {
      const float* L1i = p.L1 + ((long long)stream * nsl + i) * D * E + (long long)(32 * Id + c) * E;
      const float wi = (c < ts) ? ait[i * ts + c] : 0.f;
#pragma unroll
      for (int jj = 0; jj < JP; ++jj) {
        const int Je = part * JP + jj;
        if (Je < TJ) {
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            acc = M::mma(M::gl_contig(L1i + 32 * Je, kb, h), M::scale(gf[jj][kb], wi), acc);
        }
      }
    }
  }
  if (NP > 1 && part >= 1) {
    float* slot = part_acc + ((Id * (NP - 1) + part - 1) * 16) * WAVE;
#pragma unroll
    for (int r = 0; r < 16; ++r) slot[r * WAVE + lane] = acc[r];
  }
  __syncthreads();
  if (live && part == 0) {
#pragma unroll
    for (int pp = 1; pp < NP; ++pp) {
      const float* slot = part_acc + ((Id * (NP - 1) + pp - 1) * 16) * WAVE;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += slot[r * WAVE + lane];
    }
    const int tl = tok0 + c;
    const int tg = p.chunk * cs + tl;
    if (c < ts && tg < p.T) {
      const float* yl = p.yloc + (((long long)stream * nsl + j) * ts + c) * D;
      const long long yo = (long long)b * p.xsb + (long long)tg * p.xst + (long long)hh * p.xsh;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * Id + 8 * g4 + 4 * h;     // rows crow(4*g4 + u, h) = d0 + u
        const f32x4 qv = load4_any(p.q, yo + d0, p.io_dtype);
        const f32x4 lv = *reinterpret_cast<const f32x4*>(yl + d0);
        f32x4 yv;
#pragma unroll
        for (int u = 0; u < 4; ++u) yv[u] = qv[u] + lv[u] + acc[4 * g4 + u];
        store4_any(p.y, yo + d0, p.io_dtype, yv);
      }
    }
  }
}

// Blocks [0, n_prep): prep8 of chunk p.chunk (which forms its start weights
// from chunk p.chunk - 1); the remaining blocks: y of chunk p.chunk - 1, two
// slices per block.  Each role numbers its blocks per XCD as xcd_block does.
template <class M, int D, int E>
__global__ void __launch_bounds__(NT8)
tail8_kernel(ScanArgs p, int n_prep) {
  constexpr int TI = D / 32, NP = NW / TI;
  constexpr int PA = TI * (NP - 1) * 16 * WAVE, AI = NSL_MAX * TS_MAX;
  static_assert(2 * (PA + AI) <= Prep8L<D, E>::total, "y slots inside the dynamic LDS");
  extern __shared__ float lds[];   // prep8's layout, or the y halves' slots
  constexpr int kXCD = 8;
  const int bx = blockIdx.x;
  auto xcd_index = [](int bi, int n) {
    const int x = bi % kXCD, q = n / kXCD, r = n % kXCD;
    return x * q + (x < r ? x : r) + bi / kXCD;
  };
  if (bx < n_prep) {
    prep8_body<D, E>(p, xcd_index(bx, n_prep));
  } else {
    ScanArgs pf = p;
    pf.chunk = p.chunk - 1;
    pf.cur = p.cur ^ 1;
    const int groups = (p.nsl + 1) / 2;
    const int lb = xcd_index(bx - n_prep, (int)gridDim.x - n_prep);
    const int stream = lb / groups, g = lb % groups, half = wave_id() / 4;
    const int j = 2 * g + half;
    fin_y_half<M, D, E>(pf, stream, j < p.nsl ? j : 0, half, j < p.nsl, lds + half * (PA + AI),
                        lds + half * (PA + AI) + PA);
  }
}

}  // namespace atlas
