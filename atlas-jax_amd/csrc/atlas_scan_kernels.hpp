// Kernels of the chunk scan (one launch set per chunk of cs tokens).
//
// For one (batch, head) stream and chunk with chunk-start state
// (W1 [D,E], W2 [E,D], S1 [D,E], S2 [E,D]) the reference loop body
// _process_chunk_deep (atlas_jax/memory_layer.py:496-597) is evaluated as:
//
//   prep   H = K W2^T, Act = gelu_tanh(H), Gp = gelu'_erf(H),
//          Err = K + Act W1^T - V, Chain = (Err W1) * Gp            (fp32 MFMA)
//   coef   c[t,i] = (2/D) g_i sum_{s=i}^{min(t,i+w-1)} theta(s->t) (-eta_s)
//          (the Omega window :233-253 and momentum scan :546-552 in closed form),
//          Theta_t = prod_{r<=t} theta_r, a(s->t) = prod_{s<r<=t} alpha_r
//   S_t    S1_t = Theta_t S1 + Err^T diag(c_t) Act,
//          S2_t^T = Theta_t S2^T + K^T diag(c_t) Chain                (MFMA)
//   PE     P_t = PolarExpress(S_t)  (one wave per token, S2 in transposed form)
//   W, y   the memory scan W_t = alpha_t W_{t-1} + P_t and the read-out
//          y_t = q_t + W1_t gelu(W2_t q_t) by linearity:
//          tokens are split into n_slices slices T_j (end token end_j);
//          L_j = sum_{s in T_j} a(s->end_j) P_s  and per-slice partial
//          read-outs, combined across slices in the finalize kernel.
//
// Launches per chunk: prep, phase<2> (W2 = first MLP layer: PE of S2 and h),
// phase<1> (W1: PE of S1 and y), finalize (y, W_end).  State is ping-ponged
// between the caller's buffers and the workspace (index cur / cur^1).
#pragma once

#include "atlas_common.hpp"
#include "atlas_pe.hpp"

namespace atlas {

constexpr int NW = 4;                 // waves per workgroup
constexpr int NTHREADS = NW * WAVE;
constexpr int CS_MAX = 128;
constexpr int TS_MAX = 32;
constexpr int NSL_MAX = 32;

struct ScanArgs {
  int B, T, H, D, E;
  int cs, w_eff, use_omega, ns;
  int nsl, ts, n_chunks;
  int io_dtype, gate_dtype;
  long long xsb, xst, xsh, gsb, gst;
  const void *q, *k, *v, *alpha, *eta, *theta, *gamma;
  void* y;
  float* W1[2];
  float* W2[2];
  float* S1[2];
  float* S2[2];
  float *err, *act, *chain;     // [stream][cs][D | E | E]
  float *L1, *L2;               // [stream][nsl][D*E]  (L1 as [D][E], L2 as [E][D])
  float *hloc, *yloc, *g;       // [stream][nsl][ts][E], [stream][nsl][ts][D], [stream][cs][E]
  int chunk, cur;
};

// Gate values of chunk-local token t (reference padding at memory_layer.py:655-659).
struct Gates {
  float a, e, th, g;
};
__device__ __forceinline__ Gates load_gates(const ScanArgs& p, int b, int hh, int tg) {
  Gates G;
  if (tg < p.T) {
    const long long o = (long long)b * p.gsb + (long long)tg * p.gst + hh;
    G.a = load_any(p.alpha, o, p.gate_dtype);
    G.e = load_any(p.eta, o, p.gate_dtype);
    G.th = load_any(p.theta, o, p.gate_dtype);
    G.g = p.use_omega ? load_any(p.gamma, o, p.gate_dtype) : 1.f;
  } else {
    G.a = 1.f; G.e = 0.f; G.th = 0.f; G.g = 0.f;
  }
  return G;
}

__device__ __forceinline__ float load_x(const ScanArgs& p, const void* x, int b, int tg, int hh, int d) {
  if (tg >= p.T) return 0.f;
  return load_any(x, (long long)b * p.xsb + (long long)tg * p.xst + (long long)hh * p.xsh + d, p.io_dtype);
}

// prod_{r=s+1}^{t} g[r]  (1 when t <= s)
__device__ __forceinline__ float seg_prod(const float* g, int s, int t) {
  float p = 1.f;
  for (int r = s + 1; r <= t; ++r) p *= g[r];
  return p;
}

// ===========================================================================
// prep: inner-gradient factors at the chunk-start weights, 32 tokens per WG.
// Grid: (streams * ceil(cs/32)).  fp32 MFMA (range and precision of the
// gradient factors matter: Polar-Express normalises whatever scale they have).
// ===========================================================================
template <int D, int E>
__global__ void __launch_bounds__(NTHREADS)
prep_kernel(ScanArgs p) {
  constexpr int TI = D / 32, TJ = E / 32;
  constexpr int KS = D + 1, ES = E + 1;   // LDS row strides (floats)
  extern __shared__ float lds[];
  float* W1s = lds;                  // [D][E+1]
  float* W2s = W1s + D * ES;         // [E][D+1]
  float* Ks = W2s + E * KS;          // [32][D+1]
  float* Vs = Ks + 32 * KS;          // [32][D+1]
  float* As = Vs + 32 * KS;          // [32][E+1]  Act
  float* Rs = As + 32 * ES;          // [32][D+1]  Err

  const int nblk = (p.cs + 31) / 32;
  const int stream = blockIdx.x / nblk, blk = blockIdx.x % nblk;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, w = wave_id();
  const int t0 = blk * 32;
  const long long sDE = (long long)stream * D * E;
  const float* W1 = p.W1[p.cur] + sDE;
  const float* W2 = p.W2[p.cur] + sDE;

  for (int i = tid; i < D * E; i += NTHREADS) {
    W1s[(i / E) * ES + (i % E)] = W1[i];
    W2s[(i / D) * KS + (i % D)] = W2[i];
  }
  for (int i = tid; i < 32 * D; i += NTHREADS) {
    const int t = i / D, d = i % D;
    const int tl = t0 + t;
    const int tg = p.chunk * p.cs + tl;
    const bool ok = tl < p.cs;
    Ks[t * KS + d] = ok ? load_x(p, p.k, b, tg, hh, d) : 0.f;
    Vs[t * KS + d] = ok ? load_x(p, p.v, b, tg, hh, d) : 0.f;
  }
  __syncthreads();

  // H^T tiles [e][t]: wave w owns E-tiles w, w+NW, ...; keeps gelu' in registers.
  f32x16 gp[(TJ + NW - 1) / NW];
#pragma unroll
  for (int q = 0; q < (TJ + NW - 1) / NW; ++q) {
    const int Ie = w + q * NW;
    if (Ie >= TJ) break;
    f32x16 acc = zero16();
    for (int kb = 0; kb < D / 2; ++kb)
      acc = ModeF32::mma(W2s[(32 * Ie + c) * KS + 2 * kb + h], Ks[c * KS + 2 * kb + h], acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int e = 32 * Ie + crow(r, h);
      const float x = acc[r];
      As[c * ES + e] = gelu_tanh(x);
      gp[q][r] = gelu_erf_prime(x);
    }
  }
  __syncthreads();

  // Err^T tiles [d][t] = W1 Act^T + K^T - V^T
#pragma unroll
  for (int q = 0; q < (TI + NW - 1) / NW; ++q) {
    const int Id = w + q * NW;
    if (Id >= TI) break;
    f32x16 acc = zero16();
    for (int kb = 0; kb < E / 2; ++kb)
      acc = ModeF32::mma(W1s[(32 * Id + c) * ES + 2 * kb + h], As[c * ES + 2 * kb + h], acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * Id + crow(r, h);
      Rs[c * KS + d] = acc[r] + Ks[c * KS + d] - Vs[c * KS + d];
    }
  }
  __syncthreads();

  // Chain^T tiles [e][t] = (W1^T Err^T) * gelu'
  float* chain_out = p.chain + ((long long)stream * p.cs) * E;
#pragma unroll
  for (int q = 0; q < (TJ + NW - 1) / NW; ++q) {
    const int Ie = w + q * NW;
    if (Ie >= TJ) break;
    f32x16 acc = zero16();
    for (int kb = 0; kb < D / 2; ++kb)
      acc = ModeF32::mma(W1s[(2 * kb + h) * ES + 32 * Ie + c], Rs[c * KS + 2 * kb + h], acc);
    const int tl = t0 + c;
    if (tl < p.cs) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int e = 32 * Ie + crow(r, h);
        chain_out[(long long)tl * E + e] = acc[r] * gp[q][r];
      }
    }
  }
  // Err and Act rows to the workspace (coalesced from LDS).
  float* err_out = p.err + ((long long)stream * p.cs) * D;
  float* act_out = p.act + ((long long)stream * p.cs) * E;
  for (int i = tid; i < 32 * D; i += NTHREADS) {
    const int t = i / D, d = i % D;
    if (t0 + t < p.cs) err_out[(long long)(t0 + t) * D + d] = Rs[t * KS + d];
  }
  for (int i = tid; i < 32 * E; i += NTHREADS) {
    const int t = i / E, e = i % E;
    if (t0 + t < p.cs) act_out[(long long)(t0 + t) * E + e] = As[t * ES + e];
  }
}

template <int D, int E>
constexpr size_t prep_lds_bytes() {
  return sizeof(float) * (size_t)(D * (E + 1) + E * (D + 1) + 2 * 32 * (D + 1) + 32 * (E + 1) + 32 * (D + 1));
}

// ===========================================================================
// Runtime LDS layout of the phase kernels (host and device agree on it).
// ===========================================================================
template <class M, int D, int E>
struct PhaseLayout {
  using elem = typename M::elem;
  static constexpr int EB = sizeof(elem);
  static constexpr int PADE = (EB == 2) ? 8 : 1;   // row padding in elements
  static constexpr int SPD = D + 4;                // Sp row stride (floats)
  static constexpr int QSP = D + PADE;             // Qs row stride
  static constexpr int GSP = E + PADE;             // Gs row stride
  int csp;                                         // token-row stride of Ut/Vt/ctil
  size_t o_gate, o_R, o_C, o_ctil, o_small, o_Ut, o_Vt, o_Sp, o_Qs, o_Gs, o_scr, total;
  size_t red_bytes;

  __host__ __device__ PhaseLayout(int cs) {
    const int npad = ((cs + 15) / 16) * 16;
    csp = npad + PADE;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t r = o; o += (bytes + 15) & ~size_t(15); return r; };
    o_gate = take(4 * CS_MAX * sizeof(float));
    o_ctil = take((size_t)TS_MAX * csp * EB);
    o_small = take((size_t)(TS_MAX * 4 + TS_MAX * TS_MAX + NSL_MAX * TS_MAX + 16) * sizeof(float));
    const size_t big0 = o;
    // prologue-only coefficient scratch, aliased by the operand buffers below
    o_R = big0;
    o_C = big0 + (((size_t)TS_MAX * (CS_MAX + 1) * sizeof(float) + 15) & ~size_t(15));
    const size_t coef_end = o_C + (size_t)TS_MAX * (CS_MAX + 1) * sizeof(float);
    o_Ut = take((size_t)D * csp * EB);
    o_Vt = take((size_t)E * csp * EB);
    o_Sp = take((size_t)E * SPD * sizeof(float));
    const size_t big1 = o;
    o_Qs = take((size_t)32 * QSP * EB);
    o_Gs = take((size_t)32 * GSP * EB);
    o_scr = take((size_t)NW * Scr<M>::template elems<D>() * EB);
    if (o < coef_end) o = coef_end;
    // the epilogue reduction reuses [big0, end): two D*E fp32 tiles
    red_bytes = 2 * (size_t)D * E * sizeof(float);
    size_t need = big0 + red_bytes;
    total = o > need ? o : need;
    (void)big1;
  }
};

// ===========================================================================
// Chunk coefficients for the slice: fills (in LDS)
//   gate[4][cs]       alpha, eta, theta, gamma' of the chunk
//   ctil[t'][i]       c[t,i] / m_t  (elem)          t = tok0 + t'
//   mrow[t']          m_t = max_i |c[t,i]|
//   thp[t']           Theta_t
//   Apre[t']          prod_{r<=t} alpha_r
//   ass[s'][t']       a(s->t) masked to s <= t     (slice-local s', t')
//   ait[i][t']        a(end_i -> t)  for slices i < j
// ===========================================================================
template <class M, int D, int E>
__device__ void chunk_coefficients(const ScanArgs& p, const PhaseLayout<M, D, E>& L, char* smem,
                                   int b, int hh, int j) {
  using elem = typename M::elem;
  float* gate = reinterpret_cast<float*>(smem + L.o_gate);
  float* ga = gate;
  float* ge = gate + CS_MAX;
  float* gt = gate + 2 * CS_MAX;
  float* gg = gate + 3 * CS_MAX;
  float* R = reinterpret_cast<float*>(smem + L.o_R);
  float* C = reinterpret_cast<float*>(smem + L.o_C);
  elem* ctil = reinterpret_cast<elem*>(smem + L.o_ctil);
  float* sm = reinterpret_cast<float*>(smem + L.o_small);
  float* mrow = sm;
  float* thp = sm + TS_MAX;
  float* Apre = sm + 2 * TS_MAX;
  float* ass = sm + 4 * TS_MAX;
  float* ait = ass + TS_MAX * TS_MAX;

  const int tid = threadIdx.x;
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, n = tok0 + ts;
  for (int t = tid; t < cs; t += NTHREADS) {
    const Gates G = load_gates(p, b, hh, p.chunk * cs + t);
    ga[t] = G.a; ge[t] = G.e; gt[t] = G.th; gg[t] = G.g;
  }
  __syncthreads();

  const float scale = 2.f / (float)D;
  // Row t' of suffix sums R[t'][s] = sum_{u=s}^{t} theta(u->t) (-eta_u), s <= t.
  if (tid < ts) {
    const int t = tok0 + tid;
    float prod = 1.f, run = 0.f;
    for (int s = t; s >= 0; --s) {
      run += prod * (-ge[s]);
      R[tid * (CS_MAX + 1) + s] = run;
      prod *= gt[s];
    }
    float th = 1.f, ap = 1.f;
    for (int r = 0; r <= t; ++r) { th *= gt[r]; ap *= ga[r]; }
    thp[tid] = th;
    Apre[tid] = ap;
  }
  for (int idx = tid; idx < ts * ts; idx += NTHREADS) {
    const int s = idx / ts, t = idx % ts;
    ass[idx] = (s <= t) ? seg_prod(ga, tok0 + s, tok0 + t) : 0.f;
  }
  for (int idx = tid; idx < j * ts; idx += NTHREADS) {
    const int i = idx / ts, t = idx % ts;
    ait[idx] = seg_prod(ga, (i + 1) * ts - 1, tok0 + t);
  }
  __syncthreads();
  // c[t,i] = scale * g_i * (R[i] - R[i+w])   (R[x] = 0 for x > t)
  const int w = p.w_eff;
  for (int idx = tid; idx < ts * n; idx += NTHREADS) {
    const int tp = idx / n, i = idx % n;
    const int t = tok0 + tp;
    float cv = 0.f;
    if (i <= t) {
      const float r0 = R[tp * (CS_MAX + 1) + i];
      const float r1 = (i + w <= t) ? R[tp * (CS_MAX + 1) + i + w] : 0.f;
      cv = scale * gg[i] * (r0 - r1);
    }
    C[tp * (CS_MAX + 1) + i] = cv;
  }
  __syncthreads();
  // row maxima and normalised rows
  if (tid < ts) {
    float m = 0.f;
    for (int i = 0; i < n; ++i) m = fmaxf(m, fabsf(C[tid * (CS_MAX + 1) + i]));
    mrow[tid] = (m > 0.f) ? m : 1.f;
  }
  __syncthreads();
  for (int idx = tid; idx < ts * L.csp; idx += NTHREADS) {
    const int tp = idx / L.csp, i = idx % L.csp;
    const float v = (i < n) ? C[tp * (CS_MAX + 1) + i] / mrow[tp] : 0.f;
    ctil[tp * L.csp + i] = M::to_elem(v);
  }
  __syncthreads();   // R and C alias the operand buffers staged next
}

// ===========================================================================
// phase<MAT>: per (stream, slice j), Polar-Express of S_MAT for the slice's
// tokens plus the slice-local parts of the memory scan and read-out.
//   MAT == 2 (W2, first MLP layer): L2_j and h partials (hloc).
//   MAT == 1 (W1, second layer):    h -> g for the slice, L1_j, y partials.
// ===========================================================================
template <class M, int D, int E, int MAT>
__global__ void __launch_bounds__(NTHREADS)
__attribute__((amdgpu_waves_per_eu(1, 1)))
phase_kernel(ScanArgs p) {
  constexpr int TI = D / 32, TJ = E / 32, KPT = M::KPT;
  using elem = typename M::elem;
  using frag = typename M::frag;
  using LY = PhaseLayout<M, D, E>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const LY L(p.cs);

  const int stream = blockIdx.x / p.nsl, j = blockIdx.x % p.nsl;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, wv = wave_id();
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, n = tok0 + ts;
  const long long sDE = (long long)stream * D * E;

  chunk_coefficients<M, D, E>(p, L, smem, b, hh, j);

  float* gate = reinterpret_cast<float*>(smem + L.o_gate);
  elem* ctil = reinterpret_cast<elem*>(smem + L.o_ctil);
  float* sm = reinterpret_cast<float*>(smem + L.o_small);
  float* mrow = sm;
  float* thp = sm + TS_MAX;
  float* Apre = sm + 2 * TS_MAX;
  float* ass = sm + 4 * TS_MAX;
  float* ait = ass + TS_MAX * TS_MAX;
  float* red4 = ait + NSL_MAX * TS_MAX;
  elem* Ut = reinterpret_cast<elem*>(smem + L.o_Ut);
  elem* Vt = reinterpret_cast<elem*>(smem + L.o_Vt);
  float* Sp = reinterpret_cast<float*>(smem + L.o_Sp);
  elem* Qs = reinterpret_cast<elem*>(smem + L.o_Qs);
  elem* Gs = reinterpret_cast<elem*>(smem + L.o_Gs);
  elem* scr = reinterpret_cast<elem*>(smem + L.o_scr) + wv * Scr<M>::template elems<D>();
  (void)gate;

  // ---- stage the momentum-assembly operands (power-of-two scaled) --------
  // MAT 2: U = K (tokens x D), V = Chain (tokens x E);  MAT 1: U = Err, V = Act.
  const float* Vsrc = (MAT == 2 ? p.chain : p.act) + (long long)stream * cs * E;
  const float* Usrc = p.err + (long long)stream * cs * D;   // MAT 1 only
  float mu = 0.f, mv = 0.f;
  for (int i = tid; i < n * D; i += NTHREADS) {
    const int t = i / D, d = i % D;
    const float x = (MAT == 2) ? load_x(p, p.k, b, p.chunk * cs + t, hh, d) : Usrc[(long long)t * D + d];
    mu = fmaxf(mu, fabsf(x));
  }
  for (int i = tid; i < n * E; i += NTHREADS) mv = fmaxf(mv, fabsf(Vsrc[i]));
  const float su = pow2_scale(block_max<NW>(mu, red4));
  const float sv = pow2_scale(block_max<NW>(mv, red4 + NW));
  for (int i = tid; i < D * L.csp; i += NTHREADS) {
    const int d = i / L.csp, t = i % L.csp;
    float x = 0.f;
    if (t < n) x = (MAT == 2) ? load_x(p, p.k, b, p.chunk * cs + t, hh, d) : Usrc[(long long)t * D + d];
    Ut[d * L.csp + t] = M::to_elem(x * su);
  }
  for (int i = tid; i < E * L.csp; i += NTHREADS) {
    const int e = i / L.csp, t = i % L.csp;
    const float x = (t < n) ? Vsrc[(long long)t * E + e] : 0.f;
    Vt[e * L.csp + t] = M::to_elem(x * sv);
  }
  // chunk-start momentum, stored [e][d]
  if (MAT == 2) {
    const float* S2c = p.S2[p.cur] + sDE;
    for (int i = tid; i < E * D; i += NTHREADS) Sp[(i / D) * LY::SPD + (i % D)] = S2c[i];
  } else {
    const float* S1c = p.S1[p.cur] + sDE;
    for (int i = tid; i < E * D; i += NTHREADS) {
      const int d = i / E, e = i % E;
      Sp[e * LY::SPD + d] = S1c[i];
    }
  }
  // slice queries, rows t' < 32 (zero beyond ts)
  for (int i = tid; i < 32 * D; i += NTHREADS) {
    const int t = i / D, d = i % D;
    const float x = (t < ts) ? load_x(p, p.q, b, p.chunk * cs + tok0 + t, hh, d) : 0.f;
    Qs[t * LY::QSP + d] = M::to_elem(x);
  }
  __syncthreads();

  // ---- read-out partial accumulators -----------------------------------
  constexpr int TR = (MAT == 2) ? TJ : TI;   // tiles of the slice read-out block
  f32x16 RO[TR];
#pragma unroll
  for (int q = 0; q < TR; ++q) RO[q] = zero16();

  // query fragments with the C-layout k assignment (B operand, lane = t');
  // reloaded from LDS where needed so they are not live across Polar-Express.
  auto load_qf = [&](int K, int kb) -> frag { return M::ld_cslot(Qs + c * LY::QSP + 32 * K, kb, h); };
  const float wA = (c < ts) ? Apre[c] : 0.f;

  if (MAT == 2) {
    // hloc init (wave 0): A_t * W2 q_t
    if (wv == 0) {
      const float* W2c = p.W2[p.cur] + sDE;
#pragma unroll
      for (int Ie = 0; Ie < TJ; ++Ie)
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            RO[Ie] = M::mma(M::gl_cslot(W2c + (32 * Ie + c) * D + 32 * K, kb, h),
                            M::scale(load_qf(K, kb), wA), RO[Ie]);
    }
  } else {
    // h for the slice: hloc_j + sum_{i<j} a(end_i->t) L2_i^T q_t, then g = gelu(h)
    const float* hl = p.hloc + (((long long)stream * p.nsl + j) * ts) * E;
#pragma unroll
    for (int q = 0; q < (TJ + NW - 1) / NW; ++q) {
      const int Ie = wv + q * NW;
      if (Ie >= TJ) break;
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[r] = (c < ts) ? hl[(long long)c * E + 32 * Ie + crow(r, h)] : 0.f;
      for (int i = 0; i < j; ++i) {
        const float* L2i = p.L2 + ((long long)stream * p.nsl + i) * D * E;
        const float wi = (c < ts) ? ait[i * ts + c] : 0.f;
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            acc = M::mma(M::gl_cslot(L2i + (32 * Ie + c) * D + 32 * K, kb, h),
                         M::scale(load_qf(K, kb), wi), acc);
      }
      float* gout = p.g + ((long long)stream * cs + tok0) * E;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int e = 32 * Ie + crow(r, h);
        const float gv = (c < ts) ? gelu_tanh(acc[r]) : 0.f;
        Gs[c * LY::GSP + e] = M::to_elem(gv);
        if (c < ts) gout[(long long)c * E + e] = gv;
      }
    }
    __syncthreads();
    // yloc init (wave 0): A_t * W1 g_t
    if (wv == 0) {
      const float* W1c = p.W1[p.cur] + sDE;
#pragma unroll
      for (int Id = 0; Id < TI; ++Id)
#pragma unroll
        for (int Je = 0; Je < TJ; ++Je)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            RO[Id] = M::mma(M::gl_contig(W1c + (32 * Id + c) * E + 32 * Je, kb, h),
                            M::scale(M::ld_contig(Gs + c * LY::GSP + 32 * Je, kb, h), wA), RO[Id]);
    }
  }

  // ---- per-token momentum assembly + Polar-Express ----------------------
  f32x16 Lacc[TI][TJ];
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J) Lacc[I][J] = zero16();

  const int tpw = ts / NW;
  const int nkb = (n + M::KB - 1) / M::KB;
  const float inv_uv = 1.f / (su * sv);
  for (int it = 0; it < tpw; ++it) {
    const int sl = wv * tpw + it;      // slice-local token
    const int t = tok0 + sl;           // chunk-local token
    f32x16 X[TI][TJ];
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J) X[I][J] = zero16();
    const elem* crowp = ctil + sl * L.csp;
    for (int kb = 0; kb < nkb; ++kb) {
      const frag cf = M::ld_contig(crowp, kb, h);
      frag uf[TI];
#pragma unroll
      for (int I = 0; I < TI; ++I) uf[I] = M::scale_v(M::ld_contig(Ut + (32 * I + c) * L.csp, kb, h), cf);
#pragma unroll
      for (int J = 0; J < TJ; ++J) {
        const frag vf = M::ld_contig(Vt + (32 * J + c) * L.csp, kb, h);
#pragma unroll
        for (int I = 0; I < TI; ++I) X[I][J] = M::mma(uf[I], vf, X[I][J]);
      }
    }
    const float f = mrow[sl] * inv_uv;
    const float th = thp[sl];
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 sp = *reinterpret_cast<const f32x4*>(Sp + (32 * J + c) * LY::SPD + 32 * I + 8 * q4 + 4 * h);
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
        float* S1n = p.S1[p.cur ^ 1] + sDE;
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int J = 0; J < TJ; ++J)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              S1n[(32 * I + crow(r, h)) * E + 32 * J + c] = X[I][J][r];
      }
    }

    polar_express_wave<M, D, E>(X, p.ns, 1e-12f, scr);

    // memory-scan partial L += a(s->end_j) P (an MFMA against a scaled identity,
    // so L stays in accumulator registers) and the slice read-out partial.
    const float aend = ass[sl * ts + ts - 1];
    const float wt = (c < ts) ? ass[sl * ts + c] : 0.f;   // a(s->t') masked to t' >= s
    typename M::afrag idf[KPT];
#pragma unroll
    for (int kb = 0; kb < KPT; ++kb) idf[kb] = M::a_identity(kb, c, h, aend);
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) Lacc[I][J] = M::amma(idf[kb], M::a_from_c(X[I][J], kb), Lacc[I][J]);
      if (MAT == 2) {
        // hloc[e][t'] += sum_d P2[e][d] q_t'[d] w(t')  (X tiles as A operand = P2 rows e)
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            RO[J] = M::mma(M::from_c(X[K][J], kb), M::scale(load_qf(K, kb), wt), RO[J]);
      }
    }
    if (MAT == 1) {
      // yloc[d][t'] += sum_e P1[d][e] g_t'[e] w(t')   (P1 rows via the scratch transpose)
      constexpr int SP = Scr<M>::SP;
#pragma unroll
      for (int Je = 0; Je < TJ; ++Je) {
        scr_put_cols<M, TI, TJ>(X, Je, scr);
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) {
          const frag gw = M::scale(M::ld_contig(Gs + c * LY::GSP + 32 * Je, kb, h), wt);
#pragma unroll
          for (int Id = 0; Id < TI; ++Id)
            RO[Id] = M::mma(M::ld_contig(scr + (32 * Id + c) * SP, kb, h), gw, RO[Id]);
        }
      }
    }
  }

  // ---- deterministic reduction over the NW waves: (w0 + w2) + (w1 + w3) -----
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem + L.o_Ut);
  constexpr int NT_L = TI * TJ, NT_R = TR;
  auto slot = [&](int buf, int tile, int r) -> float& {
    return red[((size_t)buf * D * E) + ((size_t)tile * 16 + r) * WAVE + lane];
  };
  // Lacc
  if (wv >= 2) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int r = 0; r < 16; ++r) slot(wv - 2, I * TJ + J, r) = Lacc[I][J][r];
  }
  __syncthreads();
  if (wv < 2) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int r = 0; r < 16; ++r) Lacc[I][J][r] += slot(wv, I * TJ + J, r);
  }
  __syncthreads();
  if (wv == 1) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int r = 0; r < 16; ++r) slot(0, I * TJ + J, r) = Lacc[I][J][r];
  }
  __syncthreads();
  if (wv == 0) {
    float* Lout = (MAT == 2 ? p.L2 : p.L1) + ((long long)stream * p.nsl + j) * D * E;
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float v = Lacc[I][J][r] + slot(0, I * TJ + J, r);
          const int d = 32 * I + crow(r, h), e = 32 * J + c;
          if (MAT == 2) Lout[e * D + d] = v; else Lout[d * E + e] = v;
        }
  }
  __syncthreads();
  // read-out partials
  if (wv >= 2) {
#pragma unroll
    for (int q = 0; q < NT_R; ++q)
#pragma unroll
      for (int r = 0; r < 16; ++r) slot(wv - 2, q, r) = RO[q][r];
  }
  __syncthreads();
  if (wv < 2) {
#pragma unroll
    for (int q = 0; q < NT_R; ++q)
#pragma unroll
      for (int r = 0; r < 16; ++r) RO[q][r] += slot(wv, q, r);
  }
  __syncthreads();
  if (wv == 1) {
#pragma unroll
    for (int q = 0; q < NT_R; ++q)
#pragma unroll
      for (int r = 0; r < 16; ++r) slot(0, q, r) = RO[q][r];
  }
  __syncthreads();
  if (wv == 0 && c < ts) {
    if (MAT == 2) {
      float* ho = p.hloc + (((long long)stream * p.nsl + j) * ts) * E;
#pragma unroll
      for (int q = 0; q < NT_R; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) ho[(long long)c * E + 32 * q + crow(r, h)] = RO[q][r] + slot(0, q, r);
    } else {
      float* yo = p.yloc + (((long long)stream * p.nsl + j) * ts) * D;
#pragma unroll
      for (int q = 0; q < NT_R; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) yo[(long long)c * D + 32 * q + crow(r, h)] = RO[q][r] + slot(0, q, r);
    }
  }
  (void)NT_L;
}

// ===========================================================================
// finalize: y for slice j, and slice j's share of W_end (elementwise).
// ===========================================================================
template <class M, int D, int E>
__global__ void __launch_bounds__(NTHREADS)
fin_kernel(ScanArgs p) {
  constexpr int TI = D / 32, TJ = E / 32, KPT = M::KPT;
  using frag = typename M::frag;
  __shared__ float ga[CS_MAX];
  __shared__ float aend[NSL_MAX];       // a(end_i -> cs-1)
  __shared__ float ait[NSL_MAX * TS_MAX];
  __shared__ float Aend;

  const int stream = blockIdx.x / p.nsl, j = blockIdx.x % p.nsl;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, wv = wave_id();
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, nsl = p.nsl;
  const long long sDE = (long long)stream * D * E;

  for (int t = tid; t < cs; t += NTHREADS) ga[t] = load_gates(p, b, hh, p.chunk * cs + t).a;
  __syncthreads();
  if (tid < nsl) aend[tid] = seg_prod(ga, (tid + 1) * ts - 1, cs - 1);
  if (tid == NTHREADS - 1) Aend = seg_prod(ga, -1, cs - 1);
  for (int idx = tid; idx < j * ts; idx += NTHREADS) {
    const int i = idx / ts, t = idx % ts;
    ait[idx] = seg_prod(ga, (i + 1) * ts - 1, tok0 + t);
  }
  __syncthreads();

  // W_end = A_end W + sum_i a(end_i->end) L_i, elements [j*DE/nsl, (j+1)*DE/nsl)
  {
    const int DE = D * E;
    const int per = (DE + nsl - 1) / nsl;
    const int lo = j * per, hi = min(DE, lo + per);
    const float* W1c = p.W1[p.cur] + sDE;
    const float* W2c = p.W2[p.cur] + sDE;
    float* W1n = p.W1[p.cur ^ 1] + sDE;
    float* W2n = p.W2[p.cur ^ 1] + sDE;
    const float* L1s = p.L1 + (long long)stream * nsl * DE;
    const float* L2s = p.L2 + (long long)stream * nsl * DE;
    for (int i = lo + tid; i < hi; i += NTHREADS) {
      float a1 = Aend * W1c[i], a2 = Aend * W2c[i];
      for (int s = 0; s < nsl; ++s) {
        a1 += aend[s] * L1s[(long long)s * DE + i];
        a2 += aend[s] * L2s[(long long)s * DE + i];
      }
      W1n[i] = a1;
      W2n[i] = a2;
    }
  }

  // y_t = q_t + yloc_j[t] + sum_{i<j} a(end_i->t) L1_i g_t   (wave Id owns D-tile Id)
  for (int Id = wv; Id < TI; Id += NW) {
    f32x16 acc = zero16();
    const float* gsl = p.g + ((long long)stream * cs + tok0) * E;
    for (int i = 0; i < j; ++i) {
      const float* L1i = p.L1 + ((long long)stream * nsl + i) * D * E;
      const float wi = (c < ts) ? ait[i * ts + c] : 0.f;
      const float* grow = gsl + (long long)((c < ts) ? c : 0) * E;
#pragma unroll
      for (int Je = 0; Je < TJ; ++Je)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb)
          acc = M::mma(M::gl_contig(L1i + (32 * Id + c) * E + 32 * Je, kb, h),
                       M::scale(M::gl_contig(grow + 32 * Je, kb, h), wi), acc);
    }
    if (c < ts) {
      const int tl = tok0 + c;
      const int tg = p.chunk * cs + tl;
      if (tg < p.T) {
        const float* yl = p.yloc + (((long long)stream * nsl + j) * ts + c) * D;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = 32 * Id + crow(r, h);
          const float yv = load_x(p, p.q, b, tg, hh, d) + yl[d] + acc[r];
          store_any(p.y, (long long)b * p.xsb + (long long)tg * p.xst + (long long)hh * p.xsh + d, p.io_dtype, yv);
        }
      }
    }
  }
}

}  // namespace atlas
