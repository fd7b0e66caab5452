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
// Launches: one coefficient pre-pass over all chunks (gate-only tables), then
// per chunk: prep, phase<2> (W2 = first MLP layer: PE of S2 and h), phase<1>
// (W1: PE of S1 and y), finalize (y, W_end).  State is ping-ponged between the
// caller's buffers and the workspace (index cur / cur^1).
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
  float* trace;   // host side only: chunk-start states (W1, W2, S1, S2 per chunk), or null
  float *kT, *errT, *actT, *chainT;   // prep outputs [stream][D|D|E|E][cs] (token-contiguous rows)
  float *L1, *L2;               // [stream][nsl][D*E]  (L1 as [D][E], L2 as [E][D])
  float* S1T[2];                // wide kernels: chunk-start S1 transposed, [stream][E][D]
  float *hloc, *yloc, *g;       // [stream][nsl][ts][E], [stream][nsl][ts][D], [stream][cs][E]
  // gate-only chunk tables, [stream][chunk % cw][...], written by the coef
  // kernel for a window of cw chunks at a time:
  float *cmt;                   // [cs][cs]  c[t,i] / m_t
  float *cm;                    // [cs]      m_t = max_i |c[t,i]| (1 if 0)
  float *thp;                   // [cs]      Theta_t = prod_{r<=t} theta_r
  float *ap;                    // [cs]      A_t = prod_{r<=t} alpha_r
  float *am;                    // [cs][cs]  am[t][s] = a(s->t) = prod_{s<r<=t} alpha_r (0 for s > t)
  int use_prefix;               // cross-slice sums through the slice-prefix kernel (else summed directly)
  int cw;                       // chunks whose gate tables are held at once (the table window)
  int chunk, cur;
};

// Workgroups are dispatched to the 8 XCDs round-robin by blockIdx.x, and each
// XCD has its own L2.  The logical block index returned here numbers the
// blocks of one XCD consecutively, so that neighbouring logical blocks (the
// slices of one stream, which read the same chunk operands and state) share
// an L2.  A bijection on [0, gridDim.x) for any grid size.
__device__ __forceinline__ int xcd_block() {
  constexpr int kXCD = 8;
  const int b = blockIdx.x, n = gridDim.x;
  const int x = b % kXCD, q = n / kXCD, r = n % kXCD;
  return x * q + (x < r ? x : r) + b / kXCD;
}

// Index of (stream, chunk)'s gate tables: the tables of a window of cw
// consecutive chunks are held at once (slot chunk % cw).
__device__ __forceinline__ long long chunk_table(const ScanArgs& p, int stream, int chunk) {
  return (long long)stream * p.cw + chunk % p.cw;
}

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
// Token-row loads for 8 consecutive elements (bf16 / fp32 / fp16 inputs):
// the load half keeps every load of a thread in flight before any use.
// ===========================================================================
template <int D, int ROWS>
struct TokenRows {
  static constexpr int G = 8;                        // elements per vector load
  static constexpr int NG = ROWS * D / G;
  static constexpr int PER = (NG + NTHREADS - 1) / NTHREADS;
  // Raw bits of G elements: 16 bytes for 2-byte dtypes, 32 for fp32.  The
  // loads are unconditional and dtype-independent (no branch joins that would
  // make them complete early); out-of-range groups load token 0 and are
  // written as zeros by store().
  uint4 raw[PER][2];
  bool okm[PER];

  __device__ __forceinline__ void load(const ScanArgs& p, const void* x, int b, int hh, int tok0, int nrows) {
    const int esz = (p.io_dtype == 0) ? 4 : 2;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int gi = threadIdx.x + u * NTHREADS;
      const int t = gi / (D / G), d0 = (gi % (D / G)) * G;
      const int tg = p.chunk * p.cs + tok0 + t;
      const bool ok = gi < NG && t < nrows && tg < p.T;
      const long long o = (long long)b * p.xsb + (long long)(ok ? tg : 0) * p.xst + (long long)hh * p.xsh + (ok ? d0 : 0);
      const char* a = static_cast<const char*>(x) + o * esz;
      raw[u][0] = *reinterpret_cast<const uint4*>(a);
      raw[u][1] = *reinterpret_cast<const uint4*>(a + (esz == 4 ? 16 : 0));
      okm[u] = ok;
    }
  }
  // element k of group u as float
  __device__ __forceinline__ float elem(int u, int k, int dtype) const {
    const uint4 w = raw[u][(dtype == 0 && k >= 4) ? 1 : 0];
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    if (dtype == 0) return __uint_as_float(ws[k & 3]);
    const uint32_t h16 = (k & 1) ? (ws[k >> 1] >> 16) : (ws[k >> 1] & 0xffffu);
    if (dtype == 1) return __uint_as_float(h16 << 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
  }
  // rows t, elements d -> dst[t * ldd + d] (converted to T)
  template <class T>
  __device__ __forceinline__ void store(T* dst, int ldd, int dtype) const {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int gi = threadIdx.x + u * NTHREADS;
      if (gi < NG) {
        const int t = gi / (D / G), d0 = (gi % (D / G)) * G;
#pragma unroll
        for (int k = 0; k < G; ++k) dst[t * ldd + d0 + k] = okm[u] ? (T)elem(u, k, dtype) : (T)0.f;
      }
    }
  }
};

// ===========================================================================
// prep: inner-gradient factors at the chunk-start weights, 32 tokens per WG.
// Grid: (streams * ceil(cs/32)).  fp32 MFMA (range and precision of the
// gradient factors matter: Polar-Express normalises whatever scale they have).
// ===========================================================================
// The weight operands of the three products go from global memory straight
// into MFMA operand registers.  An MFMA's contraction slots may take the
// contracted index in any order as long as both operands agree, so the lane
// half h takes a contiguous half of it: a lane then reads its weight row as
// 16-byte vectors and its token row from LDS as 16-byte vectors.  Only the
// token rows (K, V, Err, Act) and the Err partial sums live in LDS.
template <int D, int E>
constexpr size_t prep_token_floats() {
  constexpr int TI = D / 32, NP = (NW / TI) > 0 ? NW / TI : 1;
  return 3 * 32 * (D + 4) + 32 * (E + 4) + TI * (NP - 1) * 16 * WAVE;
}

// Block lb of the prep grid (streams * ceil(cs/32) blocks).
template <int D, int E>
__device__ __forceinline__ void prep_body(const ScanArgs& p, int lb) {
  constexpr int TI = D / 32, TJ = E / 32;
  constexpr int KS = D + 4, ES = E + 4;              // LDS row strides (floats, 16-byte rows)
  constexpr int QT = (TJ + NW - 1) / NW;             // E-tiles per wave
  constexpr int NP = (NW / TI) > 0 ? NW / TI : 1;    // parts of the Err contraction
  constexpr int EP = E / NP;                         // contraction length per part
  constexpr int DH = D / 2, EH = EP / 2;             // contraction elements per lane half
  static_assert(DH % 4 == 0 && EH % 4 == 0, "prep: 16-byte operand rows");
  extern __shared__ float lds[];
  float* Ks = lds;                   // [32][D+4]
  float* Vs = Ks + 32 * KS;          // [32][D+4]
  float* Rs = Vs + 32 * KS;          // [32][D+4]  Err
  float* As = Rs + 32 * KS;          // [32][E+4]  Act
  float* Ps = As + 32 * ES;          // Err partial sums [TI*(NP-1)][16][64]

  const int nblk = (p.cs + 31) / 32;
  const int stream = lb / nblk, blk = lb % nblk;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, w = wave_id();
  const int t0 = blk * 32;
  const long long sDE = (long long)stream * D * E;
  const int Id = w % TI, part = w / TI;

  // ---- all global loads in flight (token rows first: they are used first) --
  const int nt = min(32, p.cs - t0);
  TokenRows<D, 32> kr, vr;
  kr.load(p, p.k, b, hh, t0, nt);
  vr.load(p, p.v, b, hh, t0, nt);
  // keeps every token-row load ahead of the weight loads, so that storing
  // the rows waits for them alone
  asm volatile("" ::: "memory");
  const float* W1 = p.W1[p.cur] + sDE;   // [D][E]
  const float* W2 = p.W2[p.cur] + sDE;   // [E][D]
  f32x4 w2a[QT][DH / 4];   // H:     W2[32 Ie + c][h DH + k]
  float w1c[QT][DH];       // Chain: W1[h DH + k][32 Ie + c]
  f32x4 w1a[EH / 4];       // Err:   W1[32 Id + c][part EP + h EH + k]
#pragma unroll
  for (int q = 0; q < QT; ++q) {
    const int Ie = (w + q * NW < TJ) ? w + q * NW : 0;   // idle tiles read tile 0
#pragma unroll
    for (int j = 0; j < DH / 4; ++j)
      w2a[q][j] = *reinterpret_cast<const f32x4*>(W2 + (32 * Ie + c) * D + h * DH + 4 * j);
  }
  {
    const int pc = part < NP ? part : 0;
#pragma unroll
    for (int j = 0; j < EH / 4; ++j)
      w1a[j] = *reinterpret_cast<const f32x4*>(W1 + (32 * Id + c) * E + pc * EP + h * EH + 4 * j);
  }
#pragma unroll
  for (int q = 0; q < QT; ++q) {
    const int Ie = (w + q * NW < TJ) ? w + q * NW : 0;
#pragma unroll
    for (int k = 0; k < DH; ++k) w1c[q][k] = W1[(h * DH + k) * E + 32 * Ie + c];
  }
  kr.store(Ks, KS, p.io_dtype);
  vr.store(Vs, KS, p.io_dtype);
  __syncthreads();

  // H^T tiles [e][t] = W2 K^T: wave w owns E-tiles w, w+NW, ...; keeps gelu'
  // in registers.
  f32x16 gp[QT];
#pragma unroll
  for (int q = 0; q < QT; ++q) {
    const int Ie = w + q * NW;
    if (Ie >= TJ) break;
    f32x16 acc = zero16();
#pragma unroll
    for (int j = 0; j < DH / 4; ++j) {
      const f32x4 kv = *reinterpret_cast<const f32x4*>(Ks + c * KS + h * DH + 4 * j);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = ModeF32::mma(w2a[q][j][u], kv[u], acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int e = 32 * Ie + crow(r, h);
      const float x = acc[r];
      As[c * ES + e] = gelu_tanh(x);
      gp[q][r] = gelu_erf_prime(x);
    }
  }
  __syncthreads();

  // Err^T tiles [d][t] = W1 Act^T + K^T - V^T.  Each D-tile's contraction over
  // E is split into NP = NW / TI parts, one per wave; the parts are summed in
  // a fixed order (part 0 first) through LDS.
  {
    f32x16 acc = zero16();
    if (part < NP) {
#pragma unroll
      for (int j = 0; j < EH / 4; ++j) {
        const f32x4 av = *reinterpret_cast<const f32x4*>(As + c * ES + part * EP + h * EH + 4 * j);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = ModeF32::mma(w1a[j][u], av[u], acc);
      }
    }
    if (part >= 1 && part < NP) {
      float* slot = Ps + ((size_t)(Id * (NP - 1) + part - 1) * 16) * WAVE;
#pragma unroll
      for (int r = 0; r < 16; ++r) slot[r * WAVE + lane] = acc[r];
    }
    __syncthreads();
    if (part == 0) {
#pragma unroll
      for (int pp = 1; pp < NP; ++pp) {
        const float* slot = Ps + ((size_t)(Id * (NP - 1) + pp - 1) * 16) * WAVE;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] += slot[r * WAVE + lane];
      }

#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = 32 * Id + crow(r, h);
        Rs[c * KS + d] = acc[r] + Ks[c * KS + d] - Vs[c * KS + d];
      }
    }
  }
  __syncthreads();

  // K, Err and Act as token-contiguous rows [d][t] / [e][t], four tokens per
  // 16-byte store (cs is a multiple of 4), issued before the Chain products
  // so that they drain while those run
  {
    float* k_out = p.kT + (long long)stream * D * p.cs;
    float* err_out = p.errT + (long long)stream * D * p.cs;
    float* act_out = p.actT + (long long)stream * E * p.cs;
    const int nt = min(32, p.cs - t0);
    for (int i = tid; i < D * 8; i += NTHREADS) {
      const int d = i / 8, t = 4 * (i % 8);
      if (t < nt) {
        f32x4 rv, kv;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          rv[u] = Rs[(t + u) * KS + d];
          kv[u] = Ks[(t + u) * KS + d];
        }
        *reinterpret_cast<f32x4*>(err_out + (long long)d * p.cs + t0 + t) = rv;
        *reinterpret_cast<f32x4*>(k_out + (long long)d * p.cs + t0 + t) = kv;
      }
    }
    for (int i = tid; i < E * 8; i += NTHREADS) {
      const int e = i / 8, t = 4 * (i % 8);
      if (t < nt) {
        f32x4 av;
#pragma unroll
        for (int u = 0; u < 4; ++u) av[u] = As[(t + u) * ES + e];
        *reinterpret_cast<f32x4*>(act_out + (long long)e * p.cs + t0 + t) = av;
      }
    }
  }

  // Chain^T tiles [e][t] = (W1^T Err^T) * gelu'  -> chainT rows (token-contiguous)
  float* chain_out = p.chainT + (long long)stream * E * p.cs;
#pragma unroll
  for (int q = 0; q < QT; ++q) {
    const int Ie = w + q * NW;
    if (Ie >= TJ) break;
    f32x16 acc = zero16();
#pragma unroll
    for (int j = 0; j < DH / 4; ++j) {
      const f32x4 rv = *reinterpret_cast<const f32x4*>(Rs + c * KS + h * DH + 4 * j);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = ModeF32::mma(w1c[q][4 * j + u], rv[u], acc);
    }
    const int tl = t0 + c;
    if (tl < p.cs) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int e = 32 * Ie + crow(r, h);
        chain_out[(long long)e * p.cs + tl] = acc[r] * gp[q][r];
      }
    }
  }
}

template <int D, int E>
__global__ void __launch_bounds__(NTHREADS)
prep_kernel(ScanArgs p) {
  prep_body<D, E>(p, xcd_block());
}

// ===========================================================================
// coef: gate-only tables of the chunks [c0, c0 + nwin) (independent of the
// memory state, so a whole window of chunks is computed in parallel, ahead of
// the chunk loop reaching it).  Grid: streams * nwin.
// Row t of the chunk is owned by thread t (cs <= CS_MAX; the block holds cs
// rounded up to whole waves).  The two cs x (cs+1) tables are sized by the
// runtime cs (coef_lds_bytes(cs)), so at cs = 64 four blocks share a CU.
//   c[t,i] = (2/D) g'_i sum_{s=i}^{min(t,i+w-1)} theta(s->t) (-eta_s),
//   evaluated as g'_i (R_t[i] - R_t[i+w]) with suffix sums
//   R_t[s] = sum_{u=s}^{t} theta(u->t) (-eta_u).
// ===========================================================================
__global__ void __launch_bounds__(CS_MAX)
coef_kernel(ScanArgs p, int c0, int nwin) {
  extern __shared__ float cl[];
  const int cs = p.cs, CP = cs + 1;
  float* ga = cl;
  float* ge = ga + CS_MAX;
  float* gt = ge + CS_MAX;
  float* gg = gt + CS_MAX;
  float* mr = gg + CS_MAX;
  float* R = mr + CS_MAX;        // [cs][CP]
  float* C = R + cs * CP;        // [cs][CP]
  const int stream = blockIdx.x / nwin, chunk = c0 + blockIdx.x % nwin;
  const int b = stream / p.H, hh = stream % p.H;
  const int t = threadIdx.x;
  if (t < cs) {
    const Gates G = load_gates(p, b, hh, chunk * cs + t);
    ga[t] = G.a; ge[t] = G.e; gt[t] = G.th; gg[t] = G.g;
  }
  __syncthreads();
  const long long tb = chunk_table(p, stream, chunk);
  if (t < cs) {
    float th = 1.f, apv = 1.f;
    for (int r = 0; r <= t; ++r) { th *= gt[r]; apv *= ga[r]; }
    p.thp[tb * cs + t] = th;
    p.ap[tb * cs + t] = apv;
    // Window sums sum_{s=i}^{min(t, i+w-1)} m_t[s], m_t[s] = theta(s->t)
    // (-eta_s) (0 past t), without subtraction: over blocks of w tokens, the
    // in-block suffix sums (into Rt) and prefix sums (into Ct); a window is
    // the suffix of its first block plus, when it is not block-aligned, the
    // prefix of the next block.  (The difference of two suffix sums
    // R_t[i] - R_t[i+w] cancels for windows far behind t, where the decayed
    // window is much smaller than the sums.)  All terms share the sign of
    // -eta.  One backward pass forms m_t (kept in Ct) and the suffix sums,
    // one forward pass turns Ct into the prefix sums in place.
    const int w = p.w_eff;
    float* __restrict__ Rt = R + t * CP;
    float* __restrict__ Ct = C + t * CP;
    for (int s = cs - 1; s > t; --s) {
      Rt[s] = 0.f;
      Ct[s] = 0.f;
    }
    {
      float prod = 1.f, suf = 0.f;
#pragma unroll 8
      for (int s = t, r = t % w; s >= 0; --s) {
        const float mv = prod * (-ge[s]);
        prod *= gt[s];
        suf = (r == w - 1 || s == t) ? mv : suf + mv;
        Rt[s] = suf;
        Ct[s] = mv;
        r = (r == 0) ? w - 1 : r - 1;
      }
      float pre = 0.f;
#pragma unroll 8
      for (int s = 0, r = 0; s < cs; ++s) {   // (past t the block's prefix stays its sum up to t)
        pre = (r == 0) ? Ct[s] : pre + Ct[s];
        Ct[s] = pre;
        if (++r == w) r = 0;
      }
    }
    const float scale = 2.f / (float)p.D;
    float m = 0.f;
#pragma unroll 8
    for (int i = 0; i < cs; ++i) {
      float cv = 0.f;
      if (i <= t) {
        const int jw = min(i + w - 1, cs - 1);
        float win = Rt[i];
        if (jw / w != i / w) win += Ct[jw];
        cv = scale * gg[i] * win;
      }
      Ct[i] = cv;   // the prefix sum at i was last read for window i - w + 1 <= i
      m = fmaxf(m, fabsf(cv));
    }
    mr[t] = (m > 0.f) ? m : 1.f;
    p.cm[tb * cs + t] = mr[t];
  }
  __syncthreads();
  // a(s->t) row t into R (R is no longer needed)
  if (t < cs) {
    float prod = 1.f;
    for (int s = cs - 1; s > t; --s) R[t * CP + s] = 0.f;
    R[t * CP + t] = 1.f;
    for (int s = t - 1; s >= 0; --s) {
      prod *= ga[s + 1];
      R[t * CP + s] = prod;
    }
  }
  __syncthreads();
  float* cmt = p.cmt + tb * cs * cs;
  float* am = p.am + tb * cs * cs;
  for (int idx = t; idx < cs * cs; idx += blockDim.x) {
    const int r = idx / cs, i = idx % cs;
    cmt[idx] = C[r * CP + i] / mr[r];
    am[idx] = R[r * CP + i];
  }
}

constexpr size_t coef_lds_bytes(int cs = CS_MAX) { return sizeof(float) * (size_t)(5 * CS_MAX + 2 * cs * (cs + 1)); }
inline dim3 coef_block(int cs) { return dim3(((cs + 63) / 64) * 64); }

template <int D, int E>
constexpr size_t prep_lds_bytes() {
  return sizeof(float) * prep_token_floats<D, E>();
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
  size_t o_ctil, o_small, o_Ut, o_Vt, o_Sp, o_Qs, o_Gs, o_scr, o_L, total, total_lsh;

  __host__ __device__ PhaseLayout(int cs) {
    const int npad = ((cs + 15) / 16) * 16;
    csp = npad + PADE;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t r = o; o += (bytes + 15) & ~size_t(15); return r; };
    o_ctil = take((size_t)TS_MAX * csp * EB);
    o_small = take((size_t)(TS_MAX * 4 + TS_MAX * TS_MAX + NSL_MAX * TS_MAX + 16) * sizeof(float));
    const size_t big0 = o;
    o_Ut = take((size_t)D * csp * EB);
    o_Vt = take((size_t)E * csp * EB);
    o_Sp = take((size_t)E * SPD * sizeof(float));
    o_Qs = take((size_t)32 * QSP * EB);
    o_Gs = take((size_t)32 * GSP * EB);
    // per-wave Gram scratch: only the fp32 path transposes through LDS
    o_scr = take(EB == 2 ? 0 : (size_t)NW * Scr<M>::template elems<D>() * EB);
    // the epilogue reuses [big0, end): two D*E fp32 reduction slots and one
    // D*E staging buffer in the global layout (register-accumulation path), or
    // the NW waves' read-out partial tiles side by side (LDS-accumulation path)
    const size_t tree = 3 * (size_t)D * E * sizeof(float);
    const size_t ro_slots = (size_t)NW * (D > E ? D : E) / 32 * 16 * WAVE * sizeof(float);
    total = o > big0 + tree ? o : big0 + tree;
    const size_t lsh_base = o > big0 + ro_slots ? o : big0 + ro_slots;
    o_L = (lsh_base + 15) & ~size_t(15);
    total_lsh = o_L + (size_t)D * E * sizeof(float);
  }
};

// ===========================================================================
// Vectorised staging helpers: every thread issues all of its loads before it
// uses any of them (one workgroup per CU leaves no other wave to hide latency).
// ===========================================================================

// rows x n fp32 values (n % 4 == 0, n <= CS_MAX, row stride ld floats,
// 16-byte aligned rows) into registers, float4 granularity.  Quad i of the
// thread block is row i / (CS_MAX/4), column quad i % (CS_MAX/4) (no runtime
// division), so MAXF4 must cover rows * CS_MAX / 4 / NTHREADS.
constexpr int QPR = CS_MAX / 4;   // quads per row slot
template <int MAXF4>
__device__ __forceinline__ void load_rows4(f32x4 (&v)[MAXF4], const float* src, int rows, int n, int ld) {
  const int n4 = n >> 2;
#pragma unroll
  for (int u = 0; u < MAXF4; ++u) {
    const int i = threadIdx.x + u * NTHREADS;
    const int r = i / QPR, c4 = i % QPR;
    // Branch-free: out-of-range quads load quad (0, 0) and hold garbage that
    // maxabs4 and store_rows4 skip.  (A bounds branch or a select right after
    // the load makes each load complete before the next one is issued.)
    const bool ok = r < rows && c4 < n4;
    const int rr = ok ? r : 0, cc = ok ? c4 : 0;
    v[u] = *reinterpret_cast<const f32x4*>(src + (long long)rr * ld + 4 * cc);
  }
}

// max |v| over the in-range quads of a load_rows4 block
template <int MAXF4>
__device__ __forceinline__ float maxabs4(const f32x4 (&v)[MAXF4], int rows, int n) {
  const int n4 = n >> 2;
  float m = 0.f;
#pragma unroll
  for (int u = 0; u < MAXF4; ++u) {
    const int i = threadIdx.x + u * NTHREADS;
    const int r = i / QPR, c4 = i % QPR;
    float mu = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) mu = fmaxf(mu, fabsf(v[u][k]));
    m = (r < rows && c4 < n4) ? fmaxf(m, mu) : m;
  }
  return m;
}

// Store the register block (as loaded by load_rows4) scaled into an LDS
// operand array dst[r * ldd + t] of element type elem.
template <class M, int MAXF4>
__device__ __forceinline__ void store_rows4(const f32x4 (&v)[MAXF4], typename M::elem* dst, int rows, int n,
                                            int ldd, float scale) {
  const int n4 = n >> 2;
#pragma unroll
  for (int u = 0; u < MAXF4; ++u) {
    const int i = threadIdx.x + u * NTHREADS;
    const int r = i / QPR, c4 = i % QPR;
    if (r < rows && c4 < n4) {
      typename M::elem* d = dst + r * ldd + 4 * c4;
#pragma unroll
      for (int k = 0; k < 4; ++k) d[k] = M::to_elem(v[u][k] * scale);
    }
  }
}


// ===========================================================================
// phase<MAT>: per (stream, slice j), Polar-Express of S_MAT for the slice's
// tokens plus the slice-local parts of the memory scan and read-out.
//   MAT == 2 (W2, first MLP layer): L2_j and h partials (hloc).
//   MAT == 1 (W1, second layer):    h -> g for the slice, L1_j, y partials.
// LSH: L_j accumulates in an fp32 LDS array (else in accumulator registers
// through an identity MFMA); the LDS form needs D*E*4 more bytes of LDS.
// ===========================================================================
template <class M, int D, int E, int MAT, bool LSH>
__global__ void __launch_bounds__(NTHREADS)
__attribute__((amdgpu_waves_per_eu(1, 1)))
phase_kernel(ScanArgs p) {
  constexpr int TI = D / 32, TJ = E / 32, KPT = M::KPT;
  constexpr int NT = TI * TJ;
  using elem = typename M::elem;
  using frag = typename M::frag;
  using LY = PhaseLayout<M, D, E>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const LY L(p.cs);

  const int lb = xcd_block();
  const int stream = lb / p.nsl, j = lb % p.nsl;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, wv = wave_id();
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, n = tok0 + ts;
  const long long sDE = (long long)stream * D * E;

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
  // LSH only: element r = 4q + u of tile tl for this lane at
  // [((tl*4 + q)*64 + lane)*4 + u], so each lane moves 16-byte quads and a
  // wave's quad accesses are contiguous
  float* Lsh = reinterpret_cast<float*>(smem + L.o_L);

  // ---- staging: every global load is issued before any of them is used ----
  // (one workgroup per CU leaves no other wave to hide the latency)
  const long long tb = chunk_table(p, stream, p.chunk);
  {
    constexpr int CF4 = TS_MAX * CS_MAX / 4 / NTHREADS;
    constexpr int UF4 = D * CS_MAX / 4 / NTHREADS, VF4 = E * CS_MAX / 4 / NTHREADS;
    constexpr int SF4 = D * E / 4 / NTHREADS;
    const float* Usrc = (MAT == 2 ? p.kT : p.errT) + (long long)stream * D * cs;
    const float* Vsrc = (MAT == 2 ? p.chainT : p.actT) + (long long)stream * E * cs;
    const float* Sc = (MAT == 2 ? p.S2[p.cur] : p.S1[p.cur]) + sDE;
    f32x4 cv[CF4], uv[UF4], vv[VF4], sv4[SF4];
    TokenRows<D, 32> qr;
    // gate-only coefficient slices (from the pre-pass)
    load_rows4<CF4>(cv, p.cmt + tb * cs * cs + (long long)tok0 * cs, ts, n, cs);
    // momentum-assembly operands: MAT 2: U = K^T (D x tokens), V = Chain^T
    // (E x tokens); MAT 1: Err^T, Act^T
    load_rows4<UF4>(uv, Usrc, D, n, cs);
    load_rows4<VF4>(vv, Vsrc, E, n, cs);
    // chunk-start momentum
#pragma unroll
    for (int u = 0; u < SF4; ++u) sv4[u] = reinterpret_cast<const f32x4*>(Sc)[tid + u * NTHREADS];
    // slice queries, rows t' < 32 (zero beyond ts)
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
    // operands power-of-two scaled into fp16 range
    const float su = pow2_scale(block_max<NW>(maxabs4<UF4>(uv, D, n), red4));
    const float sv = pow2_scale(block_max<NW>(maxabs4<VF4>(vv, E, n), red4 + NW));
    store_rows4<M, UF4>(uv, Ut, D, n, L.csp, su);
    store_rows4<M, VF4>(vv, Vt, E, n, L.csp, sv);
    // zero the K-block tail [n, 16*ceil(n/16)) of every operand row
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
    // chunk-start momentum, stored [e][d]
#pragma unroll
    for (int u = 0; u < SF4; ++u) {
      const int i = 4 * (tid + u * NTHREADS);
      if (MAT == 2) {   // S2 is [e][d]
        *reinterpret_cast<f32x4*>(Sp + (i / D) * LY::SPD + (i % D)) = sv4[u];
      } else {          // S1 is [d][e]
        const int d = i / E, e0 = i % E;
#pragma unroll
        for (int k = 0; k < 4; ++k) Sp[(e0 + k) * LY::SPD + d] = sv4[u][k];
      }
    }
    qr.template store<elem>(Qs, LY::QSP, p.io_dtype);
  }
  if (LSH) {
    for (int i = tid; i < D * E / 4; i += NTHREADS) reinterpret_cast<f32x4*>(Lsh)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();
  const float inv_uv = red4[2 * NW];

  // ---- read-out partial accumulators -----------------------------------
  constexpr int TR = (MAT == 2) ? TJ : TI;   // tiles of the slice read-out block
  f32x16 RO[TR];
#pragma unroll
  for (int q = 0; q < TR; ++q) RO[q] = zero16();

  // query fragments with the C-layout k assignment (B operand, lane = t');
  // reloaded from LDS where needed so they are not live across Polar-Express.
  auto load_qf = [&](int K, int kb) -> frag { return M::ld_cslot(Qs + c * LY::QSP + 32 * K, kb, h); };
  const float wA = (c < ts) ? Apre[c] : 0.f;

  // The slice read-out partials are summed over the waves in the epilogue,
  // so the initial terms below are split across waves (wave w takes tile
  // w, w+NW, ...), with their global operands loaded before first use.
  if (MAT == 2) {
    // hloc init: A_t * W2 q_t, wave w -> E-tiles Ie = w (mod NW)
    const float* W2c = p.W2[p.cur] + sDE;
    // (compile-time tile index: a wave-dependent index into RO would move the
    // accumulators to scratch memory)
#pragma unroll
    for (int Ie = 0; Ie < TJ; ++Ie) {
      if ((Ie % NW) != wv) continue;
      frag wf[TI][KPT];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) wf[K][kb] = M::gl_cslot(W2c + (32 * Ie + c) * D + 32 * K, kb, h);
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < KPT; ++kb) RO[Ie] = M::mma(wf[K][kb], M::scale(load_qf(K, kb), wA), RO[Ie]);
    }
  } else {
    // yloc init operands (W1 rows for this wave's E-tile), loaded up front
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
      // hloc rows: four 4-row groups per lane (t' = c, e = 32 Ie + crow(r, h))
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x4 v = (c < ts) ? *reinterpret_cast<const f32x4*>(hl + (long long)c * E + 32 * Ie + 8 * g4 + 4 * h)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[4 * g4 + u] = v[u];
      }
      // earlier slices: sum_{i<j} a(e_i -> t) L2_i^T q_t, directly (up to 4
      // slices' fragments in flight) or as a(e_{j-1} -> t) M2_j^T q_t with the
      // slice prefix M2_j (slot j of L2 after the prefix kernel)
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
          RO[Id] = M::mma(w1f[q][Id][kb], M::scale(M::ld_contig(Gs + c * LY::GSP + 32 * Je, kb, h), wA), RO[Id]);
    }
  }

  // ---- per-token momentum assembly + Polar-Express ----------------------
  f32x16 Lacc[LSH ? 1 : TI][LSH ? 1 : TJ];
  if (!LSH) {
#pragma unroll
    for (int I = 0; I < (LSH ? 1 : TI); ++I)
#pragma unroll
      for (int J = 0; J < (LSH ? 1 : TJ); ++J) Lacc[I][J] = zero16();
  }

  const int tpw = ts / NW;
  const int nkb = (n + M::KB - 1) / M::KB;
  frag idf[KPT];   // identity B operand for the fp16 read-out transpose
#pragma unroll
  for (int kb = 0; kb < KPT; ++kb) idf[kb] = M::identity(kb, c, h);
  for (int it = 0; it < tpw; ++it) {
    const int sl = wv * tpw + it;      // slice-local token
    const int t = tok0 + sl;           // chunk-local token
    f32x16 X[TI][TJ];
    // Y = sum_i c~[t,i] u_i (x) v_i on the matrix cores (the first K-block
    // starts from a zero accumulator, so X needs no initialisation)
    const elem* crowp = ctil + sl * L.csp;
    auto s_block = [&](int kb, bool first) {
      const frag cf = M::ld_contig(crowp, kb, h);
      frag uf[TI];
#pragma unroll
      for (int I = 0; I < TI; ++I) uf[I] = M::scale_v(M::ld_contig(Ut + (32 * I + c) * L.csp, kb, h), cf);
#pragma unroll
      for (int J = 0; J < TJ; ++J) {
        const frag vf = M::ld_contig(Vt + (32 * J + c) * L.csp, kb, h);
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
        // S1 is [d][e]: the lane's offset formed here (opaque) so that 64
        // per-element addresses are not hoisted out of the token loop
        float* S1n = p.S1[p.cur ^ 1] + sDE + PEWaveT<D, E>::opaque(crow(0, h) * E + c);
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int J = 0; J < TJ; ++J)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              S1n[(32 * I + 8 * (r >> 2) + (r & 3)) * E + 32 * J] = X[I][J][r];
      }
    }

    polar_express_wave<M, D, E>(X, p.ns, 1e-12f, scr);

    // memory-scan partial L += a(s->end_j) P and the slice read-out partial.
    const float aend = ass[sl * ts + ts - 1];
    const float wt = (c < ts) ? ass[sl * ts + c] : 0.f;   // a(s->t') masked to t' >= s
    if (LSH) {
      // rotated schedule: in sub-step k wave w adds into tile group (w + k) % NW;
      // each group therefore receives the waves in a fixed order.
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const int grp = (wv + k) & (NW - 1);
#pragma unroll
        for (int tl = 0; tl < NT; ++tl) {
          if ((tl & (NW - 1)) != grp) continue;
          f32x4* dst = reinterpret_cast<f32x4*>(Lsh) + (size_t)tl * 4 * WAVE + lane;
          f32x4 cur[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) cur[q] = dst[q * WAVE];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int u = 0; u < 4; ++u) cur[q][u] += aend * X[tl / TJ][tl % TJ][4 * q + u];
            dst[q * WAVE] = cur[q];
          }
        }
        __syncthreads();
      }
    } else {
      typename M::afrag aid[KPT];
#pragma unroll
      for (int kb = 0; kb < KPT; ++kb) aid[kb] = M::a_identity(kb, c, h, aend);
#pragma unroll
      for (int I = 0; I < (LSH ? 1 : TI); ++I)
#pragma unroll
        for (int J = 0; J < (LSH ? 1 : TJ); ++J)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            Lacc[I][J] = M::amma(aid[kb], M::a_from_c(X[I][J], kb), Lacc[I][J]);
    }
    if (MAT == 2) {
      // hloc[e][t'] += sum_d P2[e][d] q_t'[d] w(t')  (X tiles as A operand = P2 rows e)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb)
            RO[J] = M::mma(M::from_c(X[K][J], kb), M::scale(load_qf(K, kb), wt), RO[J]);
    } else {
      // yloc[d][t'] += sum_e P1[d][e] g_t'[e] w(t')
      if constexpr (LY::EB == 2) {
        // P1 rows via the identity-product transpose: (P1 tile)^T * I in C
        // layout has e along its rows, so as the A operand it supplies P1
        // with the k assignment of a C-layout tile (kslot).
#pragma unroll
        for (int Je = 0; Je < TJ; ++Je) {
          frag gw[KPT];
#pragma unroll
          for (int kb = 0; kb < KPT; ++kb) gw[kb] = M::scale(M::ld_cslot(Gs + c * LY::GSP + 32 * Je, kb, h), wt);
#pragma unroll
          for (int Id = 0; Id < TI; ++Id) {
            f32x16 tt = zero16();
#pragma unroll
            for (int kb = 0; kb < KPT; ++kb) tt = M::mma(M::from_c(X[Id][Je], kb), idf[kb], tt);
#pragma unroll
            for (int kb = 0; kb < KPT; ++kb) RO[Id] = M::mma(M::from_c(tt, kb), gw[kb], RO[Id]);
          }
        }
      } else {
        // P1 rows via the scratch transpose
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
  }

  // ---- epilogue ----------------------------------------------------------
  __syncthreads();
  constexpr int RW = (MAT == 2) ? E : D;   // row length of hloc / yloc
  float* ro_out = (MAT == 2 ? p.hloc : p.yloc) + (((long long)stream * p.nsl + j) * ts) * RW;
  float* Lout = (MAT == 2 ? p.L2 : p.L1) + ((long long)stream * p.nsl + j) * D * E;
  if constexpr (LSH) {
    // read-out partials of the NW waves side by side: [w][q][r][lane]
    float* ros = reinterpret_cast<float*>(smem + L.o_Ut);
#pragma unroll
    for (int q = 0; q < TR; ++q)
#pragma unroll
      for (int r = 0; r < 16; ++r) ros[((wv * TR + q) * 16 + r) * WAVE + lane] = RO[q][r];
    __syncthreads();
    // slice memory partial: Lsh quad (tile, q, lane) holds rows d0..d0+3 of
    // column e; thread i takes e = i % E (consecutive lanes, consecutive LDS
    // quads) and d0 = 4 (i / E)
    for (int i = tid; i < D * E / 4; i += NTHREADS) {
      const int e = i % E, d0 = 4 * (i / E);
      const int tl = (d0 >> 5) * TJ + (e >> 5), qd = (d0 & 31) >> 3, hd = (d0 & 7) >> 2;
      const f32x4 v = reinterpret_cast<const f32x4*>(Lsh)[(tl * 4 + qd) * WAVE + (e & 31) + 32 * hd];
      if (MAT == 2) {   // L2 is [e][d]
        *reinterpret_cast<f32x4*>(Lout + (long long)e * D + d0) = v;
      } else {          // L1 is [d][e]
#pragma unroll
        for (int u = 0; u < 4; ++u) Lout[(long long)(d0 + u) * E + e] = v[u];
      }
    }
    // read-out partial rows t' < ts: element (t', x) sits at register r of lane
    // t' + 32 h with x % 32 = 8 (r / 4) + 4 h + r % 4; the waves are summed in order
    for (int i = tid; i < ts * RW; i += NTHREADS) {
      const int tp = i / RW, x = i % RW;
      const int q = x >> 5, xl = x & 31, hx = (xl >> 2) & 1, r = 4 * (xl >> 3) + (xl & 3);
      const int ln = tp + 32 * hx;
      float acc = ros[((0 * TR + q) * 16 + r) * WAVE + ln];
#pragma unroll
      for (int w = 1; w < NW; ++w) acc += ros[((w * TR + q) * 16 + r) * WAVE + ln];
      ro_out[i] = acc;
    }
  } else {
    float* red = reinterpret_cast<float*>(smem + L.o_Ut);    // two reduction slots
    float* outb = red + 2 * (size_t)D * E;                   // staging in global layout
    auto slot = [&](int buf, int tile, int r) -> float& {
      return red[((size_t)buf * D * E) + ((size_t)tile * 16 + r) * WAVE + lane];
    };
    auto put_L = [&](int tl, int r, float v) {
      const int d = 32 * (tl / TJ) + crow(r, h), e = 32 * (tl % TJ) + c;
      outb[(MAT == 2) ? (e * D + d) : (d * E + e)] = v;
    };
    // deterministic tree over the NW waves: (w0 + w2) + (w1 + w3)
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
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J)
#pragma unroll
          for (int r = 0; r < 16; ++r) put_L(I * TJ + J, r, Lacc[I][J][r] + slot(0, I * TJ + J, r));
    }
    __syncthreads();
    for (int i = tid; i < D * E / 4; i += NTHREADS)
      reinterpret_cast<f32x4*>(Lout)[i] = reinterpret_cast<const f32x4*>(outb)[i];
    __syncthreads();
    // read-out partials: deterministic tree, then coalesced store
    if (wv >= 2) {
#pragma unroll
      for (int q = 0; q < TR; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) slot(wv - 2, q, r) = RO[q][r];
    }
    __syncthreads();
    if (wv < 2) {
#pragma unroll
      for (int q = 0; q < TR; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) RO[q][r] += slot(wv, q, r);
    }
    __syncthreads();
    if (wv == 1) {
#pragma unroll
      for (int q = 0; q < TR; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) slot(0, q, r) = RO[q][r];
    }
    __syncthreads();
    if (wv == 0 && c < ts) {
#pragma unroll
      for (int q = 0; q < TR; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) outb[c * RW + 32 * q + crow(r, h)] = RO[q][r] + slot(0, q, r);
    }
    __syncthreads();
    for (int i = tid; i < ts * RW / 4; i += NTHREADS)
      reinterpret_cast<f32x4*>(ro_out)[i] = reinterpret_cast<const f32x4*>(outb)[i];
  }
}

// ===========================================================================
// prefix: slice prefixes of the memory scan for one matrix (after its phase
// kernel).  With e_j the last token of slice j and a(s->t) the alpha product,
//   M_j = sum_{i<j} a(e_i -> e_{j-1}) L_i  (j >= 1), so that
//   sum_{i<j} a(e_i -> t) L_i = a(e_{j-1} -> t) M_j  for t in slice j,
//   W_end = A_end W + sum_i a(e_i -> e_last) L_i = A_end W + M_nsl.
// M_j overwrites slot j of L (slot 0 is not used).  Elementwise over the
// D*E entries (16-byte groups), sequential over j.  Grid: streams * nparts.
// ===========================================================================
template <int D, int E>
constexpr int kPrefixParts = (D * E / 4 + NTHREADS - 1) / NTHREADS;

template <int D, int E>
__global__ void __launch_bounds__(NTHREADS)
prefix_kernel(ScanArgs p, int mat) {
  constexpr int N4 = D * E / 4;
  constexpr int PARTS = kPrefixParts<D, E>;
  const int stream = blockIdx.x / PARTS, part = blockIdx.x % PARTS;
  const int cs = p.cs, ts = p.ts, nsl = p.nsl;
  const long long sDE = (long long)stream * D * E;
  const int i = part * NTHREADS + threadIdx.x;
  if (i >= N4) return;   // no barrier below
  const long long tb = chunk_table(p, stream, p.chunk);
  const float* am = p.am + tb * cs * cs;
  f32x4* Ls = reinterpret_cast<f32x4*>((mat == 2 ? p.L2 : p.L1) + sDE * nsl);
  const f32x4* Wc = reinterpret_cast<const f32x4*>((mat == 2 ? p.W2[p.cur] : p.W1[p.cur]) + sDE);
  f32x4* Wn = reinterpret_cast<f32x4*>((mat == 2 ? p.W2[p.cur ^ 1] : p.W1[p.cur ^ 1]) + sDE);
  const float Aend = p.ap[tb * cs + cs - 1];
  const f32x4 w = Wc[i];
  f32x4 acc = Ls[i];
  // slices in groups of 8, a group's loads and its step factors
  // a(e_{j-1} -> e_j) (every thread reads them from the cached gate table:
  // no shared table, no barrier) in flight together
  for (int j0 = 1; j0 < nsl; j0 += 8) {
    f32x4 l[8];
    float stp[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (j0 + u < nsl) {
        l[u] = Ls[(long long)(j0 + u) * N4 + i];
        stp[u] = am[((j0 + u + 1) * ts - 1) * cs + (j0 + u) * ts - 1];
      }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (j0 + u < nsl) {
        Ls[(long long)(j0 + u) * N4 + i] = acc;
        acc = stp[u] * acc + l[u];
      }
    }
  }
  Wn[i] = Aend * w + acc;
}

// ===========================================================================
// finalize: y for slice j; without the prefix kernel also slice j's share of
// W_end (elementwise).
// ===========================================================================
// Block lb of the finalize grid (streams * n_slices blocks).  PARTS: 1 = the
// slice's share of W_end (without the prefix kernel), 2 = y for the slice.
template <class M, int D, int E, int PARTS>
__device__ __forceinline__ void fin_body(const ScanArgs& p, int lb) {
  constexpr int TI = D / 32, TJ = E / 32, KPT = M::KPT;
  constexpr int NP = NW / TI;                 // waves per D-tile (E split for the read-out)
  constexpr int JP = (TJ + NP - 1) / NP;      // E-tiles per wave
  using frag = typename M::frag;
  __shared__ float aend[NSL_MAX];             // a(e_i -> cs-1)
  __shared__ float ait[NSL_MAX * TS_MAX];     // a(e_i -> t), i < j
  __shared__ float Aend;
  __shared__ float part_acc[TI * (NP - 1) * 16 * WAVE];

  const int stream = lb / p.nsl, j = lb % p.nsl;
  const int b = stream / p.H, hh = stream % p.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, wv = wave_id();
  const int cs = p.cs, ts = p.ts, tok0 = j * ts, nsl = p.nsl;
  const long long sDE = (long long)stream * D * E;
  {
    const long long tb = chunk_table(p, stream, p.chunk);
    const float* am = p.am + tb * cs * cs;
    if (tid < nsl) aend[tid] = am[(cs - 1) * cs + (tid + 1) * ts - 1];
    if (tid == NTHREADS - 1) Aend = p.ap[tb * cs + cs - 1];
    for (int idx = tid; idx < j * ts; idx += NTHREADS) {
      const int i = idx / ts, t = idx % ts;
      ait[idx] = am[(tok0 + t) * cs + (i + 1) * ts - 1];
    }
  }
  __syncthreads();

  if ((PARTS & 1) && !p.use_prefix) {
    // W_end = A_end W + sum_i a(e_i -> end) L_i over this slice's share of
    // the elements (16-byte groups; the sum runs over i in order)
    constexpr int N4 = D * E / 4;
    const int per = (N4 + nsl - 1) / nsl;
    const int lo = j * per, hi = min(N4, lo + per);
    const f32x4* W1c = reinterpret_cast<const f32x4*>(p.W1[p.cur] + sDE);
    const f32x4* W2c = reinterpret_cast<const f32x4*>(p.W2[p.cur] + sDE);
    f32x4* W1n = reinterpret_cast<f32x4*>(p.W1[p.cur ^ 1] + sDE);
    f32x4* W2n = reinterpret_cast<f32x4*>(p.W2[p.cur ^ 1] + sDE);
    const f32x4* L1s = reinterpret_cast<const f32x4*>(p.L1 + (long long)stream * nsl * D * E);
    const f32x4* L2s = reinterpret_cast<const f32x4*>(p.L2 + (long long)stream * nsl * D * E);
    for (int i = lo + tid; i < hi; i += NTHREADS) {
      f32x4 a1 = Aend * W1c[i], a2 = Aend * W2c[i];
#pragma unroll 4
      for (int s = 0; s < nsl; ++s) {
        a1 += aend[s] * L1s[(long long)s * N4 + i];
        a2 += aend[s] * L2s[(long long)s * N4 + i];
      }
      W1n[i] = a1;
      W2n[i] = a2;
    }
  }

  if constexpr ((PARTS & 2) == 0) return;
  // y_t = q_t + yloc_j[t] + sum_{i<j} a(e_i -> t) L1_i g_t (directly, or as
  // a(e_{j-1} -> t) M1_j g_t with the slice prefix).  D-tile Id = wv % TI;
  // the E contraction is split over the NP waves of a tile and their partial
  // tiles are summed in wave order through LDS.
  const int Id = wv % TI, part = wv / TI;
  f32x16 acc = zero16();
  if (j > 0) {
    const float* grow = p.g + ((long long)stream * cs + tok0 + ((c < ts) ? c : 0)) * E;
    frag gf[JP][KPT];
#pragma unroll
    for (int jj = 0; jj < JP; ++jj)
#pragma unroll
      for (int kb = 0; kb < KPT; ++kb) {
        const int Je = part * JP + jj;
        gf[jj][kb] = M::gl_contig(grow + 32 * (Je < TJ ? Je : 0), kb, h);
      }
    const int i_lo = p.use_prefix ? j : 0, i_hi = p.use_prefix ? j + 1 : j;
    for (int i = i_lo; i < i_hi; ++i) {
      const float* L1i = p.L1 + ((long long)stream * nsl + i) * D * E + (long long)(32 * Id + c) * E;
      const float wi = (c < ts) ? ait[(p.use_prefix ? j - 1 : i) * ts + c] : 0.f;
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
  if (part == 0) {
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

template <class M, int D, int E>
__global__ void __launch_bounds__(NTHREADS)
fin_kernel(ScanArgs p) {
  fin_body<M, D, E, 3>(p, xcd_block());
}

// W_end only (the y part runs in tail_kernel, next to the next chunk's prep).
template <class M, int D, int E>
__global__ void __launch_bounds__(NTHREADS)
fin_wend_kernel(ScanArgs p) {
  fin_body<M, D, E, 1>(p, xcd_block());
}

// One launch for two independent jobs: the prep of chunk p.chunk (blocks
// [0, n_prep)) and the y part of the finalize of chunk p.chunk - 1 (the
// remaining blocks, each taking `per` consecutive slices of one stream;
// n_prep = 0 after the last chunk).  The prep only needs W_end, written by
// fin_wend_kernel before this launch, and neither job reads what the other
// writes.  Each role numbers its blocks per XCD as xcd_block does (exact when
// the role boundary is a multiple of 8; otherwise only the L2 locality
// differs).
template <class M, int D, int E>
__global__ void __launch_bounds__(NTHREADS)
tail_kernel(ScanArgs p, int n_prep, int per) {
  constexpr int kXCD = 8;
  const int bx = blockIdx.x;
  auto xcd_index = [](int b, int n) {
    const int x = b % kXCD, q = n / kXCD, r = n % kXCD;
    return x * q + (x < r ? x : r) + b / kXCD;
  };
  if (bx < n_prep) {
    prep_body<D, E>(p, xcd_index(bx, n_prep));
  } else {
    ScanArgs pf = p;
    pf.chunk = p.chunk - 1;
    pf.cur = p.cur ^ 1;
    const int groups = (p.nsl + per - 1) / per;
    const int lb = xcd_index(bx - n_prep, (int)gridDim.x - n_prep);
    const int stream = lb / groups, g = lb % groups;
    for (int k = 0; k < per; ++k) {
      const int j = g * per + k;
      if (j >= p.nsl) break;
      if (k > 0) __syncthreads();   // the slice tables in LDS are reused
      fin_body<M, D, E, 2>(pf, stream * p.nsl + j);
    }
  }
}

}  // namespace atlas
