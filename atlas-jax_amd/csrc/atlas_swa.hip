// Sliding-window causal attention with rotary embeddings: the attention of
// the MAG blocks (atlas_jax/model.py:83-133, SlidingWindowAttention.__call__
// between the qkv projection and to_out; used by MAGBlock,
// atlas_jax/mag_transformer.py:63-79).
//
// Per (b, h) and query t, with q', k' the half-split rotary rotation of q, k
// (model.py:64-73) and the mask of model.py:123-127 (causal, t - s <= window):
//   out_t = sum_s softmax_s(q'_t . k'_s / sqrt(D)) v_s.
//
// One workgroup per (b, h, block of 128 queries); wave w owns 32 queries.
// Keys and values of the window are streamed through LDS in blocks of 64.
// The score tile is formed transposed, S^T = K Q^T (keys along the C-layout
// rows, queries along the lanes), so that after the online softmax the
// probabilities are already the B operand of O^T = V^T P^T (the contraction
// index -- the key -- runs along the rows).  fp16 matrix-core operands, fp32
// accumulation, scores, softmax statistics and output scaling.
#include <hip/hip_runtime.h>

#include <math.h>

#include "atlas_common.hpp"
#include "atlas_scan.h"
#include "atlas_status.hpp"

namespace atlas {
namespace {

constexpr int SWA_D = 64;           // head dim
constexpr int SWA_BQ = 128;         // queries per workgroup (4 waves x 32)
constexpr int SWA_BK = 64;          // keys per LDS block
constexpr int SWA_KSP = SWA_D + 8;  // fp16 row stride of K rows [key][d]
constexpr int SWA_VSP = SWA_BK + 8; // fp16 row stride of V^T rows [d][key]

struct SwaArgs {
  int B, T, H, window, io_dtype;
  long long sb, st, sh;             // q/k/v element strides
  const void *q, *k, *v;
  void* out;                        // (B, T, H, D) contiguous
  const float *cos_tab, *sin_tab;   // (T, D/2)
  float scale;
  float* lse;                       // (B, H, T) softmax log-normalisers of the scaled scores, or NULL
};

__device__ __forceinline__ void load8(const void* x, long long o, int dtype, float (&r)[8]) {
  if (dtype == 1) {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + o);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      r[2 * k] = __uint_as_float(ws[k] << 16);
      r[2 * k + 1] = __uint_as_float(ws[k] & 0xffff0000u);
    }
  } else {
    const f16x8 a = *reinterpret_cast<const f16x8*>(static_cast<const _Float16*>(x) + o);
#pragma unroll
    for (int k = 0; k < 8; ++k) r[k] = (float)a[k];
  }
}

__global__ void __launch_bounds__(256) swa_fwd_kernel(SwaArgs a) {
  using M = ModeF16;
  using frag = M::frag;
  __shared__ __attribute__((aligned(16))) _Float16 Ks[SWA_BK * SWA_KSP];
  __shared__ __attribute__((aligned(16))) _Float16 Vt[SWA_D * SWA_VSP];

  const int nqb = (a.T + SWA_BQ - 1) / SWA_BQ;
  const int bh = blockIdx.x / nqb, qb = blockIdx.x % nqb;
  const int b = bh / a.H, hh = bh % a.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, w = wave_id();
  const int q0 = qb * SWA_BQ, qw = q0 + 32 * w, tq = qw + c;
  const long long base_bh = (long long)b * a.sb + (long long)hh * a.sh;
  constexpr int HD = SWA_D / 2;

  // query fragments (B operand of S^T): lane (c, h) holds q'[tq][16 kb + 8 h + v]
  frag qf[4];
  {
    float x[4][8];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if (tq < a.T) {
        load8(a.q, base_bh + (long long)tq * a.st + 16 * kb + 8 * h, a.io_dtype, x[kb]);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) x[kb][u] = 0.f;
      }
    }
    // rotation pairs (d, d + D/2): K-blocks (kb, kb + 2)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int d = 16 * kb + 8 * h + u;
        const float cs = (tq < a.T) ? a.cos_tab[(long long)tq * HD + d] : 1.f;
        const float sn = (tq < a.T) ? a.sin_tab[(long long)tq * HD + d] : 0.f;
        const float x1 = x[kb][u], x2 = x[kb + 2][u];
        qf[kb][u] = (_Float16)(x1 * cs - x2 * sn);
        qf[kb + 2][u] = (_Float16)(x2 * cs + x1 * sn);
      }
  }

  float m = -INFINITY, l = 0.f;
  f32x16 O[2] = {zero16(), zero16()};
  const int kfirst = max(0, q0 - a.window) / SWA_BK * SWA_BK;
  const int kend = min(a.T, q0 + SWA_BQ);
  for (int kb0 = kfirst; kb0 < kend; kb0 += SWA_BK) {
    __syncthreads();
    {
      // K rows (rotated) and V^T: thread -> key kb0 + tid/4, d in [8p, 8p+8) and [8p+32, 8p+40)
      const int jj = tid >> 2, p = tid & 3, j = kb0 + jj, d0 = 8 * p;
      float k1[8], k2[8], v1[8], v2[8];
      if (j < a.T) {
        const long long o = base_bh + (long long)j * a.st;
        load8(a.k, o + d0, a.io_dtype, k1);
        load8(a.k, o + d0 + HD, a.io_dtype, k2);
        load8(a.v, o + d0, a.io_dtype, v1);
        load8(a.v, o + d0 + HD, a.io_dtype, v2);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) k1[u] = k2[u] = v1[u] = v2[u] = 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float cs = (j < a.T) ? a.cos_tab[(long long)j * HD + d0 + u] : 1.f;
        const float sn = (j < a.T) ? a.sin_tab[(long long)j * HD + d0 + u] : 0.f;
        Ks[jj * SWA_KSP + d0 + u] = (_Float16)(k1[u] * cs - k2[u] * sn);
        Ks[jj * SWA_KSP + d0 + HD + u] = (_Float16)(k2[u] * cs + k1[u] * sn);
        Vt[(d0 + u) * SWA_VSP + jj] = (_Float16)v1[u];
        Vt[(d0 + HD + u) * SWA_VSP + jj] = (_Float16)v2[u];
      }
    }
    __syncthreads();
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int k0 = kb0 + 32 * kt;
      // sub-tile entirely in the future or entirely out of the window of this wave's queries
      if (k0 >= a.T || k0 > qw + 31 || k0 + 31 < qw - a.window) continue;
      f32x16 S = zero16();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) S = M::mma(M::ld_contig(Ks + (32 * kt + c) * SWA_KSP, kb, h), qf[kb], S);
      // S[r]: key k0 + crow(r, h), query tq
      float mloc = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = k0 + crow(r, h);
        const bool ok = j < a.T && j <= tq && tq - j <= a.window;
        S[r] = ok ? S[r] * a.scale : -INFINITY;
        mloc = fmaxf(mloc, S[r]);
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, WAVE));
      // (no per-lane branch around the matrix-core products: a query with no
      // visible key yet keeps m = -inf, l = 0, O = 0 through msafe)
      const float mnew = fmaxf(m, mloc);
      const float msafe = (mnew == -INFINITY) ? 0.f : mnew;
      const float alpha = __expf(m - msafe);   // m = -inf -> 0
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        S[r] = __expf(S[r] - msafe);             // masked -> 0
        ps += S[r];
      }
      l = l * alpha + ps;
      m = mnew;
      O[0] *= alpha;
      O[1] *= alpha;
      frag pf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) pf[kb] = M::from_c(S, kb);
#pragma unroll
      for (int I = 0; I < 2; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          O[I] = M::mma(M::ld_cslot(Vt + (32 * I + c) * SWA_VSP + 32 * kt, kb, h), pf[kb], O[I]);
    }
  }
  // the two lane halves of a query hold the sums over complementary key rows
  const float lt = l + __shfl_xor(l, 32, WAVE);
  if (tq >= a.T) return;
  const float inv = 1.f / lt;
  if (a.lse && h == 0) a.lse[(long long)bh * a.T + tq] = m + __logf(lt);   // every query sees itself: lt > 0
  const long long oo = (((long long)b * a.T + tq) * a.H + hh) * SWA_D;
#pragma unroll
  for (int I = 0; I < 2; ++I)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * I + 8 * g + 4 * h;   // rows crow(4g + u, h) = d0 + u
      f32x4 v;
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = O[I][4 * g + u] * inv;
      store4_any(a.out, oo + d0, a.io_dtype, v);
    }
}

// ---- backward ---------------------------------------------------------------
// With P = softmax(S), S = q'k'^T / sqrt(D) over the window, O = P v and the
// cotangent dO of O (the standard attention backward, recomputing P from the
// forward's log-normalisers):
//   dv_s = sum_t P_ts dO_t,   dP_ts = dO_t . v_s,   Delta_t = dO_t . O_t,
//   dS_ts = P_ts (dP_ts - Delta_t),
//   dk'_s = scale sum_t dS_ts q'_t,   dq'_t = scale sum_s dS_ts k'_s,
// then dq, dk = the inverse rotation of dq', dk' (the rotation is
// orthogonal).  Two kernels, each owning its outputs (no atomics, so the
// backward is bitwise reproducible): swa_bwd_kv_kernel per block of 128 keys
// loops over the queries that see them, swa_bwd_q_kernel per block of 128
// queries over their window's keys.

struct SwaBwdArgs {
  SwaArgs f;                        // the forward's arguments (out = the forward's output O)
  const void* dout;                 // (B, T, H, D) contiguous, io dtype
  const float* lse;                 // (B, H, T)
  float* delta;                     // (B, H, T) workspace: Delta_t
  float *dq, *dk, *dv;              // (B, T, H, D) fp32 contiguous
};

// Delta_t = dO_t . O_t, one thread per (b, t, h)
__global__ void __launch_bounds__(256) swa_bwd_delta_kernel(SwaBwdArgs a) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;   // (b, t, h) row of the contiguous arrays
  const long long n = (long long)a.f.B * a.f.T * a.f.H;
  if (i >= n) return;
  const int hh = (int)(i % a.f.H);
  const long long bt = i / a.f.H;
  const int t = (int)(bt % a.f.T), b = (int)(bt / a.f.T);
  float acc = 0.f;
#pragma unroll
  for (int d0 = 0; d0 < SWA_D; d0 += 8) {
    float o[8], g[8];
    load8(a.f.out, i * SWA_D + d0, a.f.io_dtype, o);
    load8(a.dout, i * SWA_D + d0, a.f.io_dtype, g);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = fmaf(o[u], g[u], acc);
  }
  a.delta[((long long)b * a.f.H + hh) * a.f.T + t] = acc;
}

// 8 rotated (when rot) fp16 values of row j at d0 .. d0 + 7 and d0 + 32 ..
// d0 + 39 of x (strided q/k/v, or the contiguous dO when strided == false)
__device__ __forceinline__ void rot_pair(const SwaArgs& f, const void* x, long long o, int j, int d0, bool rot,
                                         float (&x1)[8], float (&x2)[8]) {
  constexpr int HD = SWA_D / 2;
  load8(x, o + d0, f.io_dtype, x1);
  load8(x, o + d0 + HD, f.io_dtype, x2);
  if (rot) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float cs = f.cos_tab[(long long)j * HD + d0 + u], sn = f.sin_tab[(long long)j * HD + d0 + u];
      const float a1 = x1[u], a2 = x2[u];
      x1[u] = a1 * cs - a2 * sn;
      x2[u] = a2 * cs + a1 * sn;
    }
  }
}

// dq, dk from the rotated gradients held as two C-layout tiles (rows d and
// d + 32, lane = token j) times scale, inverse-rotated and stored (fp32)
__device__ __forceinline__ void store_unrot(const SwaArgs& f, float* dst, long long row, int j, int h,
                                            const f32x16 (&G)[2], float scale, bool rot) {
  constexpr int HD = SWA_D / 2;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    f32x4 v1, v2;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = 8 * g + 4 * h + u;   // crow(4g + u, h)
      const float a1 = G[0][4 * g + u] * scale, a2 = G[1][4 * g + u] * scale;
      if (rot) {
        const float cs = f.cos_tab[(long long)j * HD + d], sn = f.sin_tab[(long long)j * HD + d];
        v1[u] = a1 * cs + a2 * sn;
        v2[u] = a2 * cs - a1 * sn;
      } else {
        v1[u] = a1;
        v2[u] = a2;
      }
    }
    *reinterpret_cast<f32x4*>(dst + row + 8 * g + 4 * h) = v1;
    *reinterpret_cast<f32x4*>(dst + row + HD + 8 * g + 4 * h) = v2;
  }
}

constexpr int SWB_BQ = 64;   // queries per LDS block of the key-side kernel

// dk, dv for 128 keys per workgroup (wave w: keys kw .. kw + 31), over the
// query blocks of 64 that see them.  Tiles: S and dP as [query][key] (rows =
// queries, lanes = keys) so that P and dS are directly the B operands of
// dV^T = dO^T P and dK^T = Q^T dS (contraction over queries).
__global__ void __launch_bounds__(256) swa_bwd_kv_kernel(SwaBwdArgs a) {
  using M = ModeF16;
  using frag = M::frag;
  const SwaArgs& f = a.f;
  __shared__ __attribute__((aligned(16))) _Float16 Qs[SWB_BQ * SWA_KSP];    // q' rows [t][d]
  __shared__ __attribute__((aligned(16))) _Float16 Qt[SWA_D * SWA_VSP];     // q'^T [d][t]
  __shared__ __attribute__((aligned(16))) _Float16 Gs[SWB_BQ * SWA_KSP];    // dO rows [t][d]
  __shared__ __attribute__((aligned(16))) _Float16 Gt[SWA_D * SWA_VSP];     // dO^T [d][t]
  __shared__ float Ls[SWB_BQ], Dl[SWB_BQ];
  const int nkb = (f.T + SWA_BQ - 1) / SWA_BQ;
  const int bh = blockIdx.x / nkb, kblk = blockIdx.x % nkb;
  const int b = bh / f.H, hh = bh % f.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, w = wave_id();
  const int K0 = kblk * SWA_BQ, kw = K0 + 32 * w, key = kw + c;
  const long long base_bh = (long long)b * f.sb + (long long)hh * f.sh;
  const long long lrow = (long long)bh * f.T;
  constexpr int HD = SWA_D / 2;

  // this lane's key: k' and v as B-operand fragments (k = d)
  frag kf[4], vf[4];
  {
    float k1[2][8], k2[2][8], v1[2][8], v2[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int d0 = 16 * kb + 8 * h;
      if (key < f.T) {
        const long long o = base_bh + (long long)key * f.st;
        rot_pair(f, f.k, o, key, d0, true, k1[kb], k2[kb]);
        rot_pair(f, f.v, o, key, d0, false, v1[kb], v2[kb]);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) k1[kb][u] = k2[kb][u] = v1[kb][u] = v2[kb][u] = 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        kf[kb][u] = (_Float16)k1[kb][u];
        kf[kb + 2][u] = (_Float16)k2[kb][u];
        vf[kb][u] = (_Float16)v1[kb][u];
        vf[kb + 2][u] = (_Float16)v2[kb][u];
      }
    }
  }
  f32x16 dK[2] = {zero16(), zero16()}, dV[2] = {zero16(), zero16()};   // [d][key] tiles
  const int qfirst = K0 / SWB_BQ * SWB_BQ;
  const int qend = min(f.T, K0 + SWA_BQ + f.window);
  for (int qb0 = qfirst; qb0 < qend; qb0 += SWB_BQ) {
    __syncthreads();
    {
      // thread -> query qb0 + tid/4, d in [8p, 8p+8) and [8p+32, 8p+40)
      const int jj = tid >> 2, p = tid & 3, t = qb0 + jj, d0 = 8 * p;
      float q1[8], q2[8], g1[8], g2[8];
      if (t < f.T) {
        rot_pair(f, f.q, base_bh + (long long)t * f.st, t, d0, true, q1, q2);
        rot_pair(f, a.dout, (((long long)b * f.T + t) * f.H + hh) * SWA_D, t, d0, false, g1, g2);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) q1[u] = q2[u] = g1[u] = g2[u] = 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        Qs[jj * SWA_KSP + d0 + u] = (_Float16)q1[u];
        Qs[jj * SWA_KSP + d0 + HD + u] = (_Float16)q2[u];
        Qt[(d0 + u) * SWA_VSP + jj] = (_Float16)q1[u];
        Qt[(d0 + HD + u) * SWA_VSP + jj] = (_Float16)q2[u];
        Gs[jj * SWA_KSP + d0 + u] = (_Float16)g1[u];
        Gs[jj * SWA_KSP + d0 + HD + u] = (_Float16)g2[u];
        Gt[(d0 + u) * SWA_VSP + jj] = (_Float16)g1[u];
        Gt[(d0 + HD + u) * SWA_VSP + jj] = (_Float16)g2[u];
      }
      if (tid < SWB_BQ) {
        const int tt = qb0 + tid;
        Ls[tid] = tt < f.T ? a.lse[lrow + tt] : 0.f;
        Dl[tid] = tt < f.T ? a.delta[lrow + tt] : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int t0 = qb0 + 32 * qt;
      // sub-tile with no query that sees any of this wave's keys
      if (t0 >= f.T || t0 + 31 < kw || t0 > kw + 31 + f.window) continue;
      f32x16 S = zero16(), dP = zero16();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        S = M::mma(M::ld_contig(Qs + (32 * qt + c) * SWA_KSP, kb, h), kf[kb], S);
        dP = M::mma(M::ld_contig(Gs + (32 * qt + c) * SWA_KSP, kb, h), vf[kb], dP);
      }
      // S[r]: query t0 + crow(r, h), key `key`
      f32x16 P, dS;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int tl = 32 * qt + crow(r, h), t = qb0 + tl;
        const bool ok = t < f.T && key < f.T && key <= t && t - key <= f.window;
        P[r] = ok ? __expf(S[r] * f.scale - Ls[tl]) : 0.f;
        dS[r] = P[r] * (dP[r] - Dl[tl]);
      }
      frag pf[2], sf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        pf[kb] = M::from_c(P, kb);
        sf[kb] = M::from_c(dS, kb);
      }
#pragma unroll
      for (int I = 0; I < 2; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          dV[I] = M::mma(M::ld_cslot(Gt + (32 * I + c) * SWA_VSP + 32 * qt, kb, h), pf[kb], dV[I]);
          dK[I] = M::mma(M::ld_cslot(Qt + (32 * I + c) * SWA_VSP + 32 * qt, kb, h), sf[kb], dK[I]);
        }
    }
  }
  if (key >= f.T) return;
  const long long row = (((long long)b * f.T + key) * f.H + hh) * SWA_D;
  store_unrot(f, a.dk, row, key, h, dK, f.scale, true);
  store_unrot(f, a.dv, row, key, h, dV, 1.f, false);
}

// dq for 128 queries per workgroup (wave w: queries qw .. qw + 31), over the
// key blocks of 64 of their window.  Tiles as in the forward: S^T and dP^T
// as [key][query] (rows = keys, lanes = queries), so that dS^T is directly
// the B operand of dQ^T = K^T dS^T (contraction over keys).
__global__ void __launch_bounds__(256) swa_bwd_q_kernel(SwaBwdArgs a) {
  using M = ModeF16;
  using frag = M::frag;
  const SwaArgs& f = a.f;
  __shared__ __attribute__((aligned(16))) _Float16 Ks[SWA_BK * SWA_KSP];    // k' rows [key][d]
  __shared__ __attribute__((aligned(16))) _Float16 Kt[SWA_D * SWA_VSP];     // k'^T [d][key]
  __shared__ __attribute__((aligned(16))) _Float16 Vs[SWA_BK * SWA_KSP];    // v rows [key][d]
  const int nqb = (f.T + SWA_BQ - 1) / SWA_BQ;
  const int bh = blockIdx.x / nqb, qblk = blockIdx.x % nqb;
  const int b = bh / f.H, hh = bh % f.H;
  const int tid = threadIdx.x, lane = lane_id(), c = lane & 31, h = lane >> 5, w = wave_id();
  const int q0 = qblk * SWA_BQ, qw = q0 + 32 * w, tq = qw + c;
  const long long base_bh = (long long)b * f.sb + (long long)hh * f.sh;
  constexpr int HD = SWA_D / 2;

  // this lane's query: q' and dO as B-operand fragments (k = d)
  frag qf[4], gf[4];
  {
    float q1[2][8], q2[2][8], g1[2][8], g2[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int d0 = 16 * kb + 8 * h;
      if (tq < f.T) {
        rot_pair(f, f.q, base_bh + (long long)tq * f.st, tq, d0, true, q1[kb], q2[kb]);
        rot_pair(f, a.dout, (((long long)b * f.T + tq) * f.H + hh) * SWA_D, tq, d0, false, g1[kb], g2[kb]);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) q1[kb][u] = q2[kb][u] = g1[kb][u] = g2[kb][u] = 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        qf[kb][u] = (_Float16)q1[kb][u];
        qf[kb + 2][u] = (_Float16)q2[kb][u];
        gf[kb][u] = (_Float16)g1[kb][u];
        gf[kb + 2][u] = (_Float16)g2[kb][u];
      }
    }
  }
  const float lq = tq < f.T ? a.lse[(long long)bh * f.T + tq] : 0.f;
  const float dq_ = tq < f.T ? a.delta[(long long)bh * f.T + tq] : 0.f;
  f32x16 dQ[2] = {zero16(), zero16()};   // [d][query] tiles
  const int kfirst = max(0, q0 - f.window) / SWA_BK * SWA_BK;
  const int kend = min(f.T, q0 + SWA_BQ);
  for (int kb0 = kfirst; kb0 < kend; kb0 += SWA_BK) {
    __syncthreads();
    {
      const int jj = tid >> 2, p = tid & 3, j = kb0 + jj, d0 = 8 * p;
      float k1[8], k2[8], v1[8], v2[8];
      if (j < f.T) {
        const long long o = base_bh + (long long)j * f.st;
        rot_pair(f, f.k, o, j, d0, true, k1, k2);
        rot_pair(f, f.v, o, j, d0, false, v1, v2);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) k1[u] = k2[u] = v1[u] = v2[u] = 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        Ks[jj * SWA_KSP + d0 + u] = (_Float16)k1[u];
        Ks[jj * SWA_KSP + d0 + HD + u] = (_Float16)k2[u];
        Kt[(d0 + u) * SWA_VSP + jj] = (_Float16)k1[u];
        Kt[(d0 + HD + u) * SWA_VSP + jj] = (_Float16)k2[u];
        Vs[jj * SWA_KSP + d0 + u] = (_Float16)v1[u];
        Vs[jj * SWA_KSP + d0 + HD + u] = (_Float16)v2[u];
      }
    }
    __syncthreads();
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int k0 = kb0 + 32 * kt;
      if (k0 >= f.T || k0 > qw + 31 || k0 + 31 < qw - f.window) continue;
      f32x16 S = zero16(), dP = zero16();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        S = M::mma(M::ld_contig(Ks + (32 * kt + c) * SWA_KSP, kb, h), qf[kb], S);
        dP = M::mma(M::ld_contig(Vs + (32 * kt + c) * SWA_KSP, kb, h), gf[kb], dP);
      }
      // S[r]: key k0 + crow(r, h), query tq
      f32x16 dS;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int j = k0 + crow(r, h);
        const bool ok = j < f.T && tq < f.T && j <= tq && tq - j <= f.window;
        const float pr = ok ? __expf(S[r] * f.scale - lq) : 0.f;
        dS[r] = pr * (dP[r] - dq_);
      }
      frag sf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) sf[kb] = M::from_c(dS, kb);
#pragma unroll
      for (int I = 0; I < 2; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          dQ[I] = M::mma(M::ld_cslot(Kt + (32 * I + c) * SWA_VSP + 32 * kt, kb, h), sf[kb], dQ[I]);
    }
  }
  if (tq >= f.T) return;
  store_unrot(f, a.dq, (((long long)b * f.T + tq) * f.H + hh) * SWA_D, tq, h, dQ, f.scale, true);
}


atlas_status swa_setup(SwaArgs& a, int32_t B, int32_t T, int32_t H, int32_t D, int32_t window, const void* q,
                       const void* k, const void* v, void* out, int64_t stride_b, int64_t stride_t,
                       int64_t stride_h, int32_t io_dtype, const float* cos_tab, const float* sin_tab) {
  if (B < 1 || T < 1 || H < 1 || window < 0)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad sizes B=%d T=%d H=%d window=%d", B, T, H, window);
  if (D != SWA_D) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "head dim %d not compiled (D = 64 only)", D);
  if (io_dtype != 1 && io_dtype != 2)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "io_dtype %d: bf16 (1) or fp16 (2) inputs only", io_dtype);
  if (!q || !k || !v || !out || !cos_tab || !sin_tab) return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL pointer");
  if ((stride_b | stride_t | stride_h) & 7 || stride_t < 1 || stride_h < 1)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "q/k/v strides must be positive multiples of 8 elements");
  const long long nqb = (T + SWA_BQ - 1) / SWA_BQ;
  if ((long long)B * H * nqb > (1LL << 31) - 1) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "grid too large");
  a.B = B; a.T = T; a.H = H; a.window = window; a.io_dtype = io_dtype;
  a.sb = stride_b; a.st = stride_t; a.sh = stride_h;
  a.q = q; a.k = k; a.v = v; a.out = out;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab;
  a.scale = 1.f / sqrtf((float)D);
  a.lse = nullptr;
  return ATLAS_OK;
}

atlas_status swa_launch_fwd(const SwaArgs& a, void* stream) {
  const long long nqb = (a.T + SWA_BQ - 1) / SWA_BQ;
  hipLaunchKernelGGL(swa_fwd_kernel, dim3((unsigned)(a.B * a.H * nqb)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "swa launch");
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" atlas_status atlas_swa_fwd(int32_t B, int32_t T, int32_t H, int32_t D, int32_t window,
                                      const void* q, const void* k, const void* v, void* out,
                                      int64_t stride_b, int64_t stride_t, int64_t stride_h, int32_t io_dtype,
                                      const float* cos_tab, const float* sin_tab, void* stream) {
  clear_error();
  SwaArgs a;
  const atlas_status r = swa_setup(a, B, T, H, D, window, q, k, v, out, stride_b, stride_t, stride_h, io_dtype,
                                   cos_tab, sin_tab);
  return r ? r : swa_launch_fwd(a, stream);
}

extern "C" atlas_status atlas_swa_fwd_lse(int32_t B, int32_t T, int32_t H, int32_t D, int32_t window,
                                          const void* q, const void* k, const void* v, void* out,
                                          int64_t stride_b, int64_t stride_t, int64_t stride_h, int32_t io_dtype,
                                          const float* cos_tab, const float* sin_tab, float* lse, void* stream) {
  clear_error();
  SwaArgs a;
  const atlas_status r = swa_setup(a, B, T, H, D, window, q, k, v, out, stride_b, stride_t, stride_h, io_dtype,
                                   cos_tab, sin_tab);
  if (r) return r;
  if (!lse) return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL lse");
  a.lse = lse;
  return swa_launch_fwd(a, stream);
}

extern "C" size_t atlas_swa_bwd_workspace_size(int32_t B, int32_t T, int32_t H) {
  if (B < 1 || T < 1 || H < 1) return 0;
  return (size_t)B * T * H * sizeof(float);
}

extern "C" atlas_status atlas_swa_bwd(int32_t B, int32_t T, int32_t H, int32_t D, int32_t window,
                                      const void* q, const void* k, const void* v, const void* out,
                                      const void* dout, const float* lse, int64_t stride_b, int64_t stride_t,
                                      int64_t stride_h, int32_t io_dtype, const float* cos_tab,
                                      const float* sin_tab, float* dq, float* dk, float* dv, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  clear_error();
  SwaBwdArgs a;
  atlas_status r = swa_setup(a.f, B, T, H, D, window, q, k, v, const_cast<void*>(out), stride_b, stride_t,
                             stride_h, io_dtype, cos_tab, sin_tab);
  if (r) return r;
  if (!dout || !lse || !dq || !dk || !dv) return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL pointer");
  const size_t need = atlas_swa_bwd_workspace_size(B, T, H);
  if (!workspace || workspace_bytes < need)
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, need);
  auto mis = [](const void* p, int al) { return reinterpret_cast<uintptr_t>(p) % al != 0; };
  if (mis(out, 16) || mis(dout, 16) || mis(dq, 16) || mis(dk, 16) || mis(dv, 16) || mis(workspace, 4) ||
      mis(lse, 4))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "out, dout, dq, dk, dv must be 16-byte aligned");
  a.dout = dout;
  a.lse = lse;
  a.delta = static_cast<float*>(workspace);
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const long long rows = (long long)B * T * H, nblk = (T + SWA_BQ - 1) / SWA_BQ;
  hipLaunchKernelGGL(swa_bwd_delta_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, a);
  hipLaunchKernelGGL(swa_bwd_kv_kernel, dim3((unsigned)(B * H * nblk)), dim3(256), 0, st, a);
  hipLaunchKernelGGL(swa_bwd_q_kernel, dim3((unsigned)(B * H * nblk)), dim3(256), 0, st, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "swa backward launch");
}
