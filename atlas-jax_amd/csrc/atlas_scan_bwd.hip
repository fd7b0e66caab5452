// atlas_scan_bwd: the backward (VJP) of the whole-layer chunk scan.
//
// The reference trains through the chunk loop of AtlasMemoryLayer.__call__
// (atlas_jax/memory_layer.py:649-711) by automatic differentiation: each
// chunk's _process_chunk_deep (:496-541) differentiated through the memory
// forward, the inner gradient (:505-520), the Omega window (:522-527) and the
// fused-chunk operator, whose custom VJP recomputes _regular_fwd and
// differentiates it (kernels/fused_chunk.py:357-379, with the reverse-time
// scan of kernels/triton_scan.py:119-161).  This file computes the same
// gradients with explicit reverse-mode formulas, chunk by chunk in reverse
// order, on the caller's stream:
//
//   trace pass     every chunk's start state (W1, W2, S1, S2), by a forward
//                  pass over all chunks but the last (kept in the workspace);
//   per chunk c = n-1 .. 0, from its start state:
//     prep         h = W2 k, act = gelu_tanh(h), err = k + W1 act - v,
//                  w1e = W1^T err, gp = gelu_erf'(h), chain = w1e * gp;
//     mom_fwd      G_t (Omega window of u_i = (2/D) x_i (x) y_i) and
//                  S_t = theta_t S_{t-1} - eta_t G_t for every token;
//     PE           P_t = PolarExpress(S_t) (atlas_pe_batched);
//     mem_fwd      W_t = alpha_t W_{t-1} + P_t;
//     readout_bwd  y_t = q_t + W1_t gelu_tanh(W2_t q_t) backwards: dq, and the
//                  rank-1 cotangents dy (x) gelu(hq) and dhq (x) q of W1_t, W2_t;
//     mem_bwd      reverse scan of W: dP_t, d alpha_t = <What_t, W_{t-1}>;
//     pe_vjp       dS_t = VJP of Polar-Express (identity with pe_ste);
//     mom_bwd      reverse scan of S: Shat_t, d theta_t = <Shat_t, S_{t-1}>,
//                  d eta_t = -<Shat_t, G_t>, and the Omega window's adjoint
//                  M_i = sum_{t=i}^{i+w-1} (-eta_t Shat_t);
//     inner_bwd    d gamma_i, d k_i, d v_i and the inner gradient's
//                  cotangents through both GELUs (the erf GELU's second
//                  derivative enters through u_W2's chain term);
//     wgrad        the chunk-start weights' cotangent (the carry into c - 1);
//     gate_grad    d alpha, d theta, d eta from the per-block partial sums,
//                  added in a fixed order (bitwise reproducible).
// All arithmetic is fp32.  Inputs and outputs are dense fp32 (B, T, H, D) /
// (B, T, H) with T a multiple of the chunk size (the caller pads as the
// reference does, :649-660).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "atlas_common.hpp"
#include "atlas_pe.hpp"
#include "atlas_scan.h"
#include "atlas_status.hpp"

namespace atlas {
// atlas_pe_batched.hip: fp16 Polar-Express of n D x E and n E x D fp32
// matrices (the backward's recompute of both memories), one launch.
atlas_status pe_recompute_both(long long n, int D, int E, int ns, const float* Xa, float* Ya, const float* Xb,
                               float* Yb, hipStream_t st);
}  // namespace atlas

extern "C" atlas_status atlas_pe_batched(int64_t n, int32_t d1, int32_t d2, int32_t ns_steps, int32_t norm_mode,
                                         const void* X, void* Y, int32_t dtype, int32_t compute, void* stream);

namespace atlas {
namespace {

constexpr int BT = 256;           // threads per block
constexpr int NWV = BT / WAVE;    // waves per block
constexpr int EPT = 4;            // state elements per thread in the element-wise scans
constexpr int EBLK = BT * EPT;    // state elements per block
constexpr int VJP_GRID = 256;     // persistent workgroups of the fp32 Polar-Express VJP (one per CU)
constexpr int VJPW_GRID = 256;    // persistent workgroups of the per-wave fp16 VJP (one per CU)

struct BwdArgs {
  int B, T, H, D, E, cs, w, ns, BH, NB, c0;
  int win;                 // Omega window active (w > 1 and gamma given)
  long long DE;
  float scale;             // 2 / D
  const float *q, *k, *v, *al, *et, *th, *ga, *dy;
  const float *W1, *W2, *S1, *S2;   // the chunk's start state
  float *h, *act, *err, *w1e, *gp, *chain, *gq, *dhq, *derr, *dw1e, *dh;   // (BH, cs, .)
  float *Sall[2], *Wall[2], *Pd[2];                                         // (BH, cs, DE)
  float *mrow[2], *mcol[2];   // Omega adjoint products: (BH, cs, rows), (BH, cs, NB, cols)
  float *cW[2], *cS[2], *tW[2];                                            // (BH, DE)
  float* gfin[2];   // (BH, DE): the Omega window sum G of the chunk's last token (nullptr: not kept)
  float *pal, *pth, *pet;                                                  // (2, BH, NB, cs)
  float *dq, *dk, *dv, *dal, *det, *dth, *dga;
};

__device__ __forceinline__ long long xrow(const BwdArgs& a, int b, int hh, int t) {
  return ((long long)(b * a.T + a.c0 + t) * a.H + hh) * a.D;
}
__device__ __forceinline__ long long grow(const BwdArgs& a, int b, int hh, int t) {
  return (long long)(b * a.T + a.c0 + t) * a.H + hh;
}

__device__ __forceinline__ float gelu_tanh_grad(float x) {
  const float c = 0.7978845608028654f;
  const float t = tanhf(c * (x + 0.044715f * x * x * x));
  return 0.5f * (1.f + t) + 0.5f * x * (1.f - t * t) * c * (1.f + 3.f * 0.044715f * x * x);
}
// d/dx of Phi(x) + x phi(x): 2 phi(x) + x phi'(x) = phi(x) (2 - x^2)
__device__ __forceinline__ float gelu_erf_second(float x) {
  return 0.3989422804014327f * expf(-0.5f * x * x) * (2.f - x * x);
}

// Sum over the block; `red` holds 2 * NWV floats, parity p alternates between
// consecutive calls so that one barrier per call suffices.
__device__ __forceinline__ float block_sum(float x, float* red, int p) {
  x = wave_sum(x);
  if (lane_id() == 0) red[p * NWV + wave_id()] = x;
  __syncthreads();
  float s = red[p * NWV];
#pragma unroll
  for (int i = 1; i < NWV; ++i) s += red[p * NWV + i];
  return s;
}

// Block sums of K values with one barrier (the scans reduce K tokens'
// partial products together, so that loads of later tokens are not held up
// by a barrier per token).  red holds 2 * K * NWV floats; p alternates.
template <int K>
__device__ __forceinline__ void block_sum_k(float (&x)[K], float* red, int p) {
#pragma unroll
  for (int j = 0; j < K; ++j) x[j] = wave_sum(x[j]);
  if (lane_id() == 0)
#pragma unroll
    for (int j = 0; j < K; ++j) red[(p * K + j) * NWV + wave_id()] = x[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < K; ++j) {
    float s = red[(p * K + j) * NWV];
#pragma unroll
    for (int i = 1; i < NWV; ++i) s += red[(p * K + j) * NWV + i];
    x[j] = s;
  }
}

__global__ void fill_kernel(float* p, long long n, float v) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Row and column products of a rows x cols fp32 matrix M in global memory
// (16-byte aligned, cols % 4 == 0): out_r[r] = sum_c M[r][c] xc[c] and
// out_c[c] = sum_r M[r][c] xr[r] (either may be skipped with nullptr).  When
// cols / 4 is a power of two up to 64, every element is loaded once, 16
// bytes per thread with consecutive threads on consecutive quads of a row;
// row sums are reduced over the cols / 4 lanes of a row by shuffles, column
// sums through red (LDS, BT * 4 floats).  Other widths take plain loops.
// xr, xc, out_r, out_c live in LDS (16-byte aligned).  Ends with a barrier.
__device__ __forceinline__ void matvec2(const float* M, int rows, int cols, const float* xr, const float* xc,
                                        float* out_r, float* out_c, float* red) {
  const int Q = cols / 4, RR = BT / Q, tid = threadIdx.x, cq = tid % Q, r0 = tid / Q;
  if ((Q & (Q - 1)) != 0 || Q > WAVE) {
    if (out_r)
      for (int r = tid; r < rows; r += BT) {
        float acc = 0.f;
        for (int c = 0; c < cols; ++c) acc = fmaf(M[(long long)r * cols + c], xc[c], acc);
        out_r[r] = acc;
      }
    if (out_c)
      for (int c = tid; c < cols; c += BT) {
        float acc = 0.f;
        for (int r = 0; r < rows; ++r) acc = fmaf(M[(long long)r * cols + c], xr[r], acc);
        out_c[c] = acc;
      }
    __syncthreads();
    return;
  }
  const f32x4 xv = xc ? *reinterpret_cast<const f32x4*>(xc + 4 * cq) : f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 cacc = {0.f, 0.f, 0.f, 0.f};
  for (int r = r0; r < rows; r += RR) {
    const f32x4 m = *reinterpret_cast<const f32x4*>(M + (long long)r * cols + 4 * cq);
    if (out_r) {
      float p = (m[0] * xv[0] + m[1] * xv[1]) + (m[2] * xv[2] + m[3] * xv[3]);
      switch (Q) {   // over the Q lanes of the row
        case 2: p = group_sum<2>(p); break;
        case 4: p = group_sum<4>(p); break;
        case 8: p = group_sum<8>(p); break;
        case 16: p = group_sum<16>(p); break;
        case 32: p = group_sum<32>(p); break;
        case 64: p = group_sum<64>(p); break;
        default: break;
      }
      if (cq == 0) out_r[r] = p;
    }
    if (out_c) cacc += xr[r] * m;
  }
  if (out_c) {
    *reinterpret_cast<f32x4*>(red + r0 * cols + 4 * cq) = cacc;
    __syncthreads();
    for (int c = tid; c < cols; c += BT) {
      float sum = 0.f;
      for (int u = 0; u < RR; ++u) sum += red[u * cols + c];
      out_c[c] = sum;
    }
  }
  __syncthreads();
}

// ---- per token: memory forward at the chunk-start weights ----------------
__global__ void __launch_bounds__(BT) prep_bwd_kernel(BwdArgs a) {
  const int s = blockIdx.x / a.cs, t = blockIdx.x % a.cs, b = s / a.H, hh = s % a.H;
  const int D = a.D, E = a.E;
  __shared__ __attribute__((aligned(16))) float kv[128], ev[128], tmpd[128], av[256], tmpe[256];
  __shared__ __attribute__((aligned(16))) float red[BT * 4];
  const long long xr = xrow(a, b, hh, t), tv = (long long)s * a.cs + t;
  const float* W1 = a.W1 + s * a.DE;   // [d][e]
  const float* W2 = a.W2 + s * a.DE;   // [e][d]
  for (int d = threadIdx.x; d < D; d += BT) kv[d] = a.k[xr + d];
  __syncthreads();
  matvec2(W2, E, D, nullptr, kv, tmpe, nullptr, red);   // h = W2 k
  float gpl = 0.f;
  for (int e = threadIdx.x; e < E; e += BT) {
    const float acc = tmpe[e];
    const float g = gelu_tanh(acc);
    av[e] = g;
    gpl = gelu_erf_prime(acc);
    a.h[tv * E + e] = acc;
    a.act[tv * E + e] = g;
    a.gp[tv * E + e] = gpl;
  }
  __syncthreads();
  matvec2(W1, D, E, nullptr, av, tmpd, nullptr, red);   // W1 gelu(h)
  for (int d = threadIdx.x; d < D; d += BT) {
    const float r = (kv[d] + tmpd[d]) - a.v[xr + d];
    ev[d] = r;
    a.err[tv * D + d] = r;
  }
  __syncthreads();
  matvec2(W1, D, E, ev, nullptr, nullptr, tmpe, red);   // W1^T err
  for (int e = threadIdx.x; e < E; e += BT) {   // E <= BT: gpl is this thread's e
    const float acc = tmpe[e];
    a.w1e[tv * E + e] = acc;
    a.chain[tv * E + e] = acc * gpl;
  }
}

// This thread's four elements (one row) of matrix m: 0 (W1/S1, [d][e]) or
// 1 (W2/S2, [e][d]).
struct Elem {
  int m, s, b, hh, row, col;
  long long i0;
};

__device__ __forceinline__ Elem elem_of(const BwdArgs& a) {
  Elem el;
  el.m = blockIdx.y;
  el.s = blockIdx.x / a.NB;
  const int blk = blockIdx.x % a.NB;
  el.b = el.s / a.H;
  el.hh = el.s % a.H;
  el.i0 = (long long)blk * EBLK + threadIdx.x * EPT;
  const int rl = el.m == 0 ? a.E : a.D;
  el.row = (int)(el.i0 / rl);
  el.col = (int)(el.i0 % rl);
  return el;
}

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }

constexpr int KT = 4;   // tokens per barrier of the momentum scan backwards
// The factors of u_t = (2/D) x_t (x) y_t at this thread's elements: matrix 0:
// x = err (D), y = act (E); matrix 1: x = chain (E), y = k (D).
__device__ __forceinline__ void xy_at(const BwdArgs& a, const Elem& el, int t, float& x, f32x4& y) {
  const long long tv = (long long)el.s * a.cs + t;
  if (el.m == 0) {
    x = a.err[tv * a.D + el.row];
    y = ld4(a.act + tv * a.E + el.col);
  } else {
    x = a.chain[tv * a.E + el.row];
    y = ld4(a.k + xrow(a, el.b, el.hh, t) + el.col);
  }
}
__device__ __forceinline__ float row_group_sum(float x, int lpr) {
  switch (lpr) {
    case 8: return group_sum<8>(x);
    case 16: return group_sum<16>(x);
    case 32: return group_sum<32>(x);
    default: return group_sum<64>(x);
  }
}
// Sum of v over the lanes of the wave that hold the same columns (lane mod
// lpr), lpr in {8, 16, 32, 64}.
__device__ __forceinline__ f32x4 col_wave_sum(f32x4 v, int lpr) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = v[i], p, q;
    if (lpr <= 8) x += __shfl_xor(x, 8);
    if (lpr <= 16) {
      swap16(x, p, q);
      x = p + q;
    }
    if (lpr <= 32) {
      swap32(x, p, q);
      x = p + q;
    }
    v[i] = x;
  }
  return v;
}

// ---- S_t for every token (momentum scan over the Omega-window inputs) ----
// The element-wise scans load a batch of tokens' inputs before using any
// of them: the stores between tokens would otherwise keep the compiler from
// issuing the next token's loads early (it cannot tell them apart), and a
// wave would have one token's loads in flight at a time.
__global__ void __launch_bounds__(BT) mom_fwd_kernel(BwdArgs a, float* fin0, float* fin1) {
  constexpr int KM = 4;
  const Elem el = elem_of(a);
  if (el.i0 >= a.DE) return;   // last block of a state whose size is not a multiple of EBLK
  const long long DE = a.DE, base = (long long)el.s * a.cs * DE + el.i0;
  f32x4 S = ld4((el.m == 0 ? a.S1 : a.S2) + el.s * DE + el.i0);
  f32x4 C = {0.f, 0.f, 0.f, 0.f}, Cl = C;
  for (int tg = 0; tg < a.cs; tg += KM) {
    float th[KM], et[KM], gac[KM], gal[KM], xt[KM], xl[KM];
    f32x4 yt[KM], yl[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      const int t = min(tg + j, a.cs - 1), tl = t - a.w;
      const long long gi = grow(a, el.b, el.hh, t);
      th[j] = a.th[gi];
      et[j] = a.et[gi];
      xy_at(a, el, t, xt[j], yt[j]);
      gac[j] = gal[j] = xl[j] = 0.f;
      yl[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (a.win) {
        gac[j] = a.ga[gi];
        if (tl >= 0) {
          gal[j] = a.ga[grow(a, el.b, el.hh, tl)];
          xy_at(a, el, tl, xl[j], yl[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      const int t = tg + j;
      if (t >= a.cs) break;
      f32x4 G = (a.scale * xt[j]) * yt[j];   // u_t
      if (a.win) {   // cumulative sum minus the sum shifted by the window (memory_layer.py:233-253)
        C += gac[j] * G;
        if (t >= a.w) Cl += gal[j] * ((a.scale * xl[j]) * yl[j]);
        G = C - Cl;
      }
      S = th[j] * S + (-(et[j] * G));
      st4(a.Sall[el.m] + base + (long long)t * DE, S);
      if (t == a.cs - 1 && a.gfin[el.m]) st4(a.gfin[el.m] + el.s * DE + el.i0, G);
    }
  }
  float* fin = el.m == 0 ? fin0 : fin1;
  if (fin) st4(fin + el.s * DE + el.i0, S);
}

// ---- W_t = alpha_t W_{t-1} + P_t ----------------------------------------
__global__ void __launch_bounds__(BT) mem_fwd_kernel(BwdArgs a, float* fin0, float* fin1) {
  const Elem el = elem_of(a);
  if (el.i0 >= a.DE) return;
  const long long DE = a.DE, base = (long long)el.s * a.cs * DE + el.i0;
  f32x4 W = ld4((el.m == 0 ? a.W1 : a.W2) + el.s * DE + el.i0);
  for (int t = 0; t < a.cs; ++t) {   // (a batch of loads first measured slower here)
    const float al = a.al[grow(a, el.b, el.hh, t)];
    W = al * W + ld4(a.Pd[el.m] + base + (long long)t * DE);
    st4(a.Wall[el.m] + base + (long long)t * DE, W);
  }
  float* fin = el.m == 0 ? fin0 : fin1;
  if (fin) st4(fin + el.s * DE + el.i0, W);
}

// ---- read-out backward per token ----------------------------------------
__global__ void __launch_bounds__(BT) readout_bwd_kernel(BwdArgs a) {
  const int s = blockIdx.x / a.cs, t = blockIdx.x % a.cs, b = s / a.H, hh = s % a.H;
  const int D = a.D, E = a.E;
  __shared__ __attribute__((aligned(16))) float qv[64], dyv[64], tmpd[64], dhv[256], hq[256], dg[256];
  __shared__ __attribute__((aligned(16))) float red[BT * 4];
  const long long xr = xrow(a, b, hh, t), tv = (long long)s * a.cs + t;
  const float* W1t = a.Wall[0] + tv * a.DE;   // [d][e]
  const float* W2t = a.Wall[1] + tv * a.DE;   // [e][d]
  for (int d = threadIdx.x; d < D; d += BT) {
    qv[d] = a.q[xr + d];
    dyv[d] = a.dy ? a.dy[xr + d] : 0.f;
  }
  __syncthreads();
  matvec2(W2t, E, D, nullptr, qv, hq, nullptr, red);    // W2_t q
  matvec2(W1t, D, E, dyv, nullptr, nullptr, dg, red);   // W1_t^T dy
  for (int e = threadIdx.x; e < E; e += BT) {
    const float dhq = dg[e] * gelu_tanh_grad(hq[e]);
    a.gq[tv * E + e] = gelu_tanh(hq[e]);
    a.dhq[tv * E + e] = dhq;
    dhv[e] = dhq;
  }
  __syncthreads();
  matvec2(W2t, E, D, dhv, nullptr, nullptr, tmpd, red);   // W2_t^T dhq
  for (int d = threadIdx.x; d < D; d += BT) a.dq[xr + d] = dyv[d] + tmpd[d];
}

// ---- reverse scan of W: dP_t and the alpha partials ----------------------
__global__ void __launch_bounds__(BT) mem_bwd_kernel(BwdArgs a) {
  constexpr int K = 4;   // tokens per partial-sum reduction
  const Elem el = elem_of(a);
  __shared__ float red[2 * K * NWV];
  const long long DE = a.DE, base = (long long)el.s * a.cs * DE + el.i0;
  const int blk = blockIdx.x % a.NB;
  const float* __restrict__ W0 = (el.m == 0 ? a.W1 : a.W2) + el.s * DE + el.i0;
  const float* __restrict__ Wall = a.Wall[el.m] + base;
  float* __restrict__ Pd = a.Pd[el.m] + base;
  f32x4 R = ld4(a.cW[el.m] + el.s * DE + el.i0);
  float* part = a.pal + (((long long)el.m * a.BH + el.s) * a.NB + blk) * a.cs;
  int par = 0;
  for (int tg = a.cs - 1; tg >= 0; tg -= K, par ^= 1) {
    float pv[K], xv[K], alv[K];
    f32x4 yv[K], Wv[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {   // the batch's inputs, all loads in flight together
      const int t = max(tg - j, 0);
      const long long tv = (long long)el.s * a.cs + t;
      const long long xr = xrow(a, el.b, el.hh, t);
      if (el.m == 0) {   // dy_t (x) gelu(hq_t)
        xv[j] = a.dy ? a.dy[xr + el.row] : 0.f;
        yv[j] = ld4(a.gq + tv * a.E + el.col);
      } else {           // dhq_t (x) q_t
        xv[j] = a.dhq[tv * a.E + el.row];
        yv[j] = ld4(a.q + xr + el.col);
      }
      Wv[j] = t > 0 ? ld4(Wall + (long long)(t - 1) * DE) : ld4(W0);
      alv[j] = a.al[grow(a, el.b, el.hh, t)];
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int t = tg - j;
      pv[j] = 0.f;
      if (t < 0) continue;
      R += xv[j] * yv[j];
      st4(Pd + (long long)t * DE, R);
      const f32x4 pr = R * Wv[j];
      pv[j] = (pr[0] + pr[1]) + (pr[2] + pr[3]);
      R = alv[j] * R;
    }
    block_sum_k<K>(pv, red, par);
    if (threadIdx.x == 0)
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (tg - j >= 0) part[tg - j] = pv[j];
  }
  st4(a.tW[el.m] + el.s * DE + el.i0, R);
}

// ---- reverse scan of S, d theta / d eta partials, Omega adjoint ----------
// The Omega adjoint M_t (rows x cols per token) is used only through four
// products in the inner-gradient backward: M1 act, M1^T err, M2 k and
// M2^T chain.  Rather than storing M_t, the scan forms them here, while
// M_t is in registers: the row products complete (a block holds whole rows;
// the lanes of a row are summed by shuffles) into mrow (tok, rows), the
// column products as one partial per block (the block's rows, summed through
// LDS in a fixed order) into mcol (tok, NB, cols).  `col` below is dynamic LDS
// of 2 * KT * NWV * max(D, E) floats.
__global__ void __launch_bounds__(BT) mom_bwd_kernel(BwdArgs a) {
  constexpr int K = KT, KP = 2;   // KP: tokens per load batch
  const Elem el = elem_of(a);
  __shared__ float red[2 * 2 * K * NWV];
  extern __shared__ __attribute__((aligned(16))) float colb[];   // [2][K][NWV][rl]
  const long long DE = a.DE, base = (long long)el.s * a.cs * DE + el.i0;
  const int blk = blockIdx.x % a.NB, wv = wave_id(), lane = lane_id();
  const int rl = el.m == 0 ? a.E : a.D, lpr = rl / 4, nrow = el.m == 0 ? a.D : a.E;
  const float* __restrict__ S0 = (el.m == 0 ? a.S1 : a.S2) + el.s * DE + el.i0;
  const float* __restrict__ Sall = a.Sall[el.m] + base;
  const float* __restrict__ Pd = a.Pd[el.m] + base;
  float* __restrict__ mrow = a.mrow[el.m] + (long long)el.s * a.cs * nrow;
  float* __restrict__ mcol = a.mcol[el.m] + ((long long)el.s * a.cs * a.NB + blk) * rl;
  f32x4 Sh = ld4(a.cS[el.m] + el.s * DE + el.i0);
  // The window sum needs Shat_{t+w} at token t.  Rather than storing Shat and
  // reading it back w tokens later, a second copy of the recurrence runs w
  // tokens behind (ShL = Shat_{t+w}, the same operations in the same order,
  // so bitwise the same values), re-reading dS_{t+w}, which the leading scan
  // loaded w tokens earlier: no per-token store of Shat.
  f32x4 ShL = Sh;
  f32x4 Dsum = {0.f, 0.f, 0.f, 0.f}, Dlag = Dsum;
  // the momentum input G_t, rebuilt backwards from the last token's window
  // sum: G_{t-1} = G_t - gamma_t u_t + gamma_{t-w} u_{t-w} (no window: u_t)
  f32x4 G = a.win ? ld4(a.gfin[el.m] + el.s * DE + el.i0) : Dsum;
  const long long po = (((long long)el.m * a.BH + el.s) * a.NB + blk) * a.cs;
  int par = 0;
  for (int tg = a.cs - 1; tg >= 0; tg -= K, par ^= 1) {
    float vth[K], vet[K];
#pragma unroll
    for (int jh = 0; jh < K; jh += KP) {
    // KP tokens' inputs, all loads in flight together (the stores below
    // would otherwise hold the next token's loads back)
    float thv[KP], etv[KP], xtv[KP], gav[KP], gwv[KP], xwv[KP], etl[KP], thl[KP];
    f32x4 dSv[KP], Spv[KP], ytv[KP], ywv[KP], dSl[KP];
#pragma unroll
    for (int jj = 0; jj < KP; ++jj) {
      const int j = jh + jj;
      const int t = max(tg - j, 0), tw = t - a.w, tl = t + a.w;
      const long long gi = grow(a, el.b, el.hh, t);
      thv[jj] = a.th[gi];
      etv[jj] = a.et[gi];
      dSv[jj] = ld4(Pd + (long long)t * DE);
      Spv[jj] = t > 0 ? ld4(Sall + (long long)(t - 1) * DE) : ld4(S0);
      xy_at(a, el, t, xtv[jj], ytv[jj]);
      gav[jj] = gwv[jj] = xwv[jj] = etl[jj] = thl[jj] = 0.f;
      ywv[jj] = dSl[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (a.win) {
        gav[jj] = a.ga[gi];
        if (tw >= 0) {
          gwv[jj] = a.ga[grow(a, el.b, el.hh, tw)];
          xy_at(a, el, tw, xwv[jj], ywv[jj]);
        }
        if (tl <= a.cs - 1) {
          const long long gl = grow(a, el.b, el.hh, tl);
          dSl[jj] = ld4(Pd + (long long)tl * DE);
          etl[jj] = a.et[gl];
          thl[jj] = a.th[gl];
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < KP; ++jj) {
      const int j = jh + jj;
      const int t = tg - j;
      vth[j] = vet[j] = 0.f;
      if (t < 0) continue;
      const float th = thv[jj], et = etv[jj];
      Sh += dSv[jj];
      const f32x4 pt = Sh * Spv[jj];
      const float xt = xtv[jj];
      const f32x4 yt = ytv[jj];
      const f32x4 ut = (a.scale * xt) * yt;
      if (!a.win) G = ut;
      const f32x4 pe = Sh * G;
      if (a.win) {
        G -= gav[jj] * ut;
        if (t >= a.w) G += gwv[jj] * ((a.scale * xwv[jj]) * ywv[jj]);
      }
      const f32x4 dG = -et * Sh;
      f32x4 M = dG;
      if (a.win) {   // M_t = sum_{u=t}^{min(t+w-1, cs-1)} dG_u
        Dsum += dG;
        const int tl = t + a.w;
        if (tl <= a.cs - 1) {
          ShL += dSl[jj];   // Shat_{tl}
          Dlag += -etl[jj] * ShL;
          ShL = thl[jj] * ShL;
        }
        M = Dsum - Dlag;
      }
      // row product (M y_t) and this wave's part of the column product (x_t^T M)
      const float rp = row_group_sum((M[0] * yt[0] + M[1] * yt[1]) + (M[2] * yt[2] + M[3] * yt[3]), lpr);
      if (lane % lpr == 0) mrow[(long long)t * nrow + el.row] = rp;
      const f32x4 cp = col_wave_sum(xt * M, lpr);
      if (lane < lpr) st4(colb + ((par * K + j) * NWV + wv) * rl + 4 * lane, cp);
      vth[j] = (pt[0] + pt[1]) + (pt[2] + pt[3]);
      vet[j] = (pe[0] + pe[1]) + (pe[2] + pe[3]);
      Sh = th * Sh;
    }
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      vth[j] = wave_sum(vth[j]);
      vet[j] = wave_sum(vet[j]);
    }
    if (lane == 0)
#pragma unroll
      for (int j = 0; j < K; ++j) {
        red[((par * 2 + 0) * K + j) * NWV + wv] = vth[j];
        red[((par * 2 + 1) * K + j) * NWV + wv] = vet[j];
      }
    __syncthreads();
    if (threadIdx.x == 0)
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (tg - j >= 0) {
          float s0 = red[((par * 2 + 0) * K + j) * NWV], s1 = red[((par * 2 + 1) * K + j) * NWV];
#pragma unroll
          for (int i = 1; i < NWV; ++i) {
            s0 += red[((par * 2 + 0) * K + j) * NWV + i];
            s1 += red[((par * 2 + 1) * K + j) * NWV + i];
          }
          a.pth[po + tg - j] = s0;
          a.pet[po + tg - j] = -s1;
        }
    // the block's column partials, summed over its waves in order
    for (int idx = threadIdx.x; idx < K * rl; idx += BT) {
      const int j = idx / rl, c = idx % rl, t = tg - j;
      if (t < 0) continue;
      const float* cb = colb + (par * K + j) * NWV * rl + c;
      float sum = cb[0];
#pragma unroll
      for (int i = 1; i < NWV; ++i) sum += cb[i * rl];
      mcol[(long long)t * a.NB * rl + c] = sum;
    }
  }
  st4(a.cS[el.m] + el.s * DE + el.i0, Sh);
}

// ---- inner-gradient backward per token ----------------------------------
__global__ void __launch_bounds__(BT) inner_bwd_kernel(BwdArgs a) {
  const int s = blockIdx.x / a.cs, t = blockIdx.x % a.cs, b = s / a.H, hh = s % a.H;
  const int D = a.D, E = a.E;
  __shared__ __attribute__((aligned(16))) float errv[64], kv[64], a1v[64], b2v[64], derrv[64], tmpd[64];
  __shared__ __attribute__((aligned(16))) float actv[256], chv[256], b1v[256], a2v[256], dw1ev[256], dhv[256],
      tmpe[256];
  __shared__ __attribute__((aligned(16))) float red[BT * 4];
  const long long xr = xrow(a, b, hh, t), tv = (long long)s * a.cs + t, gi = grow(a, b, hh, t);
  const float* W1 = a.W1 + s * a.DE;
  const float* W2 = a.W2 + s * a.DE;
  for (int d = threadIdx.x; d < D; d += BT) {
    errv[d] = a.err[tv * D + d];
    kv[d] = a.k[xr + d];
  }
  for (int e = threadIdx.x; e < E; e += BT) {
    actv[e] = a.act[tv * E + e];
    chv[e] = a.chain[tv * E + e];
  }
  __syncthreads();
  const float g1 = a.win ? a.ga[gi] * a.scale : a.scale;
  // a1 = M1 act, b1 = M1^T err; a2 = M2 k, b2 = M2^T chain (from the
  // momentum scan backwards: rows complete, columns as per-block partials
  // summed in block order)
  {
    const int NB = a.NB;
    const float* r1 = a.mrow[0] + tv * D;
    const float* r2 = a.mrow[1] + tv * E;
    const float* c1 = a.mcol[0] + tv * NB * E;
    const float* c2 = a.mcol[1] + tv * NB * D;
    for (int d = threadIdx.x; d < D; d += BT) {
      a1v[d] = r1[d];
      float sum = c2[d];
      for (int i = 1; i < NB; ++i) sum += c2[i * D + d];
      b2v[d] = sum;
    }
    for (int e = threadIdx.x; e < E; e += BT) {
      a2v[e] = r2[e];
      float sum = c1[e];
      for (int i = 1; i < NB; ++i) sum += c1[i * E + e];
      b1v[e] = sum;
    }
  }
  __syncthreads();
  float dot = 0.f;
  for (int d = threadIdx.x; d < D; d += BT) dot = fmaf(errv[d], a1v[d], dot);
  for (int e = threadIdx.x; e < E; e += BT) dot = fmaf(chv[e], a2v[e], dot);
  const float tot = block_sum(dot, red, 0);
  if (threadIdx.x == 0 && a.win && a.dga) a.dga[gi] = a.scale * tot;
  for (int e = threadIdx.x; e < E; e += BT) {
    const float hv = a.h[tv * E + e];
    const float dch = g1 * a2v[e];
    const float dw = dch * a.gp[tv * E + e];
    dw1ev[e] = dw;
    a.dw1e[tv * E + e] = dw;
    dhv[e] = dch * a.w1e[tv * E + e] * gelu_erf_second(hv);   // through gelu_erf'(h)
  }
  __syncthreads();
  matvec2(W1, D, E, nullptr, dw1ev, tmpd, nullptr, red);   // W1 dw1e
  for (int d = threadIdx.x; d < D; d += BT) {
    const float de = g1 * a1v[d] + tmpd[d];
    derrv[d] = de;
    a.derr[tv * D + d] = de;
    a.dv[xr + d] = -de;
  }
  __syncthreads();
  matvec2(W1, D, E, derrv, nullptr, nullptr, tmpe, red);   // W1^T derr
  for (int e = threadIdx.x; e < E; e += BT) {
    const float dact = g1 * b1v[e] + tmpe[e];
    const float dh = dhv[e] + dact * gelu_tanh_grad(a.h[tv * E + e]);
    dhv[e] = dh;   // this thread's own element
    a.dh[tv * E + e] = dh;
  }
  __syncthreads();
  matvec2(W2, E, D, dhv, nullptr, nullptr, tmpd, red);   // W2^T dh
  for (int d = threadIdx.x; d < D; d += BT) a.dk[xr + d] = g1 * b2v[d] + derrv[d] + tmpd[d];
}

// ---- the chunk-start weights' cotangent (carry into the previous chunk) ----
// cW[m] = tW[m] + sum_t x_t (x) y_t over the chunk's tokens, a product of
// (rows x cs) and (cs x cols) token matrices on the matrix cores (fp32
// v_mfma_f32_32x32x2f32), one 32 x 32 tile per wave: matrix 0 ([d][e]):
// err^T dw1e + derr^T act; matrix 1 ([e][d]): dh^T k.  D and E are
// multiples of 32.  The A operand of step t0 is lane (c, h) = x_{t0+h}[32I + c],
// the B operand y_{t0+h}[32J + c] (zero past an odd chunk's last token).
__global__ void __launch_bounds__(BT) wgrad_kernel(BwdArgs a) {
  const int nt = (a.D / 32) * (a.E / 32);
  const long long wv = (long long)blockIdx.x * NWV + wave_id();
  if (wv >= (long long)a.BH * 2 * nt) return;   // no barrier below
  const int s = (int)(wv / (2 * nt)), rem = (int)(wv % (2 * nt)), m = rem / nt, tile = rem % nt;
  const int rows = m == 0 ? a.D : a.E, cols = m == 0 ? a.E : a.D, I = tile / (cols / 32), J = tile % (cols / 32);
  const int c = lane_id() & 31, h = lane_id() >> 5;
  const long long o = (long long)s * a.DE + (long long)(32 * I) * cols + 32 * J + c;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = a.tW[m][o + (long long)crow(r, h) * cols];
  const long long tv0 = (long long)s * a.cs;
  if (m == 0) {
    const float* x1 = a.err + tv0 * a.D + 32 * I + c;
    const float* x2 = a.derr + tv0 * a.D + 32 * I + c;
    const float* y1 = a.dw1e + tv0 * a.E + 32 * J + c;
    const float* y2 = a.act + tv0 * a.E + 32 * J + c;
#pragma unroll 8
    for (int t0 = 0; t0 < a.cs; t0 += 2) {
      const bool ok = t0 + h < a.cs;   // else row 0, multiplied by zero
      const long long od = ok ? (long long)(t0 + h) * a.D : 0, oe = ok ? (long long)(t0 + h) * a.E : 0;
      const float u1 = x1[od], v1 = y1[oe], u2 = x2[od], v2 = y2[oe];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ok ? u1 : 0.f, v1, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ok ? u2 : 0.f, v2, acc, 0, 0, 0);
    }
  } else {
    const int b = s / a.H, hh = s % a.H;
    const float* x = a.dh + tv0 * a.E + 32 * I + c;
#pragma unroll 8
    for (int t0 = 0; t0 < a.cs; t0 += 2) {
      const bool ok = t0 + h < a.cs;
      const int t = ok ? t0 + h : 0;
      const float u = x[(long long)t * a.E], v = a.k[xrow(a, b, hh, t) + 32 * J + c];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ok ? u : 0.f, v, acc, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) a.cW[m][o + (long long)crow(r, h) * cols] = acc[r];
}

// ---- gate gradients from the partial sums (fixed order) -------------------
// One launch after the last chunk: block (s, c) adds chunk c's partials,
// kept per chunk (pchunk floats apart) so that no chunk waits for this.
__global__ void gate_grad_kernel(BwdArgs a, long long pchunk, long long cbase) {
  const int s = blockIdx.x, t = threadIdx.x;
  const long long c = cbase + blockIdx.y;
  if (t >= a.cs) return;
  a.c0 = (int)(c * a.cs);
  const long long off = c * pchunk;
  float sa = 0.f, st_ = 0.f, se = 0.f;
  for (int m = 0; m < 2; ++m)
    for (int blk = 0; blk < a.NB; ++blk) {
      const long long o = off + (((long long)m * a.BH + s) * a.NB + blk) * a.cs + t;
      sa += a.pal[o];
      st_ += a.pth[o];
      se += a.pet[o];
    }
  const long long gi = grow(a, s / a.H, s % a.H, t);
  a.dal[gi] = sa;
  a.dth[gi] = st_;
  a.det[gi] = se;
}

// ---- Polar-Express VJP per matrix ----------------------------------------
// One workgroup per matrix at a time (persistent over the batch).  The matrix
// X (D x E, E >= D; `tall` = stored transposed, E x D) and its cotangent live
// in LDS as fp32 (for 64 x 256, where they and the four D x D products would
// need 198 KiB, in the workgroup's global scratch instead: all waves of a
// workgroup share one CU's L1, and every exchange through them is ordered by
// a workgroup barrier); the iterates Y_0 .. Y_{ns-2} of the forward
// recompute are kept in a per-workgroup global scratch area.  Products use fp32 MFMA
// (v_mfma_f32_32x32x2f32) with operands read from LDS.  VJP of one step
// Y' = a Y + (b A + c A^2) Y, A = Y Y^T, for the cotangent G of Y':
//   G_Y = a G + B G + (b Gs + c (Gs A + A Gs)) Y,  Gs = G Y^T + Y G^T;
// then the normalisation's VJP: dX = G / nrm - (<G, X> 1.01 / (nrm^2 n)) X.

// acc += sum_k A(r, k) B(k, c) for tile (I, J); A(r, k) = Ap[r*ars + k*aks],
// B(k, c) = Bp[k*bks + c*bcs].
__device__ __forceinline__ f32x16 tile_mma(f32x16 acc, int I, int J, int K, const float* Ap, int ars, int aks,
                                           const float* Bp, int bks, int bcs) {
  const int c = lane_id() & 31, hf = lane_id() >> 5;
  const float* ap = Ap + (32 * I + c) * ars + hf * aks;
  const float* bp = Bp + hf * bks + (32 * J + c) * bcs;
#pragma unroll 8
  for (int k0 = 0; k0 < K; k0 += 2)
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ap[k0 * aks], bp[k0 * bks], acc, 0, 0, 0);
  return acc;
}

template <int D, int E>
struct VjpLds {
  static constexpr int LE = E + 1, LD = D + 1;   // odd row strides: conflict-free column reads
  // the iterate Y and the cotangent Gb in LDS (else in the global scratch)
  static constexpr bool YG_LDS = (2 * D * LE + 4 * D * LD + 2 * NWV) * sizeof(float) <= 160 * 1024;
  static constexpr int bytes() { return ((YG_LDS ? 2 * D * LE : 0) + 4 * D * LD + 2 * NWV) * (int)sizeof(float); }
  // per-workgroup global scratch (floats): the iterates, and Y and Gb when not in LDS
  static constexpr size_t scratch_floats(int ns) {
    return (size_t)(ns > 1 ? ns - 1 : 1) * D * E + (YG_LDS ? 0 : (size_t)2 * D * LE);
  }
};

template <int D, int E>
__global__ void __launch_bounds__(BT) pe_vjp_kernel(long long n, int ns, int tall, const float* X, float* G,
                                                    float* scratch) {
  using LY = VjpLds<D, E>;
  constexpr int LE = LY::LE, LD = LY::LD;
  constexpr int TN = (D / 32) * (E / 32), TA = (D / 32) * (D / 32);
  constexpr int TNW = (TN + NWV - 1) / NWV, TAW = (TA + NWV - 1) / NWV;
  extern __shared__ __attribute__((aligned(16))) float sm[];
  float* scr = scratch + (long long)blockIdx.x * LY::scratch_floats(ns);
  float* Y = LY::YG_LDS ? sm : scr + (size_t)(ns > 1 ? ns - 1 : 1) * D * E;
  float* Gb = Y + D * LE;
  float* A = LY::YG_LDS ? Gb + D * LE : sm;
  float* Bm = A + D * LD;
  float* Gs = Bm + D * LD;
  float* T1 = Gs + D * LD;
  float* red = T1 + D * LD;
  const int tid = threadIdx.x, wv = wave_id(), c = lane_id() & 31, hf = lane_id() >> 5;

  auto at = [&](long long base, int d, int e) -> long long {
    return base + (tall ? (long long)e * D + d : (long long)d * E + e);
  };
  // A = Y Y^T into A, then Bm = b A + c A^2 (T1 scratch)
  auto gram_b = [&](float b, float cc) {
    for (int tl = wv; tl < TA; tl += NWV) {
      const int I = tl / (D / 32), J = tl % (D / 32);
      const f32x16 acc = tile_mma(zero16(), I, J, E, Y, LE, 1, Y, 1, LE);
#pragma unroll
      for (int r = 0; r < 16; ++r) A[(32 * I + crow(r, hf)) * LD + 32 * J + c] = acc[r];
    }
    __syncthreads();
    for (int tl = wv; tl < TA; tl += NWV) {
      const int I = tl / (D / 32), J = tl % (D / 32);
      const f32x16 acc = tile_mma(zero16(), I, J, D, A, LD, 1, A, LD, 1);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = (32 * I + crow(r, hf)) * LD + 32 * J + c;
        Bm[o] = b * A[o] + cc * acc[r];
      }
    }
    __syncthreads();
  };

  for (long long mi = blockIdx.x; mi < n; mi += gridDim.x) {
    const long long base = mi * D * E;
    float ss = 0.f;
    for (int i = tid; i < D * E; i += BT) {
      const int d = i / E, e = i % E;
      const float x = X[at(base, d, e)];
      Y[d * LE + e] = x;
      ss = fmaf(x, x, ss);
    }
    const float nn = sqrtf(block_sum(ss, red, 0) + 1e-12f);
    const float nrm = nn * 1.01f + 1e-6f;
    for (int i = tid; i < D * E; i += BT) {
      const int d = i / E, e = i % E;
      Y[d * LE + e] = Y[d * LE + e] / nrm;
    }
    __syncthreads();
    // forward recompute: Y_0 .. Y_{ns-1}; Y_0 .. Y_{ns-2} to scratch
    for (int k = 0; k + 1 < ns; ++k) {
      for (int i = tid; i < D * E; i += BT) scr[(long long)k * D * E + i] = Y[(i / E) * LE + i % E];
      gram_b(kPE[k][1], kPE[k][2]);
      f32x16 acc[TNW];
#pragma unroll
      for (int q = 0; q < TNW; ++q) {
        const int tl = wv + q * NWV;
        if (tl < TN) acc[q] = tile_mma(zero16(), tl / (E / 32), tl % (E / 32), D, Bm, LD, 1, Y, LE, 1);
      }
      __syncthreads();
      const float ak = kPE[k][0];
#pragma unroll
      for (int q = 0; q < TNW; ++q) {
        const int tl = wv + q * NWV;
        if (tl >= TN) continue;
        const int I = tl / (E / 32), J = tl % (E / 32);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int o = (32 * I + crow(r, hf)) * LE + 32 * J + c;
          Y[o] = ak * Y[o] + acc[q][r];
        }
      }
      __syncthreads();
    }
    // backward through the steps
    for (int i = tid; i < D * E; i += BT) Gb[(i / E) * LE + i % E] = G[at(base, i / E, i % E)];
    __syncthreads();
    for (int k = ns - 1; k >= 0; --k) {
      if (k + 1 < ns) {
        for (int i = tid; i < D * E; i += BT) Y[(i / E) * LE + i % E] = scr[(long long)k * D * E + i];
        __syncthreads();
      }
      const float ak = kPE[k][0], bk = kPE[k][1], ck = kPE[k][2];
      gram_b(bk, ck);
      // Gh = Gb Y^T -> T1, then Gs = Gh + Gh^T
      for (int tl = wv; tl < TA; tl += NWV) {
        const int I = tl / (D / 32), J = tl % (D / 32);
        const f32x16 acc = tile_mma(zero16(), I, J, E, Gb, LE, 1, Y, 1, LE);
#pragma unroll
        for (int r = 0; r < 16; ++r) T1[(32 * I + crow(r, hf)) * LD + 32 * J + c] = acc[r];
      }
      __syncthreads();
      for (int i = tid; i < D * D; i += BT) {
        const int r = i / D, q = i % D;
        Gs[r * LD + q] = T1[r * LD + q] + T1[q * LD + r];
      }
      __syncthreads();
      // T1 = Gs A + A Gs, then Gs <- b Gs + c T1
      for (int tl = wv; tl < TA; tl += NWV) {
        const int I = tl / (D / 32), J = tl % (D / 32);
        f32x16 acc = tile_mma(zero16(), I, J, D, Gs, LD, 1, A, LD, 1);
        acc = tile_mma(acc, I, J, D, A, LD, 1, Gs, LD, 1);
#pragma unroll
        for (int r = 0; r < 16; ++r) T1[(32 * I + crow(r, hf)) * LD + 32 * J + c] = acc[r];
      }
      __syncthreads();
      for (int i = tid; i < D * D; i += BT) {
        const int o = (i / D) * LD + i % D;
        Gs[o] = bk * Gs[o] + ck * T1[o];
      }
      __syncthreads();
      // Gb <- a Gb + Bm Gb + Gs Y
      f32x16 acc[TNW];
#pragma unroll
      for (int q = 0; q < TNW; ++q) {
        const int tl = wv + q * NWV;
        if (tl >= TN) continue;
        const int I = tl / (E / 32), J = tl % (E / 32);
        acc[q] = tile_mma(zero16(), I, J, D, Bm, LD, 1, Gb, LE, 1);
        acc[q] = tile_mma(acc[q], I, J, D, Gs, LD, 1, Y, LE, 1);
      }
      __syncthreads();
#pragma unroll
      for (int q = 0; q < TNW; ++q) {
        const int tl = wv + q * NWV;
        if (tl >= TN) continue;
        const int I = tl / (E / 32), J = tl % (E / 32);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int o = (32 * I + crow(r, hf)) * LE + 32 * J + c;
          Gb[o] = ak * Gb[o] + acc[q][r];
        }
      }
      __syncthreads();
    }
    // normalisation
    float dot = 0.f;
    for (int i = tid; i < D * E; i += BT) dot = fmaf(Gb[(i / E) * LE + i % E], X[at(base, i / E, i % E)], dot);
    const float coef = block_sum(dot, red, 1) * 1.01f / (nrm * nrm * nn);
    for (int i = tid; i < D * E; i += BT) {
      const long long o = at(base, i / E, i % E);
      G[o] = Gb[(i / E) * LE + i % E] / nrm - coef * X[o];
    }
    __syncthreads();
  }
  (void)TAW;
}

template <int D, int E>
atlas_status launch_vjp(long long n, int ns, int tall, const float* X, float* G, float* scratch, hipStream_t st) {
  const int bytes = VjpLds<D, E>::bytes();
  static bool attr_set = false;   // the attribute is per function, not per device
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&pe_vjp_kernel<D, E>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return fail_hip(e, "pe_vjp shared-memory attribute");
    attr_set = true;
  }
  const long long grid = std::min<long long>(n, VJP_GRID);
  hipLaunchKernelGGL((pe_vjp_kernel<D, E>), dim3((unsigned)grid), dim3(BT), bytes, st, n, ns, tall, X, G, scratch);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_vjp launch");
}

// ---- Polar-Express VJP with fp16 operands, one matrix per wave ------------
// The VJP of polar_express_wave_t (the forward's Polar-Express): the iterate
// is carried scaled, Z_0 = 32 X / nrm, Z_{k+1} = Z_k + rho_k (kappa_k A_k +
// A_k^2) Z_k with A_k = Z_k Z_k^T, P = tau_ns Z_ns (kPEt, kPEtau).  Each
// step is p(Z) = a Z + b A Z + c A^2 Z with (a, b, c) = (1, rho kappa, rho),
// so for the cotangent G of Z_{k+1}:
//   G_k = G + B G + (b Gs + c (Gs A + A Gs)) Z,  Gs = G Z^T + Z G^T,
// B = b A + c A^2; then the normalisation's VJP
//   dX = (32 / nrm) G_0 - (32 * 1.01 <G_0, X> / (nrm^2 nn)) X.
// One wave owns one matrix (one workgroup of four waves per CU, persistent
// over the batch; no workgroup barrier).  The iterate Z is held in registers
// as MFMA C-layout tiles in fp32 exactly as polar_express_wave_t holds it;
// the cotangent G as fp16 C-layout fragments with a power-of-two scale.  The
// iterates are recomputed rather than stored: the wave's LDS keeps the fp16
// image of Z_cp (cp = (ns - 1) / 2), Z_k is recomputed from it for k > cp
// and from X for k < cp (ns = 5: six forward steps instead of four; no
// global scratch, so only X, dP and dX move through HBM).  Gram and Gs take
// their operands from transposing LDS reads of Z and G staged as rows e (the
// layout of PEWaveT's staging); A, B, Gs and C are symmetric, so their C
// tiles serve as MFMA operands as they are.  Gs and C are power-of-two
// scaled into fp16's range before rounding; A and B are in range by the
// forward's own design (PEWaveT::apply_scaled).  LDS per wave: two staged
// blocks each of Z and G and the image (35 KiB for 64 x 128).
template <int D, int E>
struct VjpWave {
  using PT = PEWaveT<D, E>;
  using W = PEWave<ModeF16, D, E>;
  using M = ModeF16;
  using frag = f16x8;
  static constexpr int TI = D / 32, TJ = E / 32;
  static constexpr int ZH = 2 * PT::BLOCK;           // Z staged two blocks at a time (halves)
  static constexpr int GH = 2 * PT::BLOCK;           // G staged two blocks at a time
  static constexpr int HALVES = ZH + GH + D * E;     // LDS per wave: staging and the checkpoint image
  static constexpr int bytes() { return NWV * HALVES * 2; }

  template <int R, int C>
  __device__ __forceinline__ static float maxabs(const f32x16 (&t)[R][C]) {
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int j = 0; j < C; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, fabsf(t[i][j][r]));
    return wave_max(m);
  }

  // Row block I (rows 32I .. 32I + 31) of a D x E matrix (or of its
  // transpose when tall) into C-layout tiles of the wide form.  vec 1: tall,
  // 16-byte aligned rows of D floats.  vec 2: not tall with E = 128, 16-byte
  // aligned: tile J's lane c holds column 4c + J instead of 32J + c (every
  // product here is invariant under a common permutation of the columns), so
  // that a lane's four tiles take one 16-byte load per row.
  // Every access is a per-lane base (passed through PT::opaque, so that the
  // compiler forms it here instead of keeping one 64-bit address per element
  // live across the matrix loop) plus a compile-time offset.
  __device__ __forceinline__ static int lane_off(int tall, int vec) {
    const int c = lane_id() & 31, h = lane_id() >> 5;
    return PT::opaque(vec == 2 ? 4 * h * E + 4 * c : tall ? c * D + 4 * h : 4 * h * E + c);
  }
  __device__ __forceinline__ static void load_rows(f32x16 (&T)[TJ], int I, const float* src, int tall, int vec) {
    const float* p = src + lane_off(tall, vec);
    if constexpr (TJ == 4) {
      if (vec == 2) {   // row 32I + 8(r/4) + 4h + r%4, columns 4c .. 4c + 3
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(p + (32 * I + 8 * (r / 4) + r % 4) * E);
#pragma unroll
          for (int J = 0; J < 4; ++J) T[J][r] = v[J];
        }
        return;
      }
    }
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      if (vec) {   // column e = 32J + c: rows 32I + 8q + 4h .. + 3 contiguous
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(p + 32 * J * D + 32 * I + 8 * q);
#pragma unroll
          for (int u = 0; u < 4; ++u) T[J][4 * q + u] = v[u];
        }
      } else if (tall) {
#pragma unroll
        for (int r = 0; r < 16; ++r) T[J][r] = p[32 * J * D + 32 * I + 8 * (r / 4) + r % 4];
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) T[J][r] = p[(32 * I + 8 * (r / 4) + r % 4) * E + 32 * J];
      }
    }
  }
  __device__ __forceinline__ static void store_rows(float* dst, const f32x16 (&T)[TJ], int I, int tall, int vec) {
    float* p = dst + lane_off(tall, vec);
    if constexpr (TJ == 4) {
      if (vec == 2) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          *reinterpret_cast<f32x4*>(p + (32 * I + 8 * (r / 4) + r % 4) * E) = f32x4{T[0][r], T[1][r], T[2][r], T[3][r]};
        return;
      }
    }
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      if (vec) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(p + 32 * J * D + 32 * I + 8 * q) =
              f32x4{T[J][4 * q], T[J][4 * q + 1], T[J][4 * q + 2], T[J][4 * q + 3]};
      } else if (tall) {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[32 * J * D + 32 * I + 8 * (r / 4) + r % 4] = T[J][r];
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[(32 * I + 8 * (r / 4) + r % 4) * E + 32 * J] = T[J][r];
      }
    }
  }
  __device__ __forceinline__ static void load(f32x16 (&T)[TI][TJ], const float* src, int tall, int vec) {
#pragma unroll
    for (int I = 0; I < TI; ++I) load_rows(T[I], I, src, tall, vec);
  }

  // Stages the fp16 C-layout fragments of column block J of a D x E matrix as
  // rows e (PEWaveT's staging layout) at buf
  __device__ __forceinline__ static void stage(const frag (&F)[TI][TJ][2], int J, _Float16* buf, int wo) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 2; ++g)   // elements 4g..4g+3 of fragment kb are rows 32I + 16kb + 8g + 4h + 0..3
          *reinterpret_cast<f16x4*>(buf + wo + 32 * I + 16 * kb + 8 * g) =
              f16x4{F[I][J][kb][4 * g], F[I][J][kb][4 * g + 1], F[I][J][kb][4 * g + 2], F[I][J][kb][4 * g + 3]};
  }

  // fp16 image of Z (C-layout fragments) in the wave's LDS, lane-contiguous
  // 16-byte records
  __device__ __forceinline__ static void put_image(const f32x16 (&Z)[TI][TJ], frag* img) {
    img += PT::opaque(lane_id());
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) img[((I * TJ + J) * 2 + kb) * WAVE] = M::from_c(Z[I][J], kb);
  }
  __device__ __forceinline__ static void get_image(f32x16 (&Z)[TI][TJ], const frag* img) {
    img += PT::opaque(lane_id());
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const frag f = img[((I * TJ + J) * 2 + kb) * WAVE];
#pragma unroll
          for (int v = 0; v < 8; ++v) Z[I][J][8 * kb + v] = (float)f[v];
        }
  }
  // the forward's own steps (polar_express_wave_t: the symmetric step at D = 64)
  __device__ __forceinline__ static void fwd_steps(f32x16 (&Z)[TI][TJ], int st0, int st1, _Float16* zs) {
    for (int st = st0; st < st1; ++st) {
      f32x16 A[TI][TI];
      PT::gram_sym(Z, A, zs);
      PT::apply_sym(Z, A, st, zs);
    }
  }

  // G <- the cotangent of Z_k from the cotangent of Z_{k+1}, for Z = Z_k
  // (fp32, consumed).  G is held as fp16 C-layout fragments Gh = fp16(sG G)
  // with a power-of-two scale sG, renormalised at the start of the step
  // (fp16 keeps 11 significant bits over its whole normal range, so each
  // step adds only the rounding of its result).  With with_dot (the last
  // step, k = 0) it also adds sG <G_0, Z_0> (Z_0 rounded to fp16) to dot (a
  // reference, not a pointer: the accumulator then stays in a register).
  __device__ __forceinline__ static void reverse_step(const f32x16 (&Z)[TI][TJ], frag (&Gh)[TI][TJ][2], float& sG,
                                                      int k, _Float16* zs, _Float16* gs, float& dot, bool with_dot) {
    const float kap = kPEt[k][0], rho = kPEt[k][1];
    {
      float m = 0.f;
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 8; ++v) m = fmaxf(m, fabsf((float)Gh[I][J][kb][v]));
      const float r = pow2_scale(wave_max(m));
      if (r != 1.f) {
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int J = 0; J < TJ; ++J)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
              for (int v = 0; v < 8; ++v) Gh[I][J][kb][v] = (_Float16)((float)Gh[I][J][kb][v] * r);
        sG *= r;
      }
    }
    frag Zc[TI][TJ][2];
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Zc[I][J][kb] = M::from_c(Z[I][J], kb);
    // A = Z Z^T and S = sG (G Z^T + Z G^T), block by block over e.  A, S, B
    // and C are symmetric: with TI == 2 only their tiles (0,0), (0,1), (1,1)
    // are formed, and the operand fragments of tile (1,0) come from tile
    // (0,1) through a staging block with k-slot-ordered transposing reads
    // (PEWaveT's symmetric step): 172 instead of 208 matrix-core products
    constexpr bool SYM = TI == 2;
    f32x16 A[TI][TI], S[TI][TI];
    const int wo = PT::opaque(PT::wr_off()), ro = PT::opaque(PT::rd_off());
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      _Float16* zb = zs + (J & 1) * PT::BLOCK;
      _Float16* gb = gs + (J & 1) * PT::BLOCK;
      stage(Zc, J, zb, wo);
      stage(Gh, J, gb, wo);
      frag zt[TI][2], gt[TI][2];
      PT::read_block(zt, zb, ro);
      PT::read_block(gt, gb, ro);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = SYM ? I : 0; I2 < TI; ++I2) {
            const bool first = J == 0 && kb == 0;
            A[I][I2] = M::mma(zt[I][kb], zt[I2][kb], first ? zero16() : A[I][I2]);
            S[I][I2] = M::mma(gt[I][kb], zt[I2][kb], first ? zero16() : S[I][I2]);
            S[I][I2] = M::mma(zt[I][kb], gt[I2][kb], S[I][I2]);
          }
    }
    // the staging blocks are free once the reads above are issued (LDS
    // operations of one wave complete in order): tile (1,0) of A, S, B, C
    // through zs[0], zs[1], gs[0], gs[1]
    const int rks = PT::opaque(PT::rd_off_ks());
    auto lower = [&](const f32x16& t01, float sc_, _Float16* buf, frag (&F)[TI][TI][2]) {
      if constexpr (SYM) {
        PT::put_tile(t01, sc_, buf, wo);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) F[1][0][kb] = PT::get_tr_ks(buf, kb, rks);
      }
    };
    auto maxabs_sym = [&](const f32x16 (&t)[TI][TI]) {
      if constexpr (SYM) {
        float m = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          m = fmaxf(m, fmaxf(fabsf(t[0][0][r]), fmaxf(fabsf(t[0][1][r]), fabsf(t[1][1][r]))));
        return wave_max(m);
      } else {
        return maxabs(t);
      }
    };
    // B = rho (kappa A + A^2) (the forward's update matrix), formed in A's
    // registers; C = b Gs + c (Gs A + A Gs) scaled as sG s2 C, formed in S's
    frag Af[TI][TI][2], Bf[TI][TI][2], Sf[TI][TI][2], Cf[TI][TI][2];
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = SYM ? K : 0; I < TI; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Af[K][I][kb] = M::from_c(A[K][I], kb);
    lower(A[0][1], 1.f, zs, Af);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = SYM ? I : 0; I2 < TI; ++I2) {
        A[I][I2] = A[I][I2] * kap;
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) A[I][I2] = M::mma(Af[K][I][kb], Af[K][I2][kb], A[I][I2]);
        const f32x16 t = A[I][I2] * rho;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Bf[I][I2][kb] = M::from_c(t, kb);   // symmetric: tile (I, I2) = (I2, I)^T
      }
    lower(A[0][1], rho, gs, Bf);
    const float s2 = pow2_scale(maxabs_sym(S));
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = SYM ? K : 0; I < TI; ++I) {
        const f32x16 t = S[K][I] * s2;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Sf[K][I][kb] = M::from_c(t, kb);
      }
    lower(S[0][1], s2, zs + PT::BLOCK, Sf);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = SYM ? I : 0; I2 < TI; ++I2) {
        S[I][I2] = S[I][I2] * (kap * s2);
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            S[I][I2] = M::mma(Sf[K][I][kb], Af[K][I2][kb], S[I][I2]);
            S[I][I2] = M::mma(Af[K][I][kb], Sf[K][I2][kb], S[I][I2]);
          }
        S[I][I2] = S[I][I2] * rho;
      }
    const float sc = pow2_scale(maxabs_sym(S));
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = SYM ? K : 0; I < TI; ++I) {
        const f32x16 t = S[K][I] * sc;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Cf[K][I][kb] = M::from_c(t, kb);
      }
    lower(S[0][1], sc, gs + PT::BLOCK, Cf);
    // G <- G + B G + C Z, one 32-column block at a time
    const float u2 = 1.f / (s2 * sc);
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      frag gf[TI][2];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) gf[K][kb] = Gh[K][J][kb];
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        f32x16 a1, a2 = zero16();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 8; ++v) a1[8 * kb + v] = (float)gf[I][kb][v];
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            a1 = M::mma(Bf[K][I][kb], gf[K][kb], a1);
            a2 = M::mma(Cf[K][I][kb], Zc[K][J][kb], a2);
          }
        const f32x16 t = a1 + a2 * u2;
        if (with_dot) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 8; ++v) dot = fmaf(t[8 * kb + v], (float)Zc[I][J][kb][v], dot);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Gh[I][J][kb] = M::from_c(t, kb);
      }
    }
  }
};

// One matrix of the fp16 VJP on one wave (Xm: the input, Gm: the cotangent,
// overwritten with dX).  VEC: the load/store path of VjpWave::load_rows (a
// template parameter: one body that holds all three paths keeps far more
// registers live).
template <int D, int E, int VEC>
__device__ __forceinline__ void vjp_wave_one(const float* Xm, float* Gm, int ns, int tall, _Float16* zs,
                                             _Float16* gs, f16x8* ckpt) {
  constexpr int vec = VEC;
  using V = VjpWave<D, E>;
  using M = ModeF16;
  using frag = f16x8;
  constexpr int TI = D / 32, TJ = E / 32;
  const int cp = (ns - 1) / 2;   // the checkpointed iterate (ns >= 2)
  {
    f32x16 Z[TI][TJ];
    V::load(Z, Xm, tall, vec);
    const float nn = sqrtf(V::W::sumsq(Z) + 1e-12f), nrm = nn * 1.01f + 1e-6f, s0 = 32.f / nrm;
    V::W::scale(Z, s0);
    // forward (polar_express_wave_t) up to Z_{ns-1}, keeping the image of Z_cp
    for (int st = 0; st + 1 < ns; ++st) {
      if (st == cp) V::put_image(Z, ckpt);
      V::fwd_steps(Z, st, st + 1, zs);
    }
    // the cotangent of Z_ns is tau_ns dP
    frag Gh[TI][TJ][2];
    float sG;
    {
      f32x16 Gb[TI][TJ];
      V::load(Gb, Gm, tall, vec);
      sG = pow2_scale(V::maxabs(Gb) * kPEtau[ns]);
      const float f = sG * kPEtau[ns];
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) Gh[I][J][kb] = M::from_c(Gb[I][J] * f, kb);
    }
    // backward sweep; Z_k recomputed from the image of Z_cp (k > cp) or from X (k < cp)
    float dot = 0.f;
    for (int k = ns - 1; k >= 0; --k) {
      if (k < ns - 1) {
        if (k >= cp) {
          V::get_image(Z, ckpt);
          V::fwd_steps(Z, cp, k, zs);
        } else {
          V::load(Z, Xm, tall, vec);
          V::W::scale(Z, s0);
          V::fwd_steps(Z, 0, k, zs);
        }
      }
      V::reverse_step(Z, Gh, sG, k, zs, gs, dot, k == 0);
    }
    // dX = s0 G_0 - (32 * 1.01 <G_0, X> / (nrm^2 nn)) X, with <G_0, X> = <G_0, Z_0> / s0
    const float ig = 1.f / sG;
    if (ns == 0) {
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 8; ++v) dot = fmaf((float)Gh[I][J][kb][v], Z[I][J][8 * kb + v], dot);   // Z = Z_0
    }
    const float coef = wave_sum(dot) * ig / s0 * 32.f * 1.01f / (nrm * nrm * nn);
#pragma unroll
    for (int I = 0; I < TI; ++I) {
      f32x16 Xr[TJ];
      V::load_rows(Xr, I, Xm, tall, vec);
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 8; ++v)
            Xr[J][8 * kb + v] = s0 * ig * (float)Gh[I][J][kb][v] - coef * Xr[J][8 * kb + v];
      V::store_rows(Gm, Xr, I, tall, vec);
    }
  }
}

// Persistent fp16 VJP over two batches of matrices of the same D x E (in
// either orientation): matrices [0, na) from (Xa, Ga), then [na, na + nb)
// from (Xb, Gb), wave by wave.  One launch for both of a chunk's memories
// (the wide W1 and the tall W2 matrices) lets a wave go from its last
// matrix of the one straight to the other, without a launch boundary where
// the GPU drains.
template <int D, int E, int VA, int VB>
__global__ void __launch_bounds__(BT) __attribute__((amdgpu_waves_per_eu(1, 1)))
pe_vjp_wave_kernel(long long na, long long nb, int ns, int talla, const float* Xa, float* Ga, int tallb,
                   const float* Xb, float* Gb) {
  using V = VjpWave<D, E>;
  extern __shared__ __attribute__((aligned(16))) char smw[];
  _Float16* zs = reinterpret_cast<_Float16*>(smw) + wave_id() * V::HALVES;
  _Float16* gs = zs + V::ZH;
  f16x8* ckpt = reinterpret_cast<f16x8*>(gs + V::GH);
  const long long nwaves = (long long)gridDim.x * NWV, DE = (long long)D * E;
  for (long long mi = (long long)blockIdx.x * NWV + wave_id(); mi < na + nb; mi += nwaves) {
    if constexpr (VA == VB) {
      const bool a = mi < na;
      vjp_wave_one<D, E, VA>(a ? Xa + mi * DE : Xb + (mi - na) * DE, a ? Ga + mi * DE : Gb + (mi - na) * DE, ns,
                             a ? talla : tallb, zs, gs, ckpt);
    } else if (mi < na) {
      vjp_wave_one<D, E, VA>(Xa + mi * DE, Ga + mi * DE, ns, talla, zs, gs, ckpt);
    } else {
      vjp_wave_one<D, E, VB>(Xb + (mi - na) * DE, Gb + (mi - na) * DE, ns, tallb, zs, gs, ckpt);
    }
  }
}

template <int D, int E, int VA, int VB>
atlas_status launch_vjp_wave_mode(long long na, long long nb, int ns, int talla, const float* Xa, float* Ga,
                                  int tallb, const float* Xb, float* Gb, hipStream_t st) {
  const int bytes = VjpWave<D, E>::bytes();
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&pe_vjp_wave_kernel<D, E, VA, VB>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return fail_hip(e, "pe_vjp_wave shared-memory attribute");
    attr_set = true;
  }
  const long long grid = std::min<long long>((na + nb + NWV - 1) / NWV, VJPW_GRID);
  hipLaunchKernelGGL((pe_vjp_wave_kernel<D, E, VA, VB>), dim3((unsigned)grid), dim3(BT), bytes, st, na, nb, ns,
                     talla, Xa, Ga, tallb, Xb, Gb);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_vjp_wave launch");
}

// The load path for one orientation: tall inputs (rows of the D x E
// iterate strided in memory) 1, wide ones 2 at E = 128, else the scalar 0
// (also whenever a pointer is not 16-byte aligned).
template <int E>
int vjp_vec(int tall, const float* X, const float* G) {
  const bool al = reinterpret_cast<uintptr_t>(X) % 16 == 0 && reinterpret_cast<uintptr_t>(G) % 16 == 0;
  if (!al) return 0;
  if (tall) return 1;
  return E == 128 ? 2 : 0;
}

template <int D, int E>
atlas_status launch_vjp_wave(long long n, int ns, int tall, const float* X, float* G, hipStream_t st) {
  switch (vjp_vec<E>(tall, X, G)) {
    case 1: return launch_vjp_wave_mode<D, E, 1, 1>(n, 0, ns, tall, X, G, tall, X, G, st);
    case 2: return launch_vjp_wave_mode<D, E, 2, 2>(n, 0, ns, tall, X, G, tall, X, G, st);
    default: return launch_vjp_wave_mode<D, E, 0, 0>(n, 0, ns, tall, X, G, tall, X, G, st);
  }
}

// Both memories of a chunk in one launch: n wide D x E matrices (Xa, Ga)
// and n tall E x D ones (Xb, Gb).
template <int D, int E>
atlas_status launch_vjp_wave_both(long long n, int ns, const float* Xa, float* Ga, const float* Xb, float* Gb,
                                  hipStream_t st) {
  const int va = vjp_vec<E>(0, Xa, Ga), vb = vjp_vec<E>(1, Xb, Gb);
  if (va == 2 && vb == 1) return launch_vjp_wave_mode<D, E, 2, 1>(n, n, ns, 0, Xa, Ga, 1, Xb, Gb, st);
  if (va == 0 && vb == 1) return launch_vjp_wave_mode<D, E, 0, 1>(n, n, ns, 0, Xa, Ga, 1, Xb, Gb, st);
  if (va == 0 && vb == 0) return launch_vjp_wave_mode<D, E, 0, 0>(n, n, ns, 0, Xa, Ga, 1, Xb, Gb, st);
  atlas_status r = launch_vjp_wave<D, E>(n, ns, 0, Xa, Ga, st);
  return r ? r : launch_vjp_wave<D, E>(n, ns, 1, Xb, Gb, st);
}

// ---- Polar-Express VJP with fp16 operands, one matrix per pair of waves ---
// For D x 2EH matrices (64 x 256): a 64 x 256 fp32 iterate does not fit one
// wave next to the cotangent and the D x D products, so each wave of a pair
// holds one 128-column half (the iterate in fp32, the cotangent as scaled
// fp16 fragments, both exactly as VjpWave holds a whole 64 x 128 matrix) and
// the pair adds its partial D x D products (the Gram A = sum_h Z_h Z_h^T and
// Gs = sum_h (G_h Z_h^T + Z_h G_h^T)) through LDS in fp32: half 0 writes its
// partials, half 1 adds its own and writes the sums back, half 0 reads them,
// so both halves continue from bitwise-equal A and Gs (B and C are formed
// by both).  The columns' updates, the cotangent's scale, the checkpoint
// image and all loads and stores stay per half.  The exchange area is the
// pair's staging LDS: every exchange starts with a barrier (both halves are
// done reading their staged blocks) and ends with one (before anything is
// staged there again), and pairs past the last matrix run on zeros so that
// every wave reaches every barrier.
template <int D, int EH>
struct VjpPair {
  using V = VjpWave<D, EH>;
  using PT = typename V::PT;
  using M = ModeF16;
  using frag = f16x8;
  static constexpr int TI = D / 32, TJ = EH / 32, E = 2 * EH;
  static constexpr int SH = V::ZH + V::GH;                      // staging halves per wave
  static constexpr int CH = D * EH;                             // checkpoint halves per wave
  static constexpr int bytes() { return NWV * (SH + CH) * 2 + 64 * (int)sizeof(float); }
  static_assert(2 * SH * 2 >= 2 * D * D * (int)sizeof(float), "the pair's staging area holds A and Gs");

  // row block I of the half's columns of a D x E matrix (or of its transpose
  // when tall); vec 1: tall, 16-byte aligned; vec 2: not tall, 16-byte
  // aligned, tile J's lane c holding column EH half + 4c + J
  __device__ __forceinline__ static void load_rows(f32x16 (&T)[TJ], int I, const float* src, int tall, int vec,
                                                   int half) {
    const int c = lane_id() & 31, h = lane_id() >> 5;
    const float* p = src + PT::opaque(vec == 2 ? 4 * h * E + EH * half + 4 * c
                                              : tall ? (EH * half + c) * D + 4 * h : 4 * h * E + EH * half + c);
    if (vec == 2) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(p + (32 * I + 8 * (r / 4) + r % 4) * E);
#pragma unroll
        for (int J = 0; J < TJ; ++J) T[J][r] = v[J & 3];
      }
      return;
    }
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      if (vec) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(p + 32 * J * D + 32 * I + 8 * q);
#pragma unroll
          for (int u = 0; u < 4; ++u) T[J][4 * q + u] = v[u];
        }
      } else if (tall) {
#pragma unroll
        for (int r = 0; r < 16; ++r) T[J][r] = p[32 * J * D + 32 * I + 8 * (r / 4) + r % 4];
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) T[J][r] = p[(32 * I + 8 * (r / 4) + r % 4) * E + 32 * J];
      }
    }
  }
  __device__ __forceinline__ static void load(f32x16 (&T)[TI][TJ], const float* src, int tall, int vec, int half) {
#pragma unroll
    for (int I = 0; I < TI; ++I) load_rows(T[I], I, src, tall, vec, half);
  }
  __device__ __forceinline__ static void store(float* dst, const f32x16 (&T)[TJ], int I, int tall, int vec,
                                               int half) {
    const int c = lane_id() & 31, h = lane_id() >> 5;
    float* p = dst + PT::opaque(vec == 2 ? 4 * h * E + EH * half + 4 * c
                                        : tall ? (EH * half + c) * D + 4 * h : 4 * h * E + EH * half + c);
    if (vec == 2) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        *reinterpret_cast<f32x4*>(p + (32 * I + 8 * (r / 4) + r % 4) * E) =
            f32x4{T[0][r], T[1 & (TJ - 1)][r], T[2 & (TJ - 1)][r], T[3 & (TJ - 1)][r]};
      return;
    }
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      if (vec) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(p + 32 * J * D + 32 * I + 8 * q) =
              f32x4{T[J][4 * q], T[J][4 * q + 1], T[J][4 * q + 2], T[J][4 * q + 3]};
      } else if (tall) {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[32 * J * D + 32 * I + 8 * (r / 4) + r % 4] = T[J][r];
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[(32 * I + 8 * (r / 4) + r % 4) * E + 32 * J] = T[J][r];
      }
    }
  }

  // sum of the pair's partials of NM D x D matrices through xa (fp32 quads:
  // tile (I, I2) register quad q of lane l at ((m * TI + I) * TI + I2) * 4 + q) * WAVE + l)
  template <int NM>
  __device__ __forceinline__ static void exchange(f32x16 (&T)[NM][TI][TI], float* xa, int half) {
    f32x4* x4 = reinterpret_cast<f32x4*>(xa) + PT::opaque(lane_id());
    auto at = [&](int m, int I, int I2, int q) -> f32x4& { return x4[(((m * TI + I) * TI + I2) * 4 + q) * WAVE]; };
    __syncthreads();   // xa spans both halves' staging: the partner has finished reading its staged blocks
    if (half == 0) {
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              at(m, I, I2, q) = f32x4{T[m][I][I2][4 * q], T[m][I][I2][4 * q + 1], T[m][I][I2][4 * q + 2],
                                      T[m][I][I2][4 * q + 3]};
    }
    __syncthreads();
    if (half == 1) {
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 o = at(m, I, I2, q);
#pragma unroll
              for (int u = 0; u < 4; ++u) T[m][I][I2][4 * q + u] = o[u] + T[m][I][I2][4 * q + u];
              at(m, I, I2, q) = f32x4{T[m][I][I2][4 * q], T[m][I][I2][4 * q + 1], T[m][I][I2][4 * q + 2],
                                      T[m][I][I2][4 * q + 3]};
            }
    }
    __syncthreads();
    if (half == 0) {
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 o = at(m, I, I2, q);
#pragma unroll
              for (int u = 0; u < 4; ++u) T[m][I][I2][4 * q + u] = o[u];
            }
    }
    __syncthreads();   // xa is staging space again
  }
  // x_0 + x_1 in both halves (slot: two floats of the pair, reused only after a barrier)
  __device__ __forceinline__ static float exchange_scalar(float x, float* slot, int half) {
    if (lane_id() == 0) slot[half] = x;
    __syncthreads();
    const float sum = slot[0] + slot[1];
    __syncthreads();
    return sum;
  }

  __device__ __forceinline__ static void fwd_steps(f32x16 (&Z)[TI][TJ], int st0, int st1, _Float16* zs, float* xa,
                                                   int half) {
    for (int st = st0; st < st1; ++st) {
      f32x16 A[1][TI][TI];
      PT::gram(Z, A[0], zs);
      exchange<1>(A, xa, half);
      PT::apply_scaled(Z, A[0], st);
    }
  }

  // VjpWave::reverse_step for the half, with A and Gs summed over the pair
  __device__ __forceinline__ static void reverse_step(const f32x16 (&Z)[TI][TJ], frag (&Gh)[TI][TJ][2], float& sG,
                                                      int k, _Float16* zs, _Float16* gs, float* xa, int half,
                                                      float& dot, bool with_dot) {
    const float kap = kPEt[k][0], rho = kPEt[k][1];
    {
      float m = 0.f;
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 8; ++v) m = fmaxf(m, fabsf((float)Gh[I][J][kb][v]));
      const float r = pow2_scale(wave_max(m));
      if (r != 1.f) {
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int J = 0; J < TJ; ++J)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
              for (int v = 0; v < 8; ++v) Gh[I][J][kb][v] = (_Float16)((float)Gh[I][J][kb][v] * r);
        sG *= r;
      }
    }
    frag Zc[TI][TJ][2];
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Zc[I][J][kb] = M::from_c(Z[I][J], kb);
    f32x16 AS[2][TI][TI];   // A, then Gs (true units after the exchange)
    const int wo = PT::opaque(PT::wr_off()), ro = PT::opaque(PT::rd_off());
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      _Float16* zb = zs + (J & 1) * PT::BLOCK;
      _Float16* gb = gs + (J & 1) * PT::BLOCK;
      V::stage(Zc, J, zb, wo);
      V::stage(Gh, J, gb, wo);
      frag zt[TI][2], gt[TI][2];
      PT::read_block(zt, zb, ro);
      PT::read_block(gt, gb, ro);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int I2 = 0; I2 < TI; ++I2) {
            const bool first = J == 0 && kb == 0;
            AS[0][I][I2] = M::mma(zt[I][kb], zt[I2][kb], first ? zero16() : AS[0][I][I2]);
            AS[1][I][I2] = M::mma(gt[I][kb], zt[I2][kb], first ? zero16() : AS[1][I][I2]);
            AS[1][I][I2] = M::mma(zt[I][kb], gt[I2][kb], AS[1][I][I2]);
          }
    }
    {
      const float ig = 1.f / sG;
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int I2 = 0; I2 < TI; ++I2) AS[1][I][I2] = AS[1][I][I2] * ig;
    }
    exchange<2>(AS, xa, half);
    frag Af[TI][TI][2], Bf[TI][TI][2], Sf[TI][TI][2], Cf[TI][TI][2];
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Af[K][I][kb] = M::from_c(AS[0][K][I], kb);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) {
        AS[0][I][I2] = AS[0][I][I2] * kap;
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) AS[0][I][I2] = M::mma(Af[K][I][kb], Af[K][I2][kb], AS[0][I][I2]);
        const f32x16 t = AS[0][I][I2] * rho;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Bf[I][I2][kb] = M::from_c(t, kb);
      }
    const float s2 = pow2_scale(V::maxabs(AS[1]));
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        const f32x16 t = AS[1][K][I] * s2;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Sf[K][I][kb] = M::from_c(t, kb);
      }
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int I2 = 0; I2 < TI; ++I2) {
        AS[1][I][I2] = AS[1][I][I2] * (kap * s2);
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            AS[1][I][I2] = M::mma(Sf[K][I][kb], Af[K][I2][kb], AS[1][I][I2]);
            AS[1][I][I2] = M::mma(Af[K][I][kb], Sf[K][I2][kb], AS[1][I][I2]);
          }
        AS[1][I][I2] = AS[1][I][I2] * rho;
      }
    const float sc = pow2_scale(V::maxabs(AS[1]));
#pragma unroll
    for (int K = 0; K < TI; ++K)
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        const f32x16 t = AS[1][K][I] * sc;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Cf[K][I][kb] = M::from_c(t, kb);
      }
    // G_h <- G_h + B G_h + C Z_h (C scaled by s2 sc, G_h by sG)
    const float u2 = sG / (s2 * sc);
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      frag gf[TI][2];
#pragma unroll
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) gf[K][kb] = Gh[K][J][kb];
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        f32x16 a1, a2 = zero16();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 8; ++v) a1[8 * kb + v] = (float)gf[I][kb][v];
#pragma unroll
        for (int K = 0; K < TI; ++K)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            a1 = M::mma(Bf[K][I][kb], gf[K][kb], a1);
            a2 = M::mma(Cf[K][I][kb], Zc[K][J][kb], a2);
          }
        const f32x16 t = a1 + a2 * u2;
        if (with_dot) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 8; ++v) dot = fmaf(t[8 * kb + v], (float)Zc[I][J][kb][v], dot);
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) Gh[I][J][kb] = M::from_c(t, kb);
      }
    }
  }
};

template <int D, int EH, int VEC>
__global__ void __launch_bounds__(BT) __attribute__((amdgpu_waves_per_eu(1, 1)))
pe_vjp_pair_kernel(long long n, int ns, int tall, const float* X, float* G) {
  constexpr int vec = VEC;
  using P = VjpPair<D, EH>;
  using V = typename P::V;
  using M = ModeF16;
  using frag = f16x8;
  constexpr int TI = D / 32, TJ = EH / 32, E = 2 * EH;
  extern __shared__ __attribute__((aligned(16))) char smp[];
  const int wv = wave_id(), pair = wv >> 1, half = wv & 1;
  _Float16* zs = reinterpret_cast<_Float16*>(smp) + wv * P::SH;
  _Float16* gs = zs + V::ZH;
  float* xa = reinterpret_cast<float*>(reinterpret_cast<_Float16*>(smp) + 2 * pair * P::SH);   // the pair's staging
  frag* ckpt = reinterpret_cast<frag*>(reinterpret_cast<_Float16*>(smp) + NWV * P::SH + wv * P::CH);
  float* slot = reinterpret_cast<float*>(reinterpret_cast<_Float16*>(smp) + NWV * (P::SH + P::CH)) + 8 * pair;
  const int cp = (ns - 1) / 2;
  for (long long base = (long long)blockIdx.x * 2; base < n; base += (long long)gridDim.x * 2) {
    const long long mi = base + pair;
    const bool live = mi < n;   // a pair past the last matrix runs on zeros (every barrier is reached)
    const float* Xm = X + (live ? mi : 0) * D * E;
    float* Gm = G + (live ? mi : 0) * D * E;
    f32x16 Z[TI][TJ];
    if (live) P::load(Z, Xm, tall, vec, half);
    else
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J) Z[I][J] = zero16();
    const float nn = sqrtf(P::exchange_scalar(V::W::sumsq(Z), slot, half) + 1e-12f);
    const float nrm = nn * 1.01f + 1e-6f, s0 = 32.f / nrm;
    V::W::scale(Z, s0);
    for (int st = 0; st + 1 < ns; ++st) {
      if (st == cp) V::put_image(Z, ckpt);
      P::fwd_steps(Z, st, st + 1, zs, xa, half);
    }
    frag Gh[TI][TJ][2];
    float sG;
    {
      f32x16 Gb[TI][TJ];
      if (live) P::load(Gb, Gm, tall, vec, half);
      else
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int J = 0; J < TJ; ++J) Gb[I][J] = zero16();
      sG = pow2_scale(V::maxabs(Gb) * kPEtau[ns]);
      const float f = sG * kPEtau[ns];
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) Gh[I][J][kb] = M::from_c(Gb[I][J] * f, kb);
    }
    float dot = 0.f;
    for (int k = ns - 1; k >= 0; --k) {
      if (k < ns - 1) {
        if (k >= cp) {
          V::get_image(Z, ckpt);
          P::fwd_steps(Z, cp, k, zs, xa, half);
        } else {
          if (live) P::load(Z, Xm, tall, vec, half);
          V::W::scale(Z, s0);
          P::fwd_steps(Z, 0, k, zs, xa, half);
        }
      }
      P::reverse_step(Z, Gh, sG, k, zs, gs, xa, half, dot, k == 0);
    }
    const float ig = 1.f / sG;
    if (ns == 0) {
#pragma unroll
      for (int I = 0; I < TI; ++I)
#pragma unroll
        for (int J = 0; J < TJ; ++J)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 8; ++v) dot = fmaf((float)Gh[I][J][kb][v], Z[I][J][8 * kb + v], dot);
    }
    // <G_0, Z_0> over both halves (each half's dot in its own cotangent scale)
    const float tot = P::exchange_scalar(wave_sum(dot) * ig, slot, half);
    const float coef = tot / s0 * 32.f * 1.01f / (nrm * nrm * nn);
#pragma unroll
    for (int I = 0; I < TI; ++I) {
      f32x16 Xr[TJ];
      if (live) P::load_rows(Xr, I, Xm, tall, vec, half);
      else
#pragma unroll
        for (int J = 0; J < TJ; ++J) Xr[J] = zero16();
#pragma unroll
      for (int J = 0; J < TJ; ++J)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 8; ++v)
            Xr[J][8 * kb + v] = s0 * ig * (float)Gh[I][J][kb][v] - coef * Xr[J][8 * kb + v];
      if (live) P::store(Gm, Xr, I, tall, vec, half);
    }
  }
}

template <int D, int EH, int VEC>
atlas_status launch_vjp_pair_mode(long long n, int ns, int tall, const float* X, float* G, hipStream_t st) {
  const int bytes = VjpPair<D, EH>::bytes();
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&pe_vjp_pair_kernel<D, EH, VEC>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return fail_hip(e, "pe_vjp_pair shared-memory attribute");
    attr_set = true;
  }
  const long long grid = std::min<long long>((n + 1) / 2, VJPW_GRID);
  hipLaunchKernelGGL((pe_vjp_pair_kernel<D, EH, VEC>), dim3((unsigned)grid), dim3(BT), bytes, st, n, ns, tall, X, G);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_vjp_pair launch");
}

template <int D, int EH>
atlas_status launch_vjp_pair(long long n, int ns, int tall, const float* X, float* G, hipStream_t st) {
  const bool al = reinterpret_cast<uintptr_t>(X) % 16 == 0 && reinterpret_cast<uintptr_t>(G) % 16 == 0;
  if (al && tall) return launch_vjp_pair_mode<D, EH, 1>(n, ns, tall, X, G, st);
  if (al) return launch_vjp_pair_mode<D, EH, 2>(n, ns, tall, X, G, st);
  return launch_vjp_pair_mode<D, EH, 0>(n, ns, tall, X, G, st);
}

// dX for n matrices of d1 x d2 (X and the cotangent G, dX written over G),
// with fp32 or fp16 matrix-core operands.
atlas_status pe_vjp(long long n, int d1, int d2, int ns, const float* X, float* G, float* scratch, bool f16,
                    hipStream_t st) {
  const int tall = d1 > d2;
  const int D = tall ? d2 : d1, E = tall ? d1 : d2;
#define ATLAS_VJP_CASE(DD, EE)                                                          \
  if (D == DD && E == EE)                                                               \
    return f16 ? launch_vjp_wave<DD, EE>(n, ns, tall, X, G, st)                          \
               : launch_vjp<DD, EE>(n, ns, tall, X, G, scratch, st);
  ATLAS_VJP_CASE(32, 32)
  ATLAS_VJP_CASE(32, 64)
  ATLAS_VJP_CASE(32, 128)
  ATLAS_VJP_CASE(64, 64)
  ATLAS_VJP_CASE(64, 128)
#undef ATLAS_VJP_CASE
  if (D == 64 && E == 256)
    return f16 ? launch_vjp_pair<64, 128>(n, ns, tall, X, G, st) : launch_vjp<64, 256>(n, ns, tall, X, G, scratch, st);
  return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "Polar-Express VJP for %d x %d is not compiled", d1, d2);
}

// dX for both memories of a chunk: n D x E matrices (X0, G0) and n E x D
// ones (X1, G1); the fp16 wave kernel takes them in one launch.
atlas_status pe_vjp_both(long long n, int D, int E, int ns, const float* X0, float* G0, const float* X1, float* G1,
                         float* scratch, bool f16, hipStream_t st) {
  if (f16) {
#define ATLAS_VJP_BOTH(DD, EE) \
  if (D == DD && E == EE) return launch_vjp_wave_both<DD, EE>(n, ns, X0, G0, X1, G1, st);
    ATLAS_VJP_BOTH(32, 32)
    ATLAS_VJP_BOTH(32, 64)
    ATLAS_VJP_BOTH(32, 128)
    ATLAS_VJP_BOTH(64, 64)
    ATLAS_VJP_BOTH(64, 128)
#undef ATLAS_VJP_BOTH
  }
  atlas_status r = pe_vjp(n, D, E, ns, X0, G0, scratch, f16, st);
  return r ? r : pe_vjp(n, E, D, ns, X1, G1, scratch, f16, st);
}

size_t vjp_scratch_floats(int D, int E, int ns) {
  // the fp32 VJP's per-workgroup scratch (the fp16 VJP needs none)
  size_t f32 = (size_t)(ns > 1 ? ns - 1 : 1) * D * E;
  if (D == 64 && E == 256) f32 = VjpLds<64, 256>::scratch_floats(ns);
  return (size_t)VJP_GRID * f32;
}

// Shapes the backward is compiled for.
bool shape_ok(int D, int E, bool f16) {
  (void)f16;
  return (D == 32 && (E == 32 || E == 64 || E == 128)) || (D == 64 && (E == 64 || E == 128 || E == 256));
}

// Workspace of the backward.  The per-chunk buffers (the (cs, DE) matrices,
// the per-token vectors and the Omega window's last sum) come in two slots
// when there is more than one chunk: chunk c uses slot c % 2, so that the
// forward recompute of chunk c - 1 (on a second stream) overlaps the
// backward of chunk c.
struct Layout {
  long long BH, DE, cs, nc, NB, tok;
  int slots;
  size_t o_trace, o_mat, o_adj, o_tokv, o_carry, o_gfin, o_part, o_vjp, total;
  Layout(const atlas_scan_desc* d) {
    BH = (long long)d->B * d->H;
    DE = (long long)d->D * d->E;
    cs = d->chunk_size;
    nc = d->T / d->chunk_size;
    NB = DE / EBLK;
    tok = BH * cs;
    slots = nc > 1 ? 2 : 1;
    size_t o = 0;
    auto take = [&](size_t floats) { size_t r = o; o += (floats * sizeof(float) + 255) & ~size_t(255); return r; };
    o_trace = take((size_t)(nc > 1 ? nc - 1 : 0) * 4 * BH * DE);
    o_mat = take((size_t)slots * 6 * tok * DE);
    o_adj = take((size_t)slots * tok * (d->D + d->E) * (1 + NB));
    o_tokv = take((size_t)slots * tok * (9 * d->E + 2 * d->D));
    o_carry = take((size_t)6 * BH * DE);
    o_gfin = take((size_t)slots * 2 * BH * DE);
    o_part = take((size_t)nc * 6 * BH * NB * cs);   // per chunk
    o_vjp = take(d->compute == ATLAS_COMPUTE_F16 ? 4 : vjp_scratch_floats(d->D, d->E, d->ns_steps));
    total = o;
  }
};

atlas_status check_desc(const atlas_scan_desc* d) {
  if (!d) return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL descriptor");
  if (d->B < 1 || d->T < 1 || d->H < 1 || d->chunk_size < 1)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad sizes");
  if (!shape_ok(d->D, d->E, d->compute == ATLAS_COMPUTE_F16))
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE,
                "backward compiled for D 32 (E 32/64/128) and D 64 (E 64/128/256), got D %d E %d",
                d->D, d->E);
  if (d->chunk_size > BT) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "chunk_size %d > %d", d->chunk_size, BT);
  if (d->T % d->chunk_size) return fail(ATLAS_ERR_INVALID_ARGUMENT, "T %d is not a multiple of the chunk size", d->T);
  if (d->ns_steps < 0 || d->ns_steps > 5) return fail(ATLAS_ERR_INVALID_ARGUMENT, "ns_steps outside [0, 5]");
  if (d->io_dtype != ATLAS_DTYPE_F32 || d->gate_dtype != ATLAS_DTYPE_F32)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "the backward takes fp32 inputs");
  if (d->compute != ATLAS_COMPUTE_F32 && d->compute != ATLAS_COMPUTE_F16)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad compute mode %d", d->compute);
  // strides: 0 = dense, as in atlas_scan_fwd; anything else must be dense
  const long long HD = (long long)d->H * d->D;
  auto dense = [](long long s, long long want) { return s == 0 || s == want; };
  if (!dense(d->x_stride_h, d->D) || !dense(d->x_stride_t, HD) || !dense(d->x_stride_b, (long long)d->T * HD) ||
      !dense(d->g_stride_t, d->H) || !dense(d->g_stride_b, (long long)d->T * d->H))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "the backward takes dense (B, T, H, D) / (B, T, H) arrays");
  return ATLAS_OK;
}

bool misaligned16(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 15u); }

// ---- generic forward ------------------------------------------------------
// atlas_scan_fwd for the (D, E) the phase kernels are not built for (any D <=
// 64 and E <= 256 that are multiples of 4, E = 256 in fp32 included) and for
// chunk sizes outside theirs: per chunk, the chunk's rows of q, k, v and the
// gates are gathered into dense fp32 (padded rows as the reference pads),
// then the per-token kernels of the backward's recompute run (memory forward
// at the chunk-start weights, the Omega sums and S_t, Polar-Express of every
// S_t, W_t) and a read-out kernel writes y.  The state is updated in place.

// chunk rows of q, k, v (any dtype, strided) and of the gates -> dense fp32
__global__ void gather_chunk_kernel(const atlas_scan_desc d, int c0, const void* q, const void* k, const void* v,
                                    const void* al, const void* et, const void* th, const void* ga, float* qd,
                                    float* kd, float* vd, float* gd, int has_g) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const int cs = d.chunk_size, D = d.D, H = d.H;
  const long long nx = (long long)d.B * cs * H * D;
  const long long xsh = d.x_stride_h ? d.x_stride_h : D, xst = d.x_stride_t ? d.x_stride_t : (long long)H * D;
  const long long xsb = d.x_stride_b ? d.x_stride_b : (long long)d.T * H * D;
  const long long gst = d.g_stride_t ? d.g_stride_t : H, gsb = d.g_stride_b ? d.g_stride_b : (long long)d.T * H;
  if (i < nx) {
    const int dd = (int)(i % D), hh = (int)(i / D % H), t = (int)(i / ((long long)D * H) % cs);
    const int b = (int)(i / ((long long)D * H * cs));
    const int tt = c0 + t;
    float x = 0.f, y = 0.f, z = 0.f;
    if (tt < d.T) {
      const long long o = b * xsb + tt * xst + hh * xsh + dd;
      x = load_any(q, o, d.io_dtype);
      y = load_any(k, o, d.io_dtype);
      z = load_any(v, o, d.io_dtype);
    }
    qd[i] = x;
    kd[i] = y;
    vd[i] = z;
  }
  const long long ng = (long long)d.B * cs * H;
  if (i < ng) {
    const int hh = (int)(i % H), t = (int)(i / H % cs), b = (int)(i / ((long long)H * cs));
    const int tt = c0 + t;
    const bool in = tt < d.T;
    const long long o = b * gsb + tt * gst + hh;
    gd[i] = in ? load_any(al, o, d.gate_dtype) : 1.f;
    gd[ng + i] = in ? load_any(et, o, d.gate_dtype) : 0.f;
    gd[2 * ng + i] = in ? load_any(th, o, d.gate_dtype) : 0.f;
    gd[3 * ng + i] = (in && has_g) ? load_any(ga, o, d.gate_dtype) : 0.f;
  }
}

// y_t = q_t + W1_t gelu_tanh(W2_t q_t) per token (memory_layer.py:592-595)
__global__ void __launch_bounds__(BT) readout_fwd_kernel(BwdArgs a, const atlas_scan_desc d, int c0, void* y) {
  const int s = blockIdx.x / a.cs, t = blockIdx.x % a.cs, b = s / a.H, hh = s % a.H;
  const int D = a.D, E = a.E;
  if (c0 + t >= d.T) return;
  __shared__ float qv[128], gv[256];
  const long long xr = xrow(a, b, hh, t), tv = (long long)s * a.cs + t;
  const float* W1t = a.Wall[0] + tv * a.DE;   // [d][e]
  const float* W2t = a.Wall[1] + tv * a.DE;   // [e][d]
  for (int dd = threadIdx.x; dd < D; dd += BT) qv[dd] = a.q[xr + dd];
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += BT) {
    float hq = 0.f;
    for (int dd = 0; dd < D; ++dd) hq = fmaf(W2t[e * D + dd], qv[dd], hq);
    gv[e] = gelu_tanh(hq);
  }
  __syncthreads();
  const long long xsh = d.x_stride_h ? d.x_stride_h : D, xst = d.x_stride_t ? d.x_stride_t : (long long)a.H * D;
  const long long xsb = d.x_stride_b ? d.x_stride_b : (long long)d.T * a.H * D;
  for (int dd = threadIdx.x; dd < D; dd += BT) {
    float acc = 0.f;
    for (int e = 0; e < E; ++e) acc = fmaf(W1t[dd * E + e], gv[e], acc);
    store_any(y, b * xsb + (long long)(c0 + t) * xst + hh * xsh + dd, d.io_dtype, qv[dd] + acc);
  }
}

struct GenericLayout {
  long long BH, DE, cs, tok;
  size_t o_x, o_g, o_tokv, o_mat, total;
  explicit GenericLayout(const atlas_scan_desc* d) {
    BH = (long long)d->B * d->H;
    DE = (long long)d->D * d->E;
    cs = d->chunk_size;
    tok = BH * cs;
    size_t o = 0;
    auto take = [&](size_t floats) { size_t r = o; o += (floats * sizeof(float) + 255) & ~size_t(255); return r; };
    o_x = take((size_t)3 * tok * d->D);
    o_g = take((size_t)4 * tok);
    o_tokv = take((size_t)tok * (9 * d->E + 2 * d->D));
    o_mat = take((size_t)6 * tok * DE);
    total = o;
  }
};

}  // namespace

// Whether the generic forward covers the descriptor (its arguments already
// validated except for the shape).
bool generic_fwd_supported(const atlas_scan_desc* d) {
  return d && d->D >= 4 && d->D <= 128 && d->D % 4 == 0 && d->E >= 4 && d->E <= 256 && d->E % 4 == 0 &&
         d->chunk_size >= 1 && d->chunk_size <= 4096 && d->ns_steps >= 0 && d->ns_steps <= 5 && d->B >= 1 &&
         d->T >= 1 && d->H >= 1 && d->io_dtype >= 0 && d->io_dtype <= 2 && d->gate_dtype >= 0 &&
         d->gate_dtype <= 2 && (d->compute == ATLAS_COMPUTE_F32 || d->compute == ATLAS_COMPUTE_F16) &&
         d->omega_window >= 0;
}

size_t generic_fwd_workspace(const atlas_scan_desc* d) { return generic_fwd_supported(d) ? GenericLayout(d).total : 0; }

atlas_status generic_fwd(const atlas_scan_desc* d, const void* q, const void* k, const void* v, const void* alpha,
                         const void* eta, const void* theta, const void* gamma, float* W1, float* W2, float* S1,
                         float* S2, void* y, float* trace, void* workspace, hipStream_t st) {
  const GenericLayout Lo(d);
  char* ws = static_cast<char*>(workspace);
  const int D = d->D, E = d->E, cs = d->chunk_size;
  const long long BH = Lo.BH, DE = Lo.DE, tok = Lo.tok;
  BwdArgs a{};
  a.B = d->B; a.T = cs; a.H = d->H; a.D = D; a.E = E; a.cs = cs; a.ns = d->ns_steps;
  a.BH = (int)BH;
  a.NB = (int)((DE + EBLK - 1) / EBLK);
  a.win = (d->omega_window > 1 && gamma) ? 1 : 0;
  a.w = d->omega_window;
  a.DE = DE;
  a.scale = 2.f / (float)D;
  a.c0 = 0;   // the chunk's dense copies start at its first token
  float* xd = reinterpret_cast<float*>(ws + Lo.o_x);
  float* gd = reinterpret_cast<float*>(ws + Lo.o_g);
  a.q = xd; a.k = xd + tok * D; a.v = xd + 2 * tok * D;
  a.al = gd; a.et = gd + tok; a.th = gd + 2 * tok; a.ga = a.win ? gd + 3 * tok : nullptr;
  a.dy = nullptr;
  float* tv = reinterpret_cast<float*>(ws + Lo.o_tokv);
  a.h = tv; tv += tok * E;
  a.act = tv; tv += tok * E;
  a.w1e = tv; tv += tok * E;
  a.gp = tv; tv += tok * E;
  a.chain = tv; tv += tok * E;
  a.gq = tv; tv += tok * E;
  a.dhq = tv; tv += tok * E;
  a.dw1e = tv; tv += tok * E;
  a.dh = tv; tv += tok * E;
  a.err = tv; tv += tok * D;
  a.derr = tv;
  float* mat = reinterpret_cast<float*>(ws + Lo.o_mat);
  for (int m = 0; m < 2; ++m) {
    a.Sall[m] = mat + (0 + m) * tok * DE;
    a.Wall[m] = mat + (2 + m) * tok * DE;
    a.Pd[m] = mat + (4 + m) * tok * DE;
  }
  a.W1 = W1; a.W2 = W2; a.S1 = S1; a.S2 = S2;
  const int nc = (d->T + cs - 1) / cs;
  const long long nx = tok * D;
  const dim3 egrid((unsigned)(BH * a.NB), 2), tgrid((unsigned)tok);
  const size_t sb = (size_t)BH * DE * sizeof(float);
  for (int c = 0; c < nc; ++c) {
    if (trace) {
      float* dst = trace + (size_t)c * 4 * BH * DE;
      hipError_t e = hipMemcpyAsync(dst, W1, sb, hipMemcpyDeviceToDevice, st);
      if (e == hipSuccess) e = hipMemcpyAsync(dst + BH * DE, W2, sb, hipMemcpyDeviceToDevice, st);
      if (e == hipSuccess) e = hipMemcpyAsync(dst + 2 * BH * DE, S1, sb, hipMemcpyDeviceToDevice, st);
      if (e == hipSuccess) e = hipMemcpyAsync(dst + 3 * BH * DE, S2, sb, hipMemcpyDeviceToDevice, st);
      if (e != hipSuccess) return fail_hip(e, "state trace copy");
    }
    hipLaunchKernelGGL(gather_chunk_kernel, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, st, *d, c * cs, q, k,
                       v, alpha, eta, theta, gamma, xd, xd + tok * D, xd + 2 * tok * D, gd, gamma ? 1 : 0);
    hipLaunchKernelGGL(prep_bwd_kernel, tgrid, dim3(BT), 0, st, a);
    hipLaunchKernelGGL(mom_fwd_kernel, egrid, dim3(BT), 0, st, a, S1, S2);   // S updated in place
    atlas_status r;
    if ((r = atlas_pe_batched(tok, D, E, a.ns, ATLAS_PE_NORM_EPS, a.Sall[0], a.Pd[0], ATLAS_DTYPE_F32, d->compute,
                              st)))
      return r;
    if ((r = atlas_pe_batched(tok, E, D, a.ns, ATLAS_PE_NORM_EPS, a.Sall[1], a.Pd[1], ATLAS_DTYPE_F32, d->compute,
                              st)))
      return r;
    hipLaunchKernelGGL(mem_fwd_kernel, egrid, dim3(BT), 0, st, a, W1, W2);   // W updated in place
    hipLaunchKernelGGL(readout_fwd_kernel, tgrid, dim3(BT), 0, st, a, *d, c * cs, y);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail_hip(e, "generic scan launch");
  }
  return ATLAS_OK;
}

namespace {

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" size_t atlas_pe_vjp_workspace_size(int32_t d1, int32_t d2, int32_t ns_steps) {
  const int D = d1 < d2 ? d1 : d2, E = d1 < d2 ? d2 : d1;
  if (!shape_ok(D, E, true) || ns_steps < 0 || ns_steps > 5) return 0;
  // sized for the fp32 VJP (the fp16 VJPs need no scratch)
  return vjp_scratch_floats(D, E, ns_steps) * sizeof(float);
}

extern "C" atlas_status atlas_pe_vjp_batched(int64_t n, int32_t d1, int32_t d2, int32_t ns_steps, const float* X,
                                             float* G, int32_t compute, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  clear_error();
  if (n < 0) return fail(ATLAS_ERR_INVALID_ARGUMENT, "n < 0");
  if (ns_steps < 0 || ns_steps > 5) return fail(ATLAS_ERR_INVALID_ARGUMENT, "ns_steps outside [0, 5]");
  if (compute != ATLAS_COMPUTE_F32 && compute != ATLAS_COMPUTE_F16)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad compute mode %d", compute);
  const int D = d1 < d2 ? d1 : d2, E = d1 < d2 ? d2 : d1;
  if (!shape_ok(D, E, compute == ATLAS_COMPUTE_F16))
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "Polar-Express VJP for %d x %d is not compiled in this compute mode", d1,
                d2);
  if (n == 0) return ATLAS_OK;
  if (!X || !G) return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL pointer");
  const size_t need = atlas_pe_vjp_workspace_size(d1, d2, ns_steps);
  if (!workspace || workspace_bytes < need)
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, need);
  if (misaligned16(X) || misaligned16(G) || misaligned16(workspace))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "X, G and the workspace must be 16-byte aligned");
  return pe_vjp(n, d1, d2, ns_steps, X, G, static_cast<float*>(workspace), compute == ATLAS_COMPUTE_F16,
                static_cast<hipStream_t>(stream));
}

namespace atlas {
namespace {
// The backward's second stream on each device: default priority, created on
// first use and kept until the process ends.
std::mutex g_side_mu;
hipStream_t g_side[64] = {};
atlas_status side_stream(hipStream_t* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= 64) return fail(ATLAS_ERR_INVALID_ARGUMENT, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_side_mu);
  if (!g_side[dev]) {
    e = hipStreamCreateWithFlags(&g_side[dev], hipStreamNonBlocking);
    if (e != hipSuccess) {
      g_side[dev] = nullptr;
      return fail_hip(e, "scan_bwd side stream");
    }
  }
  *out = g_side[dev];
  return ATLAS_OK;
}
// Events of the two-stream backward (destroyed on return; a destroyed
// event's pending record and waits still complete).  Once `side` is set (the side stream
// has been given work), leaving the scope -- on success or on any error
// return -- records e[4] on the side stream and makes `main` wait for it, so
// that no side-stream kernel can still read or write the workspace, the trace
// or the inputs when the caller's stream moves on (and the caller frees them).
struct ScopedEvents {
  hipEvent_t e[5] = {};
  hipStream_t side = nullptr, main = nullptr;
  atlas_status create() {
    for (auto& x : e) {
      // (only ever waited on by the two streams of this device: a device-scope
      // release is enough, and skipping the system-scope fence measured 0.3 %
      // faster per training step)
      const hipError_t r = hipEventCreateWithFlags(&x, hipEventDisableTiming | hipEventDisableSystemFence);
      if (r != hipSuccess) return fail_hip(r, "scan_bwd event");
    }
    return ATLAS_OK;
  }
  ~ScopedEvents() {
    if (side && main && e[4] && hipEventRecord(e[4], side) == hipSuccess) (void)hipStreamWaitEvent(main, e[4], 0);
    for (auto x : e)
      if (x) (void)hipEventDestroy(x);
  }
};
}  // namespace
}  // namespace atlas

extern "C" size_t atlas_scan_bwd_workspace_size(const atlas_scan_desc* desc) {
  if (check_desc(desc) != ATLAS_OK) return 0;
  return Layout(desc).total;
}

extern "C" atlas_status atlas_scan_bwd(const atlas_scan_desc* desc, int32_t flags, const float* q, const float* k,
                                       const float* v, const float* alpha, const float* eta, const float* theta,
                                       const float* gamma, const float* W1, const float* W2, const float* S1,
                                       const float* S2, const float* state_trace, const float* dy,
                                       const float* dW1, const float* dW2,
                                       const float* dS1, const float* dS2, float* dq, float* dk, float* dv,
                                       float* dalpha, float* deta, float* dtheta, float* dgamma, float* dW1_0,
                                       float* dW2_0, float* dS1_0, float* dS2_0, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  clear_error();
  atlas_status s;
  if ((s = check_desc(desc))) return s;
  if (flags & ~(ATLAS_BWD_PE_STE | ATLAS_BWD_STOP_GRAD_CHUNKS))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "unknown flag bits 0x%x", flags);
  if (!q || !k || !v || !alpha || !eta || !theta || !W1 || !W2 || !S1 || !S2 || !dq || !dk || !dv || !dalpha ||
      !deta || !dtheta || !dW1_0 || !dW2_0 || !dS1_0 || !dS2_0)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL pointer (only gamma, dgamma, dy and the state cotangents may be NULL)");
  const Layout Lo(desc);
  if (!workspace || workspace_bytes < Lo.total)
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, Lo.total);
  for (const void* p : {(const void*)q, (const void*)k, (const void*)W1, (const void*)W2, (const void*)S1,
                        (const void*)S2, (const void*)dW1, (const void*)dW2, (const void*)dS1, (const void*)dS2,
                        (const void*)dW1_0, (const void*)dW2_0, (const void*)dS1_0, (const void*)dS2_0,
                        (const void*)workspace})
    if (misaligned16(p)) return fail(ATLAS_ERR_INVALID_ARGUMENT, "q, k, the states and their cotangents must be 16-byte aligned");
  if (misaligned16(state_trace)) return fail(ATLAS_ERR_INVALID_ARGUMENT, "state_trace must be 16-byte aligned");

  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int D = desc->D, E = desc->E, cs = desc->chunk_size, ns = desc->ns_steps;
  const bool f16 = desc->compute == ATLAS_COMPUTE_F16;   // 16-bit matrix-core operands for Polar-Express
  const long long BH = Lo.BH, DE = Lo.DE, tok = Lo.tok, nc = Lo.nc;

  BwdArgs base{};
  base.B = desc->B; base.T = desc->T; base.H = desc->H; base.D = D; base.E = E; base.cs = cs; base.ns = ns;
  base.BH = (int)BH; base.NB = (int)Lo.NB;
  base.win = (desc->omega_window > 1 && gamma) ? 1 : 0;
  base.w = desc->omega_window;
  base.DE = DE;
  base.scale = 2.f / (float)D;
  base.q = q; base.k = k; base.v = v; base.al = alpha; base.et = eta; base.th = theta; base.ga = gamma;
  base.dy = dy;
  float* trace = reinterpret_cast<float*>(ws + Lo.o_trace);
  float* carry = reinterpret_cast<float*>(ws + Lo.o_carry);
  base.cW[0] = carry; base.cW[1] = carry + BH * DE;
  base.cS[0] = carry + 2 * BH * DE; base.cS[1] = carry + 3 * BH * DE;
  base.tW[0] = carry + 4 * BH * DE; base.tW[1] = carry + 5 * BH * DE;
  float* part = reinterpret_cast<float*>(ws + Lo.o_part);
  const long long np = 2 * BH * Lo.NB * cs;
  base.pal = part; base.pth = part + np; base.pet = part + 2 * np;
  float* vjp_scr = reinterpret_cast<float*>(ws + Lo.o_vjp);
  base.dq = dq; base.dk = dk; base.dv = dv; base.dal = dalpha; base.det = deta; base.dth = dtheta; base.dga = dgamma;
  BwdArgs as[2] = {base, base};   // per slot: the per-chunk buffers
  for (int sl = 0; sl < Lo.slots; ++sl) {
    BwdArgs& a = as[sl];
    float* mat = reinterpret_cast<float*>(ws + Lo.o_mat) + (size_t)sl * 6 * tok * DE;
    for (int m = 0; m < 2; ++m) {
      a.Sall[m] = mat + (0 + m) * tok * DE;
      a.Wall[m] = mat + (2 + m) * tok * DE;
      a.Pd[m] = mat + (4 + m) * tok * DE;
    }
    float* adj = reinterpret_cast<float*>(ws + Lo.o_adj) + (size_t)sl * tok * (D + E) * (1 + Lo.NB);
    a.mrow[0] = adj;                       // (tok, D)
    a.mrow[1] = adj + tok * D;             // (tok, E)
    a.mcol[0] = adj + tok * (D + E);       // (tok, NB, E)
    a.mcol[1] = a.mcol[0] + tok * Lo.NB * E;   // (tok, NB, D)
    float* tv = reinterpret_cast<float*>(ws + Lo.o_tokv) + (size_t)sl * tok * (9 * E + 2 * D);
    a.h = tv; tv += tok * E;
    a.act = tv; tv += tok * E;
    a.w1e = tv; tv += tok * E;
    a.gp = tv; tv += tok * E;
    a.chain = tv; tv += tok * E;
    a.gq = tv; tv += tok * E;
    a.dhq = tv; tv += tok * E;
    a.dw1e = tv; tv += tok * E;
    a.dh = tv; tv += tok * E;
    a.err = tv; tv += tok * D;
    a.derr = tv;
    float* gf = reinterpret_cast<float*>(ws + Lo.o_gfin) + (size_t)sl * 2 * BH * DE;
    a.gfin[0] = gf; a.gfin[1] = gf + BH * DE;
  }

  const dim3 egrid((unsigned)(BH * Lo.NB), 2), tgrid((unsigned)tok);
  const size_t mom_lds = (size_t)2 * KT * NWV * (D > E ? D : E) * sizeof(float);
  auto state_of = [&](long long c, int i) -> const float* {
    if (state_trace) return state_trace + (c * 4 + i) * BH * DE;
    if (c == 0) return i == 0 ? W1 : i == 1 ? W2 : i == 2 ? S1 : S2;
    return trace + ((c - 1) * 4 + i) * BH * DE;
  };
  auto set_chunk = [&](BwdArgs& a, long long c) {
    a.c0 = (int)(c * cs);
    a.W1 = state_of(c, 0); a.W2 = state_of(c, 1); a.S1 = state_of(c, 2); a.S2 = state_of(c, 3);
  };
  // chunk c's forward recompute into its slot, on stream sx: parts 1 (the
  // per-token prep and the momentum scan) and/or 2 (Polar-Express and the
  // memory scan)
  auto chunk_forward = [&](long long c, bool keep_end, hipStream_t sx, int parts = 3) -> atlas_status {
    BwdArgs& a = as[c % Lo.slots];
    float* nxt = keep_end ? trace + c * 4 * BH * DE : nullptr;   // start state of chunk c + 1
    if (parts & 1) {
      set_chunk(a, c);
      hipLaunchKernelGGL(prep_bwd_kernel, tgrid, dim3(BT), 0, sx, a);
      hipLaunchKernelGGL(mom_fwd_kernel, egrid, dim3(BT), 0, sx, a, nxt ? nxt + 2 * BH * DE : nullptr,
                         nxt ? nxt + 3 * BH * DE : nullptr);
    }
    if (parts & 2) {
      atlas_status r;
      if (desc->compute == ATLAS_COMPUTE_F16) {
        if ((r = pe_recompute_both(tok, D, E, ns, a.Sall[0], a.Pd[0], a.Sall[1], a.Pd[1], sx))) return r;
      } else {
        if ((r = atlas_pe_batched(tok, D, E, ns, ATLAS_PE_NORM_EPS, a.Sall[0], a.Pd[0], ATLAS_DTYPE_F32,
                                  desc->compute, sx)))
          return r;
        if ((r = atlas_pe_batched(tok, E, D, ns, ATLAS_PE_NORM_EPS, a.Sall[1], a.Pd[1], ATLAS_DTYPE_F32,
                                  desc->compute, sx)))
          return r;
      }
      hipLaunchKernelGGL(mem_fwd_kernel, egrid, dim3(BT), 0, sx, a, nxt, nxt ? nxt + BH * DE : nullptr);
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? ATLAS_OK : fail_hip(e, "scan_bwd forward launch");
  };
  auto init = [&](float* dst, const float* src, hipStream_t sx) {
    if (src) {
      const hipError_t e = hipMemcpyAsync(dst, src, BH * DE * sizeof(float), hipMemcpyDeviceToDevice, sx);
      return e;
    }
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((BH * DE + 255) / 256)), dim3(256), 0, sx, dst, BH * DE, 0.f);
    return hipGetLastError();
  };

  // trace pass: start states of chunks 1 .. nc-1 (unless the forward kept them)
  for (long long c = 0; !state_trace && c + 1 < nc; ++c)
    if ((s = chunk_forward(c, true, st))) return s;
  // cotangents of the final state
  hipError_t e;
  if ((e = init(base.cW[0], dW1, st)) || (e = init(base.cW[1], dW2, st)) || (e = init(base.cS[0], dS1, st)) ||
      (e = init(base.cS[1], dS2, st)))
    return fail_hip(e, "scan_bwd cotangent init");
  const bool pe_ste = flags & ATLAS_BWD_PE_STE, stop = flags & ATLAS_BWD_STOP_GRAD_CHUNKS;
  // With two slots the forward recompute of chunk c - 1 (which depends only
  // on the chunk's start state) runs beside chunk c's backward, in two parts
  // placed around chunk c's Polar-Express VJP (which holds every CU, and which
  // contending work was measured to slow by a third): the per-token prep and
  // the momentum scan next to the read-out and memory scans backwards (part
  // 1), then Polar-Express on the matrix cores and the memory scan next to the
  // memory-bound momentum scan backwards and the per-token kernels (part 2).
  // The two streams swap roles every chunk: chunk c - 1's recompute runs on
  // the stream that then runs chunk c - 1's backward, which follows it in
  // stream order (the recompute's memory scan ends later than chunk c's
  // backward, and a cross-stream wait on it cost ~18 us per chunk).  Waits
  // across the streams, each for an event recorded earlier on the other one:
  //   - part 1 of chunk c - 1's recompute after chunk c's memory scan
  //     (event fe: the memory-bound parts do not overlap; its slot's previous
  //     user, chunk c + 1's backward, is earlier on the same stream);
  //   - chunk c's backward, from its memory scan backwards on (the first
  //     kernel to read the carry), after chunk c + 1's backward (event done);
  //   - part 2 of chunk c - 1's recompute after chunk c's VJP (event mid).
  const bool two = Lo.slots == 2;
  hipStream_t sb = st;
  ScopedEvents ev;
  hipEvent_t& fe = ev.e[0];
  hipEvent_t& mid = ev.e[2];
  hipEvent_t& done = ev.e[3];
  if (two) {
    if ((s = side_stream(&sb))) return s;
    if ((s = ev.create())) return s;
    // the side stream starts after the caller's work so far, and is joined
    // back into the caller's stream when this scope ends (ScopedEvents)
    if ((e = hipEventRecord(done, st)) || (e = hipStreamWaitEvent(sb, done, 0)))
      return fail_hip(e, "scan_bwd stream join");
    ev.side = sb;
    ev.main = st;
  }
  // the stream of chunk c's recompute and backward
  auto cstream = [&](long long c) -> hipStream_t { return (two && ((nc - 1 - c) & 1)) ? sb : st; };
  if (two) {
    if ((s = chunk_forward(nc - 1, false, st))) return s;
    if ((e = hipEventRecord(fe, st))) return fail_hip(e, "scan_bwd event record");
  }
  for (long long c = nc - 1; c >= 0; --c) {
    const int sl = (int)(c % Lo.slots);
    const hipStream_t sx = cstream(c), sy = c >= 1 ? cstream(c - 1) : sx;
    if (two) {
      if (c >= 1) {   // part 1 of chunk c - 1's recompute
        if ((e = hipStreamWaitEvent(sy, fe, 0))) return fail_hip(e, "scan_bwd stream wait");
        if ((s = chunk_forward(c - 1, false, sy, 1))) return s;
      }
    } else if ((s = chunk_forward(c, false, st))) {
      return s;
    }
    as[sl].pal = base.pal + c * 3 * np;   // this chunk's gate partial sums
    as[sl].pth = as[sl].pal + np;
    as[sl].pet = as[sl].pal + 2 * np;
    const BwdArgs& a = as[sl];
    hipLaunchKernelGGL(readout_bwd_kernel, tgrid, dim3(BT), 0, sx, a);
    if (two && c < nc - 1 && (e = hipStreamWaitEvent(sx, done, 0))) return fail_hip(e, "scan_bwd stream wait");
    hipLaunchKernelGGL(mem_bwd_kernel, egrid, dim3(BT), 0, sx, a);
    if ((e = hipGetLastError())) return fail_hip(e, "scan_bwd read-out launch");
    if (!pe_ste) {
      if ((s = pe_vjp_both(tok, D, E, ns, a.Sall[0], a.Pd[0], a.Sall[1], a.Pd[1], vjp_scr, f16, sx))) return s;
    }
    if (two && c >= 1) {   // part 2 of chunk c - 1's recompute
      if ((e = hipEventRecord(mid, sx)) || (e = hipStreamWaitEvent(sy, mid, 0)))
        return fail_hip(e, "scan_bwd stream wait");
      if ((s = chunk_forward(c - 1, false, sy, 2))) return s;
      if ((e = hipEventRecord(fe, sy))) return fail_hip(e, "scan_bwd event record");
    }
    hipLaunchKernelGGL(mom_bwd_kernel, egrid, dim3(BT), mom_lds, sx, a);
    hipLaunchKernelGGL(inner_bwd_kernel, tgrid, dim3(BT), 0, sx, a);
    hipLaunchKernelGGL(wgrad_kernel, dim3((unsigned)((BH * 2 * (D / 32) * (E / 32) + NWV - 1) / NWV)), dim3(BT), 0, sx,
                       a);
    if ((e = hipGetLastError())) return fail_hip(e, "scan_bwd backward launch");
    if (stop)   // the carry is detached at every chunk start (memory_layer.py:665)
      for (int i = 0; i < 2; ++i)
        if ((e = init(a.cW[i], nullptr, sx)) || (e = init(a.cS[i], nullptr, sx)))
          return fail_hip(e, "scan_bwd carry reset");
    if (two && (e = hipEventRecord(done, sx))) return fail_hip(e, "scan_bwd event record");
  }
  // the rest on the caller's stream, after chunk 0's backward
  if (two && cstream(0) != st && (e = hipStreamWaitEvent(st, done, 0))) return fail_hip(e, "scan_bwd stream wait");
  // d alpha, d theta, d eta of every chunk from the per-chunk partial sums
  for (long long c0 = 0; c0 < nc; c0 += 65535) {
    const long long m = std::min<long long>(nc - c0, 65535);
    hipLaunchKernelGGL(gate_grad_kernel, dim3((unsigned)BH, (unsigned)m), dim3(BT), 0, st, base, 3 * np, c0);
    if ((e = hipGetLastError())) return fail_hip(e, "scan_bwd gate gradient launch");
  }
  const size_t nb = BH * DE * sizeof(float);
  if ((e = hipMemcpyAsync(dW1_0, base.cW[0], nb, hipMemcpyDeviceToDevice, st)) ||
      (e = hipMemcpyAsync(dW2_0, base.cW[1], nb, hipMemcpyDeviceToDevice, st)) ||
      (e = hipMemcpyAsync(dS1_0, base.cS[0], nb, hipMemcpyDeviceToDevice, st)) ||
      (e = hipMemcpyAsync(dS2_0, base.cS[1], nb, hipMemcpyDeviceToDevice, st)))
    return fail_hip(e, "scan_bwd output copy");
  if (!base.win && dgamma) {   // no window: gamma does not enter the scan
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((desc->B * (long long)desc->T * desc->H + 255) / 256)), dim3(256),
                       0, st, dgamma, (long long)desc->B * desc->T * desc->H, 0.f);
    if ((e = hipGetLastError())) return fail_hip(e, "scan_bwd dgamma fill");
  }
  return ATLAS_OK;
}
