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

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" atlas_status atlas_swa_fwd(int32_t B, int32_t T, int32_t H, int32_t D, int32_t window,
                                      const void* q, const void* k, const void* v, void* out,
                                      int64_t stride_b, int64_t stride_t, int64_t stride_h, int32_t io_dtype,
                                      const float* cos_tab, const float* sin_tab, void* stream) {
  clear_error();
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
  SwaArgs a;
  a.B = B; a.T = T; a.H = H; a.window = window; a.io_dtype = io_dtype;
  a.sb = stride_b; a.st = stride_t; a.sh = stride_h;
  a.q = q; a.k = k; a.v = v; a.out = out;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab;
  a.scale = 1.f / sqrtf((float)D);
  hipLaunchKernelGGL(swa_fwd_kernel, dim3((unsigned)(B * H * nqb)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "swa launch");
}
