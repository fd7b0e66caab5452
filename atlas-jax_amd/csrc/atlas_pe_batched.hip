// atlas_pe_batched: Polar-Express on a batch of small independent matrices,
// one wavefront per matrix (atlas_jax/memory_layer.py:43-71,
// kernels/triton_pe.py:26-69; with ATLAS_PE_NORM_NO_EPS the normalisation of
// optim.py:69-83).
//
// A (d1 x d2) input is processed in its wide orientation: if d1 > d2 the
// kernel works on X^T (PE(X)^T = PE(X^T)), so the Gram is always the smaller
// (D x D) one.  The matrix is zero-padded to the compiled (D, E) tile shape;
// zero rows/columns stay zero through every Newton-Schulz step, so padding
// does not change the result.  Wide sides of 129..256 are split over a pair
// of waves (128 columns each, the Gram summed through LDS).  Short sides of
// 65..128 run on a workgroup of eight waves per matrix (pe_wg_kernel, fp32
// operands).
#include <hip/hip_runtime.h>

#include "atlas_pe.hpp"
#include "atlas_scan.h"
#include "atlas_status.hpp"

namespace atlas {
namespace {

template <class M, int D, int E>
__global__ void __launch_bounds__(256)
pe_batched_kernel(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype) {
  constexpr int TI = D / 32, TJ = E / 32;
  __shared__ __attribute__((aligned(16))) typename M::elem scr_all[4 * Scr<M>::template elems<D>()];
  const long long mat = (long long)blockIdx.x * 4 + wave_id();
  if (mat >= n) return;
  typename M::elem* scr = scr_all + wave_id() * Scr<M>::template elems<D>();
  const int c = lane_id() & 31, h = lane_id() >> 5;
  const bool tall = d1 > d2;
  const int rows = tall ? d2 : d1, cols = tall ? d1 : d2;   // wide orientation
  const long long base = mat * (long long)d1 * d2;
  f32x16 Xr[TI][TJ];
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * I + crow(r, h), j = 32 * J + c;   // (row, col) of the wide form
        float v = 0.f;
        if (i < rows && j < cols) v = load_any(X, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype);
        Xr[I][J][r] = v;
      }
  polar_express_wave<M, D, E>(Xr, ns, eps, scr);
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * I + crow(r, h), j = 32 * J + c;
        if (i < rows && j < cols)
          store_any(Y, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype, Xr[I][J][r]);
      }
}

// fp16 operands, wide side <= 128: the scan's own Polar-Express
// (polar_express_wave_t: Gram operands transposed through a per-wave LDS
// staging area, iterate carried scaled), one wave per matrix.  With `vec` set
// (tall input whose short side is D, buffers aligned) the transposed layout
// is read and written as runs of 4 along the short side, which is what the
// C layout gives each lane; otherwise element by element.  FAST >= 0: fp32
// input and output with vec = FAST fixed at compile time (the backward's
// recompute); a kernel that keeps every dtype and load path spills.
template <int D, int E, int FAST>
__device__ __forceinline__ void pe_wave_t_one(long long mat, long long n, int d1, int d2, int ns, float eps,
                                              const void* X, void* Y, int dtype_, int vec_, _Float16* xs) {
  const int dtype = FAST >= 0 ? 0 : dtype_, vec = FAST >= 0 ? FAST : vec_;
  using PT = PEWaveT<D, E>;
  constexpr int TI = D / 32, TJ = E / 32;
  if (mat >= n) return;   // no workgroup barrier below
  const int c = lane_id() & 31, h = lane_id() >> 5;
  const bool tall = d1 > d2;
  const int rows = tall ? d2 : d1, cols = tall ? d1 : d2;
  const long long base = mat * (long long)d1 * d2;
  f32x16 Xr[TI][TJ];
  // vec 2 (wide input of exactly D x 128 floats, aligned): tile J's lane c
  // holds column 4c + J (Polar-Express is invariant under a common
  // permutation of the columns), one 16-byte load per row for four tiles
  const bool wide4 = TJ == 4 && vec == 2;
  if (wide4) {
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(X) + base +
                                                         (long long)(32 * I + crow(r, h)) * E + 4 * c);
#pragma unroll
        for (int J = 0; J < TJ; ++J) Xr[I][J][r] = v[J & 3];
      }
  }
#pragma unroll
  for (int I = 0; I < TI && !wide4; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      const int j = 32 * J + c;
      if (vec == 1) {   // rows crow(4q + u, h) = 8q + 4h + u of column j: X^T[j][..] contiguous
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = j < cols ? load4_any(X, base + (long long)j * d2 + 32 * I + 8 * q + 4 * h, dtype)
                                   : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = 0; u < 4; ++u) Xr[I][J][4 * q + u] = v[u];
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = 32 * I + crow(r, h);
          float v = 0.f;
          if (i < rows && j < cols) v = load_any(X, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype);
          Xr[I][J][r] = v;
        }
      }
    }
  const float ps = polar_express_wave_t<D, E>(Xr, ns, eps, xs);
  if (wide4) {
    // the lane's offset through opaque(): formed here rather than 32 row
    // addresses kept (spilled) across Polar-Express
    float* yl = static_cast<float*>(Y) + base + PT::opaque(4 * h * E + 4 * c);
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        *reinterpret_cast<f32x4*>(yl + (32 * I + 8 * (r / 4) + r % 4) * E) =
            f32x4{Xr[I][0][r] * ps, Xr[I][1 & (TJ - 1)][r] * ps, Xr[I][2 & (TJ - 1)][r] * ps,
                  Xr[I][3 & (TJ - 1)][r] * ps};
    return;
  }
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J) {
      const int j = 32 * J + c;
      if (vec == 1) {
        if (j < cols) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            store4_any(Y, base + (long long)j * d2 + 32 * I + 8 * q + 4 * h, dtype,
                       f32x4{Xr[I][J][4 * q] * ps, Xr[I][J][4 * q + 1] * ps, Xr[I][J][4 * q + 2] * ps,
                             Xr[I][J][4 * q + 3] * ps});
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = 32 * I + crow(r, h);
          if (i < rows && j < cols)
            store_any(Y, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype, Xr[I][J][r] * ps);
        }
      }
    }
}

template <int D, int E, int FAST = -1>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
pe_wave_t_kernel(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype_, int vec_) {
  __shared__ __attribute__((aligned(16))) _Float16 xs_all[4 * PEWaveT<D, E>::ELEMS];
  pe_wave_t_one<D, E, FAST>((long long)blockIdx.x * 4 + wave_id(), n, d1, d2, ns, eps, X, Y, dtype_, vec_,
                            xs_all + wave_id() * PEWaveT<D, E>::ELEMS);
}

// The backward's recompute of both memories in one launch (fp32 in and out):
// blocks [0, ceil(n / 4)) take the n wide D x E matrices (Xa -> Ya, load path
// FA), the rest the n tall E x D ones (Xb -> Yb, load path FB), so that the
// second batch starts on every CU the first one frees.
template <int D, int E, int FA, int FB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
pe_wave_t_both_kernel(long long n, int ns, float eps, const float* Xa, float* Ya, const float* Xb, float* Yb) {
  __shared__ __attribute__((aligned(16))) _Float16 xs_all[4 * PEWaveT<D, E>::ELEMS];
  _Float16* xs = xs_all + wave_id() * PEWaveT<D, E>::ELEMS;
  const long long ba = (n + 3) / 4;
  if (blockIdx.x < ba)
    pe_wave_t_one<D, E, FA>((long long)blockIdx.x * 4 + wave_id(), n, D, E, ns, eps, Xa, Ya, 0, FA, xs);
  else
    pe_wave_t_one<D, E, FB>((long long)(blockIdx.x - ba) * 4 + wave_id(), n, E, D, ns, eps, Xb, Yb, 0, FB, xs);
}

// Two waves per matrix: wave 2p+half holds columns [128 half, 128 half + 128)
// of matrix 2 blockIdx + p (wide orientation).  Workgroups past the last
// matrix still run every step on zeros so that all barriers are reached.
template <class M, int D>
__global__ void __launch_bounds__(256)
pe_pair_kernel(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype) {
  constexpr int EH = 128, TI = D / 32, TJ = EH / 32;
  __shared__ __attribute__((aligned(16))) typename M::elem scr_all[4 * Scr<M>::template elems<D>()];
  __shared__ float xch[4][D * D];
  const int wv = wave_id(), pair = wv >> 1, half = wv & 1;
  const long long mat = (long long)blockIdx.x * 2 + pair;
  const bool live = mat < n;
  typename M::elem* scr = scr_all + wv * Scr<M>::template elems<D>();
  const int c = lane_id() & 31, h = lane_id() >> 5;
  const bool tall = d1 > d2;
  const int rows = tall ? d2 : d1, cols = tall ? d1 : d2;
  const long long base = (live ? mat : 0) * (long long)d1 * d2;
  f32x16 Xr[TI][TJ];
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * I + crow(r, h), j = EH * half + 32 * J + c;
        float v = 0.f;
        if (live && i < rows && j < cols)
          v = load_any(X, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype);
        Xr[I][J][r] = v;
      }
  // fp16: Gram operands transposed on the matrix cores (no staging area),
  // result = X * ps
  const float ps = polar_express_pair<M, D, EH>(Xr, ns, eps, sizeof(typename M::elem) == 2 ? nullptr : scr,
                                                xch[wv], xch[wv ^ 1], half);
  if (!live) return;
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int J = 0; J < TJ; ++J)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * I + crow(r, h), j = EH * half + 32 * J + c;
        if (i < rows && j < cols)
          store_any(Y, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype, Xr[I][J][r] * ps);
      }
}

// One workgroup of eight waves per matrix whose short side is 65..128 (TI =
// 3 or 4 row tiles of 32; long side <= 256), fp32 matrix-core operands in
// either compute mode.  The iterate X (wide orientation, zero-padded to TI x
// 32 rows and whole 32-column blocks) is held in registers as C-layout tiles,
// column block J by wave J.  Per Newton-Schulz step:
//   Gram  G = X X^T: the column blocks are staged in LDS one at a time (fp32
//         rows d, double buffered) and every wave accumulates its own tiles
//         of G (tile t = wave + 8q) over all blocks;
//   B     = b G + c G^2 from G in LDS (each wave its own tiles), written back
//         over G once every wave has read it;
//   X     <- a X + B X for the wave's column block, B from LDS.
// Every sum has a fixed order (bitwise reproducible).  LDS: two staging
// blocks (DP x 33 floats) and G/B (DP x (DP + 1) floats), at most 100 KiB.
template <int TI>
struct PEWg {
  static constexpr int NWG = 8;
  static constexpr int DP = 32 * TI;
  static constexpr int SS = 33;                 // staging row stride (floats)
  static constexpr int GS = DP + 1;             // G/B row stride (floats)
  static constexpr int NT = (TI * TI + NWG - 1) / NWG;
  static constexpr size_t lds_bytes() { return (size_t)(2 * DP * SS + DP * GS + NWG) * sizeof(float); }
};

template <int TI>
__global__ void __launch_bounds__(512)
pe_wg_kernel(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype) {
  using W = PEWg<TI>;
  using M = ModeF32;
  constexpr int DP = W::DP, SS = W::SS, GS = W::GS, NT = W::NT, NWG = W::NWG;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* stg = lds;                   // [2][DP][SS]
  float* gm = lds + 2 * DP * SS;      // [DP][GS]
  float* red = gm + DP * GS;          // [NWG]
  const long long mat = blockIdx.x;
  const int wv = wave_id(), lane = lane_id(), c = lane & 31, h = lane >> 5;
  const bool tall = d1 > d2;
  const int rows = tall ? d2 : d1, cols = tall ? d1 : d2;   // wide orientation
  const int NJ = (cols + 31) / 32;                          // <= NWG
  const bool own = wv < NJ;
  const long long base = mat * (long long)d1 * d2;
  f32x16 Xr[TI];
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * I + crow(r, h), j = 32 * wv + c;
      float v = 0.f;
      if (own && i < rows && j < cols) v = load_any(X, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype);
      Xr[I][r] = v;
    }
  {
    float ss = 0.f;
#pragma unroll
    for (int I = 0; I < TI; ++I)
#pragma unroll
      for (int r = 0; r < 16; ++r) ss += Xr[I][r] * Xr[I][r];
    ss = wave_sum(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NWG; ++w) tot += red[w];
    const float inv = 1.f / (sqrtf(tot + eps) * 1.01f + 1e-6f);
#pragma unroll
    for (int I = 0; I < TI; ++I) Xr[I] *= inv;
  }
  for (int st = 0; st < ns; ++st) {
    const float pa = kPE[st][0], pb = kPE[st][1], pc = kPE[st][2];
    f32x16 G[NT];
#pragma unroll
    for (int q = 0; q < NT; ++q) G[q] = zero16();
    // ---- Gram over the staged column blocks
    for (int J = 0; J < NJ; ++J) {
      float* buf = stg + (J & 1) * DP * SS;
      if (wv == J) {
#pragma unroll
        for (int I = 0; I < TI; ++I)
#pragma unroll
          for (int r = 0; r < 16; ++r) buf[(32 * I + crow(r, h)) * SS + c] = Xr[I][r];
      }
      __syncthreads();   // the block is staged; the reads of this buffer two blocks ago are done
#pragma unroll
      for (int q = 0; q < NT; ++q) {
        const int t = wv + NWG * q;
        if (t >= TI * TI) break;
        const int I = t / TI, I2 = t % TI;
        const float* ra = buf + (32 * I + c) * SS;
        const float* rb = buf + (32 * I2 + c) * SS;
#pragma unroll
        for (int kb = 0; kb < 16; ++kb) G[q] = M::mma(M::ld_contig(ra, kb, h), M::ld_contig(rb, kb, h), G[q]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // ---- B = b G + c G^2
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const int t = wv + NWG * q;
      if (t >= TI * TI) break;
      const int I = t / TI, I2 = t % TI;
#pragma unroll
      for (int r = 0; r < 16; ++r) gm[(32 * I + crow(r, h)) * GS + 32 * I2 + c] = G[q][r];
    }
    __syncthreads();
    f32x16 Bt[NT];
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const int t = wv + NWG * q;
      if (t >= TI * TI) break;
      const int I = t / TI, I2 = t % TI;
      f32x16 acc = zero16();
#pragma unroll 1
      for (int K = 0; K < TI; ++K)
#pragma unroll
        for (int kb = 0; kb < 16; ++kb) {
          // A: G[32I + m][32K + k]; B: G[32K + k][32I2 + n] (k = 2kb + h)
          const float a = gm[(32 * I + c) * GS + 32 * K + 2 * kb + h];
          const float b = gm[(32 * K + 2 * kb + h) * GS + 32 * I2 + c];
          acc = M::mma(a, b, acc);
        }
      Bt[q] = pb * G[q] + pc * acc;
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();   // every wave has read G
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const int t = wv + NWG * q;
      if (t >= TI * TI) break;
      const int I = t / TI, I2 = t % TI;
#pragma unroll
      for (int r = 0; r < 16; ++r) gm[(32 * I + crow(r, h)) * GS + 32 * I2 + c] = Bt[q][r];
    }
    __syncthreads();
    // ---- X <- a X + B X for this wave's column block (the next step's first
    // barrier orders these reads of B before G overwrites it)
    if (own) {
      f32x16 Xn[TI];
#pragma unroll
      for (int I = 0; I < TI; ++I) {
        Xn[I] = pa * Xr[I];
#pragma unroll
        for (int K = 0; K < TI; ++K) {
#pragma unroll
          for (int kb = 0; kb < 16; ++kb)
            Xn[I] = M::mma(M::ld_cslot(gm + (32 * I + c) * GS + 32 * K, kb, h), M::from_c(Xr[K], kb), Xn[I]);
          __builtin_amdgcn_sched_barrier(0);   // keeps the B loads of later blocks from being hoisted (registers)
        }
      }
#pragma unroll
      for (int I = 0; I < TI; ++I) Xr[I] = Xn[I];
    }
  }
  if (!own) return;
#pragma unroll
  for (int I = 0; I < TI; ++I)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * I + crow(r, h), j = 32 * wv + c;
      if (i < rows && j < cols)
        store_any(Y, base + (tall ? (long long)j * d2 + i : (long long)i * d2 + j), dtype, Xr[I][r]);
    }
}

template <int TI>
atlas_status launch_wg(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype,
                       hipStream_t st) {
  if (n > 0x7fffffffLL) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "n too large for the workgroup kernel");
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(pe_wg_kernel<TI>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int)PEWg<TI>::lds_bytes());
  if (attr != hipSuccess) return fail_hip(attr, "pe_wg attribute");
  hipLaunchKernelGGL((pe_wg_kernel<TI>), dim3((unsigned)n), dim3(512), PEWg<TI>::lds_bytes(), st, n, d1, d2, ns, eps,
                     X, Y, dtype);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_batched launch");
}

template <class M, int D>
atlas_status launch_pair(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype,
                         hipStream_t st) {
  const long long blocks = (n + 1) / 2;
  hipLaunchKernelGGL((pe_pair_kernel<M, D>), dim3((unsigned)blocks), dim3(256), 0, st, n, d1, d2, ns, eps, X, Y,
                     dtype);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_batched launch");
}

template <class M, int D, int E>
atlas_status launch(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype,
                    hipStream_t st) {
  const long long blocks = (n + 3) / 4;
  hipLaunchKernelGGL((pe_batched_kernel<M, D, E>), dim3((unsigned)blocks), dim3(256), 0, st, n, d1, d2, ns, eps, X,
                     Y, dtype);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_batched launch");
}

template <int D, int E>
atlas_status launch_t(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype,
                      hipStream_t st) {
  const long long blocks = (n + 3) / 4;
  const size_t align = dtype == 0 ? 16 : 8;
  const bool al = reinterpret_cast<uintptr_t>(X) % align == 0 && reinterpret_cast<uintptr_t>(Y) % align == 0;
  const int vec = !al ? 0 : (d1 > d2 && d2 == D) ? 1 : (d1 == D && d2 == E && E == 128 && dtype == 0) ? 2 : 0;
  if (dtype == 0 && vec == 1)
    hipLaunchKernelGGL((pe_wave_t_kernel<D, E, 1>), dim3((unsigned)blocks), dim3(256), 0, st, n, d1, d2, ns, eps, X, Y,
                       dtype, vec);
  else if (dtype == 0 && vec == 2)
    hipLaunchKernelGGL((pe_wave_t_kernel<D, E, 2>), dim3((unsigned)blocks), dim3(256), 0, st, n, d1, d2, ns, eps, X, Y,
                       dtype, vec);
  else
    hipLaunchKernelGGL((pe_wave_t_kernel<D, E>), dim3((unsigned)blocks), dim3(256), 0, st, n, d1, d2, ns, eps, X, Y,
                       dtype, vec);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_batched launch");
}

template <class M>
atlas_status dispatch(long long n, int d1, int d2, int ns, float eps, const void* X, void* Y, int dtype,
                      hipStream_t st) {
  const int rows = d1 < d2 ? d1 : d2, cols = d1 < d2 ? d2 : d1;
  if (rows > 64) return rows <= 96 ? launch_wg<3>(n, d1, d2, ns, eps, X, Y, dtype, st)
                                   : launch_wg<4>(n, d1, d2, ns, eps, X, Y, dtype, st);
  const int D = rows <= 32 ? 32 : 64;
  if (cols > 128) return D == 32 ? launch_pair<M, 32>(n, d1, d2, ns, eps, X, Y, dtype, st)
                                 : launch_pair<M, 64>(n, d1, d2, ns, eps, X, Y, dtype, st);
  const int E = cols <= 32 ? 32 : (cols <= 64 ? 64 : 128);
  if constexpr (sizeof(typename M::elem) == 2) {
    if (D == 32 && E == 32) return launch_t<32, 32>(n, d1, d2, ns, eps, X, Y, dtype, st);
    if (D == 32 && E == 64) return launch_t<32, 64>(n, d1, d2, ns, eps, X, Y, dtype, st);
    if (D == 32 && E == 128) return launch_t<32, 128>(n, d1, d2, ns, eps, X, Y, dtype, st);
    if (D == 64 && E == 64) return launch_t<64, 64>(n, d1, d2, ns, eps, X, Y, dtype, st);
    return launch_t<64, 128>(n, d1, d2, ns, eps, X, Y, dtype, st);
  }
  if (D == 32 && E == 32) return launch<M, 32, 32>(n, d1, d2, ns, eps, X, Y, dtype, st);
  if (D == 32 && E == 64) return launch<M, 32, 64>(n, d1, d2, ns, eps, X, Y, dtype, st);
  if (D == 32 && E == 128) return launch<M, 32, 128>(n, d1, d2, ns, eps, X, Y, dtype, st);
  if (D == 64 && E == 64) return launch<M, 64, 64>(n, d1, d2, ns, eps, X, Y, dtype, st);
  return launch<M, 64, 128>(n, d1, d2, ns, eps, X, Y, dtype, st);
}

}  // namespace

// fp16 Polar-Express of the backward's recompute for both memories of a
// chunk: n D x E matrices (Xa -> Ya) and n E x D ones (Xb -> Yb), fp32, in one
// launch when the one-wave kernel covers the shape and the buffers are
// 16-byte aligned; otherwise through atlas_pe_batched, one call per batch.
atlas_status pe_recompute_both(long long n, int D, int E, int ns, const float* Xa, float* Ya, const float* Xb,
                               float* Yb, hipStream_t st) {
  const bool al = ((reinterpret_cast<uintptr_t>(Xa) | reinterpret_cast<uintptr_t>(Ya) |
                    reinterpret_cast<uintptr_t>(Xb) | reinterpret_cast<uintptr_t>(Yb)) & 15) == 0;
  if (n > 0 && al && D == 64 && E == 128) {
    hipLaunchKernelGGL((pe_wave_t_both_kernel<64, 128, 2, 1>), dim3((unsigned)(2 * ((n + 3) / 4))), dim3(256), 0, st,
                       n, ns, 1e-12f, Xa, Ya, Xb, Yb);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? ATLAS_OK : fail_hip(e, "pe_batched launch");
  }
  atlas_status r = atlas_pe_batched(n, D, E, ns, ATLAS_PE_NORM_EPS, Xa, Ya, ATLAS_DTYPE_F32, ATLAS_COMPUTE_F16, st);
  return r ? r : atlas_pe_batched(n, E, D, ns, ATLAS_PE_NORM_EPS, Xb, Yb, ATLAS_DTYPE_F32, ATLAS_COMPUTE_F16, st);
}

}  // namespace atlas

using namespace atlas;

extern "C" atlas_status atlas_pe_batched(int64_t n, int32_t d1, int32_t d2, int32_t ns_steps, int32_t norm_mode,
                                         const void* X, void* Y, int32_t dtype, int32_t compute, void* stream) {
  clear_error();
  if (n < 0 || d1 < 1 || d2 < 1) return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad sizes n=%lld d1=%d d2=%d", (long long)n, d1, d2);
  if (n == 0) return ATLAS_OK;
  if (!X || !Y) return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL X or Y");
  if (ns_steps < 0 || ns_steps > 5) return fail(ATLAS_ERR_INVALID_ARGUMENT, "ns_steps %d outside [0, 5]", ns_steps);
  if (norm_mode != ATLAS_PE_NORM_EPS && norm_mode != ATLAS_PE_NORM_NO_EPS)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad norm_mode %d", norm_mode);
  if (dtype < 0 || dtype > 2) return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad dtype %d", dtype);
  const int rows = d1 < d2 ? d1 : d2, cols = d1 < d2 ? d2 : d1;
  if (rows > 128 || cols > 256)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "matrix %dx%d: the kernels need min dim <= 128 and max dim <= 256",
                d1, d2);
  if (n > (1LL << 33)) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "n too large");
  const float eps = norm_mode == ATLAS_PE_NORM_EPS ? 1e-12f : 0.f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (compute == ATLAS_COMPUTE_F16) return dispatch<ModeF16>(n, d1, d2, ns_steps, eps, X, Y, dtype, st);
  if (compute == ATLAS_COMPUTE_F32) return dispatch<ModeF32>(n, d1, d2, ns_steps, eps, X, Y, dtype, st);
  return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad compute mode %d", compute);
}
