// Memory-layer prologue after the input projections (atlas_jax/memory_layer.py
// :606-633): causal depthwise convolutions of q/k/v (ShortConv, :303-329),
// RMS norm (:211-216) and the polynomial feature map (:459-466) with the
// q/k asymmetry (q: norm then map; k: map then norm), and the sigmoid gates
// (eta times max_lr).  One wave per (b, t, h) token-head: lane l owns
// channels h*D + l and h*D + l + 64 of q, k and v (head dims up to 128); the
// RMS norm is a wave reduction.
//
// Input: the output of ONE projection GEMM x @ W_all^T with columns
//   [q (H*D) | k (H*D) | v (H*D) | gates (n_gates*H) | retrieve (H, optional)]
// (W_all stacks c_q, c_k, c_v, gate_alpha, gate_eta, gate_theta[, gate_gamma]
// [, retrieve_gate]); gate biases are added here.  All arithmetic is fp32.
#include <hip/hip_runtime.h>

#include "atlas_common.hpp"
#include "atlas_scan.h"
#include "atlas_status.hpp"

namespace atlas {
namespace {

constexpr int PRO_WAVES = 4;   // token-heads per workgroup
constexpr int PRO_CH = 2;      // channels per lane (head dims up to 2 x 64)

struct ProArgs {
  int B, T, H, D, K, P, NG, has_r;
  const void* proj;
  long long ld;
  int proj_dtype;
  const float* conv_w;   // (3, H*D, K)
  const float* conv_b;   // (3, H*D)
  const float* poly;     // (P)
  const float* gate_b;   // (NG, H)
  float max_lr;
  void *q, *k, *v;
  int out_dtype;
  float* gates;          // (NG, B, T, H)
  float* retrieve;       // (B, T, H)
};

__device__ __forceinline__ float poly_map(float x, const float* a, int P) {
  // sum_{i=1..P} a[i-1] x^i, powers accumulated left to right (as :459-466)
  float out = a[0] * x, xp = x;
  for (int i = 1; i < P; ++i) {
    xp *= x;
    out += a[i] * xp;
  }
  return out;
}

__global__ void __launch_bounds__(PRO_WAVES * WAVE) prologue_kernel(ProArgs a) {
  const int lane = lane_id();
  const long long item = (long long)blockIdx.x * PRO_WAVES + wave_id();   // (b, t, h)
  const long long n_items = (long long)a.B * a.T * a.H;
  if (item >= n_items) return;
  const int h = (int)(item % a.H);
  const long long bt = item / a.H;
  const int t = (int)(bt % a.T), b = (int)(bt / a.T);
  const int HD = a.H * a.D;
  // lane owns channels d = lane + 64 u (u < PRO_CH): head dims up to 128
  float vals[PRO_CH][3];
  bool act[PRO_CH];
#pragma unroll
  for (int u = 0; u < PRO_CH; ++u) {
    act[u] = lane + WAVE * u < a.D;
    const int d = act[u] ? lane + WAVE * u : 0;
#pragma unroll
    for (int which = 0; which < 3; ++which) {
      const int ch = which * HD + h * a.D + d;
      float acc = a.conv_b[which * HD + h * a.D + d];
      for (int j = 0; j < a.K; ++j) {
        const int ts = t - (a.K - 1) + j;
        if (ts >= 0)
          acc += a.conv_w[((long long)which * HD + h * a.D + d) * a.K + j] *
                 load_any(a.proj, ((long long)b * a.T + ts) * a.ld + ch, a.proj_dtype);
      }
      vals[u][which] = act[u] ? acc : 0.f;
    }
  }
  float qv[PRO_CH], kv[PRO_CH];
  const float inv_d = 1.f / (float)a.D;
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < PRO_CH; ++u) sq += vals[u][0] * vals[u][0];
  const float rq = rsqrtf(wave_sum(sq) * inv_d + 1e-6f);
#pragma unroll
  for (int u = 0; u < PRO_CH; ++u) {
    qv[u] = vals[u][0] * rq;
    if (a.P > 0) qv[u] = poly_map(qv[u], a.poly, a.P);
    kv[u] = (a.P > 0 && act[u]) ? poly_map(vals[u][1], a.poly, a.P) : vals[u][1];
  }
  float sk = 0.f;
#pragma unroll
  for (int u = 0; u < PRO_CH; ++u) sk += kv[u] * kv[u];
  const float rk = rsqrtf(wave_sum(sk) * inv_d + 1e-6f);
#pragma unroll
  for (int u = 0; u < PRO_CH; ++u) {
    if (act[u]) {
      const long long o = item * a.D + lane + WAVE * u;   // (B, T, H, D) dense
      store_any(a.q, o, a.out_dtype, qv[u]);
      store_any(a.k, o, a.out_dtype, kv[u] * rk);
      store_any(a.v, o, a.out_dtype, vals[u][2]);
    }
  }
  // gates: lanes 0..NG-1; retrieve gate: lane NG
  const long long row = ((long long)b * a.T + t) * a.ld + 3LL * HD;
  if (lane < a.NG) {
    const float z = load_any(a.proj, row + (long long)lane * a.H + h, a.proj_dtype) + a.gate_b[lane * a.H + h];
    float g = 1.f / (1.f + __expf(-z));
    if (lane == 1) g *= a.max_lr;
    a.gates[(long long)lane * n_items + item] = g;
  } else if (lane == a.NG && a.has_r) {
    const float z = load_any(a.proj, row + (long long)a.NG * a.H + h, a.proj_dtype);
    a.retrieve[item] = 1.f / (1.f + __expf(-z));
  }
}

// Vectorised variant for D in {16, 32, 64} and conv_kernel <= 4 (every
// configuration of the reference): one thread per four consecutive channels
// of a token row (the same four channels of q, k and v), a block per
// (b, run of PRO_TT tokens).  The thread keeps its 3 x 4 x K convolution
// weights in registers and slides a window of the last K projection rows
// over its tokens, so each projection element is loaded once, 4 channels per
// load (8 or 16 bytes), and q, k, v are stored 4 channels per store.  The
// RMS norms reduce over the D/4 threads of a head with lane shuffles.
constexpr int PRO_TT = 16;   // tokens per block

template <int K>
__global__ void __launch_bounds__(256) prologue_vec_kernel(ProArgs a, int nthr) {
  const int tid = threadIdx.x;
  const int nruns = (a.T + PRO_TT - 1) / PRO_TT;
  const int b = blockIdx.x / nruns, t0 = (blockIdx.x % nruns) * PRO_TT;
  const int HD = a.H * a.D, QD = a.D / 4;   // threads per head
  const bool act = tid < nthr;
  const int j = act ? tid : 0, ch = 4 * j;
  f32x4 w[3][K], bias[3];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long base = ((long long)m * HD + ch + u) * a.K;
#pragma unroll
      for (int tap = 0; tap < K; ++tap) w[m][tap][u] = a.conv_w[base + tap];
      bias[m][u] = a.conv_b[m * HD + ch + u];
    }
  }
  // window: x[m][i] = projection row t - (K - 1) + i (zero before the sequence)
  f32x4 x[3][K];
#pragma unroll
  for (int m = 0; m < 3; ++m)
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
      const int ts = t0 - (K - 1) + i;
      x[m][i] = (ts >= 0) ? load4_any(a.proj, ((long long)b * a.T + ts) * a.ld + m * HD + ch, a.proj_dtype)
                          : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  const float inv_d = 1.f / (float)a.D;
  const long long n_items = (long long)a.B * a.T * a.H;
  const int t1 = min(t0 + PRO_TT, a.T);
  for (int t = t0; t < t1; ++t) {
    const long long row = ((long long)b * a.T + t) * a.ld;
#pragma unroll
    for (int m = 0; m < 3; ++m) x[m][K - 1] = load4_any(a.proj, row + m * HD + ch, a.proj_dtype);
    f32x4 v3[3];
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      f32x4 acc = bias[m];
#pragma unroll
      for (int tap = 0; tap < K; ++tap) acc += w[m][tap] * x[m][tap];
      v3[m] = acc;
    }
    // q: norm then map; k: map then norm (memory_layer.py:612-616)
    auto head_sum = [&](f32x4 y) {
      float sq = (y[0] * y[0] + y[1] * y[1]) + (y[2] * y[2] + y[3] * y[3]);
      for (int off = QD / 2; off >= 1; off >>= 1) sq += __shfl_xor(sq, off, WAVE);
      return sq;
    };
    f32x4 qv = v3[0] * rsqrtf(head_sum(v3[0]) * inv_d + 1e-6f);
    f32x4 kv = v3[1];
    if (a.P > 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        qv[u] = poly_map(qv[u], a.poly, a.P);
        kv[u] = poly_map(kv[u], a.poly, a.P);
      }
    }
    kv = kv * rsqrtf(head_sum(kv) * inv_d + 1e-6f);
    if (act) {
      const long long o = ((long long)b * a.T + t) * HD + ch;   // (B, T, H, D) dense
      store4_any(a.q, o, a.out_dtype, qv);
      store4_any(a.k, o, a.out_dtype, kv);
      store4_any(a.v, o, a.out_dtype, v3[2]);
    }
    // gates (n_gates x H) and the retrieve gate (H): one thread each
    const int ng = a.NG * a.H, nr = a.has_r ? a.H : 0;
    for (int g = tid; g < ng + nr; g += blockDim.x) {
      const long long item = ((long long)b * a.T + t) * a.H + (g % a.H);
      const float z = load_any(a.proj, row + 3LL * HD + g, a.proj_dtype);
      if (g < ng) {
        const int gi = g / a.H;
        float gv = 1.f / (1.f + __expf(-(z + a.gate_b[g])));
        if (gi == 1) gv *= a.max_lr;
        a.gates[(long long)gi * n_items + item] = gv;
      } else {
        a.retrieve[item] = 1.f / (1.f + __expf(-z));
      }
    }
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int i = 0; i + 1 < K; ++i) x[m][i] = x[m][i + 1];
  }
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" atlas_status atlas_layer_prologue(int32_t B, int32_t T, int32_t H, int32_t D, int32_t conv_kernel,
                                             int32_t poly_degree, int32_t n_gates, int32_t has_retrieve,
                                             const void* proj, int64_t proj_ld, int32_t proj_dtype,
                                             const float* conv_w, const float* conv_b, const float* poly,
                                             const float* gate_b, float max_lr, void* q, void* k, void* v,
                                             int32_t out_dtype, float* gates, float* retrieve, void* stream) {
  clear_error();
  if (B < 1 || T < 1 || H < 1) return fail(ATLAS_ERR_INVALID_ARGUMENT, "B, T, H must be >= 1");
  if (D < 1 || D > PRO_CH * WAVE)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "head dim %d outside [1, %d]", D, PRO_CH * WAVE);
  if (conv_kernel < 1 || conv_kernel > 16) return fail(ATLAS_ERR_INVALID_ARGUMENT, "conv_kernel %d", conv_kernel);
  if (poly_degree < 0 || poly_degree > 8) return fail(ATLAS_ERR_INVALID_ARGUMENT, "poly_degree %d", poly_degree);
  if (n_gates < 3 || n_gates > 4) return fail(ATLAS_ERR_INVALID_ARGUMENT, "n_gates %d must be 3 or 4", n_gates);
  if (proj_dtype < 0 || proj_dtype > 2 || out_dtype < 0 || out_dtype > 2)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad dtype");
  const long long need = 3LL * H * D + (long long)(n_gates + (has_retrieve ? 1 : 0)) * H;
  if (proj_ld < need) return fail(ATLAS_ERR_INVALID_ARGUMENT, "proj_ld %lld < %lld columns", (long long)proj_ld, need);
  if (!proj || !conv_w || !conv_b || !gate_b || !q || !k || !v || !gates || (poly_degree > 0 && !poly) ||
      (has_retrieve && !retrieve))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "null pointer");
  ProArgs a{B, T, H, D, conv_kernel, poly_degree, n_gates, has_retrieve ? 1 : 0, proj, proj_ld, proj_dtype,
            conv_w, conv_b, poly, gate_b, max_lr, q, k, v, out_dtype, gates, retrieve};
  hipStream_t st = static_cast<hipStream_t>(stream);
  // vectorised path: 4-channel loads need the projection row, its stride and
  // the outputs aligned to 4 elements
  const int esz = proj_dtype == 0 ? 4 : 2, osz = out_dtype == 0 ? 4 : 2;
  const bool vec = (D == 16 || D == 32 || D == 64) && conv_kernel <= 4 && H * D / 4 <= 256 &&
                   proj_ld % 4 == 0 && reinterpret_cast<uintptr_t>(proj) % (4 * esz) == 0 &&
                   reinterpret_cast<uintptr_t>(q) % (4 * osz) == 0 && reinterpret_cast<uintptr_t>(k) % (4 * osz) == 0 &&
                   reinterpret_cast<uintptr_t>(v) % (4 * osz) == 0;
  if (vec) {
    const int nthr = H * D / 4, threads = (nthr + WAVE - 1) / WAVE * WAVE;
    const long long blocks = (long long)B * ((T + PRO_TT - 1) / PRO_TT);
    if (blocks > 0x7fffffffLL) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "too many token rows");
    switch (conv_kernel) {
      case 1: hipLaunchKernelGGL(prologue_vec_kernel<1>, dim3((unsigned)blocks), dim3(threads), 0, st, a, nthr); break;
      case 2: hipLaunchKernelGGL(prologue_vec_kernel<2>, dim3((unsigned)blocks), dim3(threads), 0, st, a, nthr); break;
      case 3: hipLaunchKernelGGL(prologue_vec_kernel<3>, dim3((unsigned)blocks), dim3(threads), 0, st, a, nthr); break;
      default: hipLaunchKernelGGL(prologue_vec_kernel<4>, dim3((unsigned)blocks), dim3(threads), 0, st, a, nthr); break;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail_hip(e, "prologue launch");
    return ATLAS_OK;
  }
  const long long items = (long long)B * T * H;
  const long long blocks = (items + PRO_WAVES - 1) / PRO_WAVES;
  if (blocks > 0x7fffffffLL) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "too many token-heads");
  hipLaunchKernelGGL(prologue_kernel, dim3((unsigned)blocks), dim3(PRO_WAVES * WAVE), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "prologue launch");
  return ATLAS_OK;
}
