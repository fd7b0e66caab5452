// Memory-layer prologue after the input projections (atlas_jax/memory_layer.py
// :606-633): causal depthwise convolutions of q/k/v (ShortConv, :303-329),
// RMS norm (:211-216) and the polynomial feature map (:459-466) with the
// q/k asymmetry (q: norm then map; k: map then norm), and the sigmoid gates
// (eta times max_lr).  One wave per (b, t, h) token-head: lane d owns channel
// h*D + d of q, k and v; the RMS norm is a wave reduction over the D lanes.
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
  const bool act = lane < a.D;
  const int d = act ? lane : 0;

  float vals[3];
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
    vals[which] = act ? acc : 0.f;
  }
  float qv = vals[0], kv = vals[1];
  const float inv_d = 1.f / (float)a.D;
  if (a.P > 0) {
    qv = qv * rsqrtf(wave_sum(qv * qv) * inv_d + 1e-6f);
    qv = poly_map(qv, a.poly, a.P);
    kv = act ? poly_map(kv, a.poly, a.P) : 0.f;
    kv = kv * rsqrtf(wave_sum(kv * kv) * inv_d + 1e-6f);
  } else {
    qv = qv * rsqrtf(wave_sum(qv * qv) * inv_d + 1e-6f);
    kv = kv * rsqrtf(wave_sum(kv * kv) * inv_d + 1e-6f);
  }
  if (act) {
    const long long o = item * a.D + d;   // (B, T, H, D) dense
    store_any(a.q, o, a.out_dtype, qv);
    store_any(a.k, o, a.out_dtype, kv);
    store_any(a.v, o, a.out_dtype, vals[2]);
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
  if (D < 1 || D > WAVE) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "head dim %d outside [1, %d]", D, WAVE);
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
  const long long items = (long long)B * T * H;
  const long long blocks = (items + PRO_WAVES - 1) / PRO_WAVES;
  if (blocks > 0x7fffffffLL) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "too many token-heads");
  hipLaunchKernelGGL(prologue_kernel, dim3((unsigned)blocks), dim3(PRO_WAVES * WAVE), 0,
                     static_cast<hipStream_t>(stream), a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "prologue launch");
  return ATLAS_OK;
}
