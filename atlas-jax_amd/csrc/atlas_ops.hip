// atlas_linear_scan, atlas_linear_scan_bwd and atlas_fused_chunk_fwd.
//
// atlas_linear_scan: h_t = g_t h_{t-1} + x_t (memory_layer.py:256-296,
// kernels/triton_scan.py:15-48).  HBM-bound; one thread per (b, h, state
// element), sequential over T, coalesced along the state element.
//
// atlas_fused_chunk_fwd: the plugin operator fused_chunk_scan
// (kernels/fused_chunk.py:321-355) with the semantics of its _regular_fwd
// (:279-314): momentum scans over precomputed momentum inputs, Polar-Express
// of every S_t, memory scans, read-out y_t = q_t + W1_t gelu_tanh(W2_t q_t).
// It is built from the linear-scan kernel, the batched Polar-Express kernel
// and a read-out kernel; the per-token states live in the workspace.
#include <hip/hip_runtime.h>

#include "atlas_common.hpp"
#include "atlas_scan.h"
#include "atlas_status.hpp"

extern "C" atlas_status atlas_pe_batched(int64_t n, int32_t d1, int32_t d2, int32_t ns_steps, int32_t norm_mode,
                                         const void* X, void* Y, int32_t dtype, int32_t compute, void* stream);

namespace atlas {
namespace {

// h_all[b,t,h,:] for inputs laid out (B, T, H, N) with gates (B, T, H).
// in_dtype/gate_dtype select the loads; state and outputs are fp32.
__global__ void linear_scan_kernel(int B, int T, int H, long long N, const float* h_init, const void* gates,
                                   int gate_dtype, const void* inputs, int in_dtype, float* h_all,
                                   float* h_final) {
  const long long per = (N + blockDim.x - 1) / blockDim.x;
  const long long bh = blockIdx.x / per;
  const long long n = (blockIdx.x % per) * blockDim.x + threadIdx.x;
  if (bh >= (long long)B * H || n >= N) return;
  const long long b = bh / H, hh = bh % H;
  float h = h_init[bh * N + n];
  for (int t = 0; t < T; ++t) {
    const long long gi = (b * T + t) * H + hh;
    const long long xi = gi * N + n;
    h = load_any(gates, gi, gate_dtype) * h + load_any(inputs, xi, in_dtype);
    if (h_all) h_all[xi] = h;
  }
  h_final[bh * N + n] = h;
}

atlas_status launch_linear_scan(int B, int T, int H, long long N, const float* h_init, const void* gates,
                                int gate_dtype, const void* inputs, int in_dtype, float* h_all, float* h_final,
                                hipStream_t st) {
  const int tpb = 256;
  const long long per = (N + tpb - 1) / tpb;
  const long long blocks = (long long)B * H * per;
  if (blocks > 0x7fffffffLL) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "linear scan grid too large");
  hipLaunchKernelGGL(linear_scan_kernel, dim3((unsigned)blocks), dim3(tpb), 0, st, B, T, H, N, h_init, gates,
                     gate_dtype, inputs, in_dtype, h_all, h_final);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "linear_scan launch");
}

// Backward of the linear scan (kernels/triton_scan.py:119-161): with
// G_t = dh_all_t + [t = T-1] dh_final + g_{t+1} G_{t+1} (reverse in time),
//   d inputs_t = G_t,  d h_init = g_0 G_0,  d gates_t = <G_t, h_{t-1}>
// (h_{-1} = h_init).  One thread per (b, h, state element) as in the forward;
// each wave writes its partial of <G_t, h_{t-1}> to gpart[(b,t,h)][wave
// index], summed in a fixed order by linear_scan_gate_grad_kernel.
__global__ void linear_scan_bwd_kernel(int B, int T, int H, long long N, const float* h_init, const float* gates,
                                       const float* h_all, const float* dh_all, const float* dh_final,
                                       float* d_inputs, float* d_h_init, float* gpart, int nparts) {
  const long long per = (N + blockDim.x - 1) / blockDim.x;
  const long long bh = blockIdx.x / per;
  const long long blk = blockIdx.x % per;
  const long long n = blk * blockDim.x + threadIdx.x;
  const bool live = n < N;
  const long long b = bh / H, hh = bh % H;
  const int part = (int)(blk * (blockDim.x / WAVE) + threadIdx.x / WAVE);
  float G = (live && dh_final) ? dh_final[bh * N + n] : 0.f;
  for (int t = T - 1; t >= 0; --t) {
    const long long gi = (b * T + t) * H + hh;
    const long long xi = gi * N + n;
    if (t < T - 1) G *= gates[(b * T + t + 1) * H + hh];
    if (live) {
      if (dh_all) G += dh_all[xi];
      d_inputs[xi] = G;
    }
    const float hp = live ? (t > 0 ? h_all[xi - (long long)H * N] : h_init[bh * N + n]) : 0.f;
    const float s = wave_sum(G * hp);
    if (lane_id() == 0) gpart[gi * nparts + part] = s;
  }
  if (live) d_h_init[bh * N + n] = gates[(b * T) * H + hh] * G;
}

__global__ void linear_scan_gate_grad_kernel(long long rows, int nparts, const float* gpart, float* d_gates) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows) return;
  float s = 0.f;
  for (int p = 0; p < nparts; ++p) s += gpart[i * nparts + p];
  d_gates[i] = s;
}

// y[b,t,h,:] = q + W1_t gelu_tanh(W2_t q) with W1_t (D,E), W2_t (E,D) from the
// per-token memory states (B, cs, H, D*E).  One workgroup per token.
__global__ void readout_kernel(int D, int E, const float* W1all, const float* W2all, const void* q, void* y,
                               int io_dtype) {
  extern __shared__ float sh[];
  float* qs = sh;       // [D]
  float* gs = sh + D;   // [E]
  const long long tok = blockIdx.x;
  const float* W1 = W1all + tok * D * E;
  const float* W2 = W2all + tok * D * E;
  for (int d = threadIdx.x; d < D; d += blockDim.x) qs[d] = load_any(q, tok * D + d, io_dtype);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc += W2[(long long)e * D + d] * qs[d];
    gs[e] = gelu_tanh(acc);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f;
    for (int e = 0; e < E; ++e) acc += W1[(long long)d * E + e] * gs[e];
    store_any(y, tok * D + d, io_dtype, qs[d] + acc);
  }
}

}  // namespace
}  // namespace atlas

using namespace atlas;

extern "C" atlas_status atlas_linear_scan(int32_t B, int32_t T, int32_t H, int64_t N, const float* h_init,
                                          const float* gates, const float* inputs, float* h_all, float* h_final,
                                          void* stream) {
  clear_error();
  if (B < 1 || T < 0 || H < 1 || N < 1) return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad sizes");
  if (!h_init || !gates || !inputs || !h_final || (T > 0 && !h_all))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL pointer");
  return launch_linear_scan(B, T, H, N, h_init, gates, 0, inputs, 0, h_all, h_final,
                            static_cast<hipStream_t>(stream));
}

extern "C" size_t atlas_linear_scan_bwd_workspace_size(int32_t B, int32_t T, int32_t H, int64_t N) {
  if (B < 1 || T < 1 || H < 1 || N < 1) return 0;
  const long long nparts = (N + 255) / 256 * 4;
  return (size_t)B * T * H * nparts * sizeof(float);
}

extern "C" atlas_status atlas_linear_scan_bwd(int32_t B, int32_t T, int32_t H, int64_t N, const float* h_init,
                                              const float* gates, const float* h_all, const float* dh_all,
                                              const float* dh_final, float* d_h_init, float* d_gates,
                                              float* d_inputs, void* workspace, size_t workspace_bytes,
                                              void* stream) {
  clear_error();
  if (B < 1 || T < 1 || H < 1 || N < 1) return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad sizes");
  if (!h_init || !gates || !h_all || !d_h_init || !d_gates || !d_inputs)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL pointer (only dh_all / dh_final may be NULL)");
  const size_t need = atlas_linear_scan_bwd_workspace_size(B, T, H, N);
  if (!workspace || workspace_bytes < need)
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, need);
  const int tpb = 256;
  const long long per = (N + tpb - 1) / tpb;
  const long long blocks = (long long)B * H * per;
  if (blocks > 0x7fffffffLL) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "linear scan grid too large");
  const int nparts = (int)(per * (tpb / WAVE));
  float* gpart = static_cast<float*>(workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(linear_scan_bwd_kernel, dim3((unsigned)blocks), dim3(tpb), 0, st, B, T, H, N, h_init, gates,
                     h_all, dh_all, dh_final, d_inputs, d_h_init, gpart, nparts);
  const long long rows = (long long)B * T * H;
  hipLaunchKernelGGL(linear_scan_gate_grad_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, rows,
                     nparts, gpart, d_gates);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "linear_scan_bwd launch");
}

extern "C" size_t atlas_fused_chunk_workspace_size(int32_t B, int32_t H, int32_t D, int32_t E, int32_t cs) {
  if (B < 1 || H < 1 || D < 1 || E < 1 || cs < 1) return 0;
  // S_all and W_all for both weights, fp32
  return (size_t)4 * B * cs * H * (size_t)D * E * sizeof(float);
}

extern "C" atlas_status atlas_fused_chunk_fwd(int32_t B, int32_t cs, int32_t H, int32_t D, int32_t E,
                                              int32_t ns_steps, int32_t io_dtype, int32_t gate_dtype,
                                              int32_t compute, float* W1, float* W2, float* SW1, float* SW2,
                                              const void* momW1, const void* momW2, const void* theta,
                                              const void* alpha, const void* q, void* y, void* workspace,
                                              size_t workspace_bytes, void* stream) {
  clear_error();
  if (B < 1 || cs < 1 || H < 1 || D < 1 || E < 1) return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad sizes");
  if (ns_steps < 0 || ns_steps > 5) return fail(ATLAS_ERR_INVALID_ARGUMENT, "ns_steps %d outside [0, 5]", ns_steps);
  if (!W1 || !W2 || !SW1 || !SW2 || !momW1 || !momW2 || !theta || !alpha || !q || !y)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (io_dtype < 0 || io_dtype > 2 || gate_dtype < 0 || gate_dtype > 2)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad dtype");
  const size_t need = atlas_fused_chunk_workspace_size(B, H, D, E, cs);
  if (!workspace || workspace_bytes < need)
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const long long DE = (long long)D * E, ntok = (long long)B * cs * H;
  float* S1all = static_cast<float*>(workspace);
  float* S2all = S1all + ntok * DE;
  float* W1all = S2all + ntok * DE;
  float* W2all = W1all + ntok * DE;
  atlas_status s;
  // momentum scans S_t = theta_t S_{t-1} + mom_t (state updated in place)
  if ((s = launch_linear_scan(B, cs, H, DE, SW1, theta, gate_dtype, momW1, io_dtype, S1all, SW1, st))) return s;
  if ((s = launch_linear_scan(B, cs, H, DE, SW2, theta, gate_dtype, momW2, io_dtype, S2all, SW2, st))) return s;
  // P_t = PE(S_t): W1 states are (D, E), W2 states (E, D)
  if ((s = atlas_pe_batched(ntok, D, E, ns_steps, ATLAS_PE_NORM_EPS, S1all, S1all, 0, compute, st))) return s;
  if ((s = atlas_pe_batched(ntok, E, D, ns_steps, ATLAS_PE_NORM_EPS, S2all, S2all, 0, compute, st))) return s;
  // memory scans W_t = alpha_t W_{t-1} + P_t
  if ((s = launch_linear_scan(B, cs, H, DE, W1, alpha, gate_dtype, S1all, 0, W1all, W1, st))) return s;
  if ((s = launch_linear_scan(B, cs, H, DE, W2, alpha, gate_dtype, S2all, 0, W2all, W2, st))) return s;
  hipLaunchKernelGGL(readout_kernel, dim3((unsigned)ntok), dim3(128), (size_t)(D + E) * sizeof(float), st, D, E,
                     W1all, W2all, q, y, io_dtype);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "readout launch");
}
