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

// ---- backward ---------------------------------------------------------------
// Gradients of the prologue (memory_layer.py:606-633) for the cotangents of
// q, k, v, the gates and the retrieve gate, with respect to the projection
// output, the conv weights and biases, the polynomial coefficients and the
// gate biases.  Per channel c of q/k/v with conv output y and cotangent dy of
// y (below): dx_s = sum_j w_j dy_{s+K-1-j}, dw_j = sum_t dy_t x_{t-K+1+j},
// db = sum_t dy_t.  dy from the normalisations (n = y r, r = (mean y^2 +
// 1e-6)^{-1/2}: d y = r (dn - n <dn, n> / D)):
//   q = poly(n):          dn = dq poly'(n);   dpoly_i += <dq, n^i>
//   k = rms(kp), kp = poly(y):  dkp = rms backward of dk;  dy = dkp poly'(y);
//                         dpoly_i += <dkp, y^i>
//   v:                    dy = dv
// (without the polynomial, q = rms(y) and k = rms(y)); gates g = s(z + b)
// (eta's times max_lr) and the retrieve gate r = s(z): dz = dg * scale * s(1 - s).
// One block per (b, run of PRO_BR tokens) with the forward vector kernel's
// thread layout (four channels of q, k and v per thread, head reductions by
// lane shuffles); each block also recomputes dy for the K - 1 tokens after
// its run (the halo its last tokens' dx needs).  The weight gradients are
// per-block partial sums, added in block order by prologue_bwd_reduce_kernel
// (bitwise reproducible).
constexpr int PRO_BR = 64;   // tokens per backward block

struct ProBwdArgs {
  ProArgs f;                  // forward arguments (q, k, v, gates, retrieve unused)
  const void *gq, *gk, *gv;   // (B, T, H, D) cotangents, dtype gdt
  int gdt;
  const float* ggates;        // (NG, B, T, H)
  const float* gret;          // (B, T, H) or NULL
  float* dproj;               // (B, T, dld) fp32
  long long dld;
  float* part;                // per block: dw (3*HD*K), db (3*HD), dgb (NG*H), dpoly (P)
  int part_len;
};

// four consecutive projection elements by scalar loads (rows need not be
// 4-element aligned: the projection has 3 H D + (n_gates + 1) H columns)
__device__ __forceinline__ f32x4 ld4s(const void* p, int64_t i, int dtype) {
  return f32x4{load_any(p, i, dtype), load_any(p, i + 1, dtype), load_any(p, i + 2, dtype), load_any(p, i + 3, dtype)};
}

template <int K>
__global__ void __launch_bounds__(256) prologue_bwd_kernel(ProBwdArgs a, int nthr) {
  const ProArgs& f = a.f;
  const int tid = threadIdx.x;
  const int nruns = (f.T + PRO_BR - 1) / PRO_BR;
  const int b = blockIdx.x / nruns, t0 = (blockIdx.x % nruns) * PRO_BR;
  const int t1 = min(t0 + PRO_BR, f.T);   // owned tokens [t0, t1)
  const int HD = f.H * f.D, QD = f.D / 4;
  const bool act = tid < nthr;
  const int j = act ? tid : 0, ch = 4 * j;
  const float inv_d = 1.f / (float)f.D;
  f32x4 w[3][K], bias[3];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long base = ((long long)m * HD + ch + u) * f.K;
#pragma unroll
      for (int tap = 0; tap < K; ++tap) w[m][tap][u] = f.conv_w[base + tap];
      bias[m][u] = f.conv_b[m * HD + ch + u];
    }
  }
  f32x4 x[3][K], dyw[3][K];   // windows: x rows t-K+1 .. t, dy rows t-K+1 .. t
  f32x4 dw[3][K], db[3];
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    db[m] = z4;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      dw[m][i] = z4;
      dyw[m][i] = z4;
    }
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
      const int ts = t0 - (K - 1) + i;
      x[m][i] = (ts >= 0) ? ld4s(f.proj, ((long long)b * f.T + ts) * f.ld + m * HD + ch, f.proj_dtype) : z4;
    }
  }
  float dpoly[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto head_sum = [&](float v) {
    for (int off = QD / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return v;
  };
  auto dot4 = [](f32x4 p, f32x4 q) { return (p[0] * q[0] + p[1] * q[1]) + (p[2] * q[2] + p[3] * q[3]); };
  const long long n_items = (long long)f.B * f.T * f.H;
  const int ng = f.NG * f.H, nr = f.has_r ? f.H : 0;
  float dgb = 0.f;   // this thread's gate bias (g = tid < ng), summed over the run
  // t runs over the owned tokens and the K - 1 after them: the halo's dy
  // (recomputed; zero past the sequence end) completes the last owned dx
  for (int t = t0; t < t1 + K - 1; ++t) {
    const bool valid = t < f.T, own = t < t1;
    const long long row = ((long long)b * f.T + (valid ? t : 0)) * f.ld;
    f32x4 dy[3] = {z4, z4, z4};
    if (valid) {   // block-uniform: the shuffles below see every lane
#pragma unroll
      for (int m = 0; m < 3; ++m) x[m][K - 1] = ld4s(f.proj, row + m * HD + ch, f.proj_dtype);
      f32x4 y[3];
#pragma unroll
      for (int m = 0; m < 3; ++m) {
        f32x4 acc = bias[m];
#pragma unroll
        for (int tap = 0; tap < K; ++tap) acc += w[m][tap] * x[m][tap];
        y[m] = acc;
      }
      const long long o = ((long long)b * f.T + t) * HD + ch;   // (B, T, H, D) dense
      const f32x4 gq = act ? load4_any(a.gq, o, a.gdt) : z4;
      const f32x4 gk = act ? load4_any(a.gk, o, a.gdt) : z4;
      const f32x4 gv = act ? load4_any(a.gv, o, a.gdt) : z4;
      // q: n = rms(y), q = poly(n)
      {
        const float r = rsqrtf(head_sum(dot4(y[0], y[0])) * inv_d + 1e-6f);
        const f32x4 n = y[0] * r;
        f32x4 dn = gq;
        if (f.P > 0) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            float dp = f.poly[0], np = 1.f;   // poly'(n) = sum_i i a_i n^{i-1}
            for (int i = 1; i < f.P; ++i) {
              np *= n[u];
              dp += (float)(i + 1) * f.poly[i] * np;
            }
            if (own) {
              float pw = n[u];
              for (int i = 0; i < f.P; ++i) {
                dpoly[i] += gq[u] * pw;
                pw *= n[u];
              }
            }
            dn[u] = gq[u] * dp;
          }
        }
        const float sdot = head_sum(dot4(dn, n)) * inv_d;
        dy[0] = (dn - n * sdot) * r;
      }
      // k: kp = poly(y), k = rms(kp)
      {
        f32x4 kp = y[1], dpy = {1.f, 1.f, 1.f, 1.f};
        if (f.P > 0) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            kp[u] = poly_map(y[1][u], f.poly, f.P);
            float dp = f.poly[0], yp = 1.f;
            for (int i = 1; i < f.P; ++i) {
              yp *= y[1][u];
              dp += (float)(i + 1) * f.poly[i] * yp;
            }
            dpy[u] = dp;
          }
        }
        const float r = rsqrtf(head_sum(dot4(kp, kp)) * inv_d + 1e-6f);
        const f32x4 kn = kp * r;
        const float sdot = head_sum(dot4(gk, kn)) * inv_d;
        const f32x4 dkp = (gk - kn * sdot) * r;
        if (f.P > 0 && own) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            float pw = y[1][u];
            for (int i = 0; i < f.P; ++i) {
              dpoly[i] += dkp[u] * pw;
              pw *= y[1][u];
            }
          }
        }
        dy[1] = dkp * dpy;
      }
      dy[2] = gv;
      if (!act) dy[0] = dy[1] = z4;
      if (own) {
#pragma unroll
        for (int m = 0; m < 3; ++m) {
          db[m] += dy[m];
#pragma unroll
          for (int tap = 0; tap < K; ++tap) dw[m][tap] += dy[m] * x[m][tap];
        }
        // gates and the retrieve gate (one thread each)
        const long long drow = ((long long)b * f.T + t) * a.dld;
        for (int g = tid; g < ng + nr; g += blockDim.x) {
          const long long item = ((long long)b * f.T + t) * f.H + (g % f.H);
          const float zz = load_any(f.proj, row + 3LL * HD + g, f.proj_dtype);
          float dz;
          if (g < ng) {
            const int gi = g / f.H;
            const float sg = 1.f / (1.f + __expf(-(zz + f.gate_b[g])));
            dz = a.ggates[(long long)gi * n_items + item] * (gi == 1 ? f.max_lr : 1.f) * sg * (1.f - sg);
            if (g == tid) dgb += dz;
          } else {
            const float sg = 1.f / (1.f + __expf(-zz));
            dz = a.gret ? a.gret[item] * sg * (1.f - sg) : 0.f;
          }
          a.dproj[drow + 3LL * HD + g] = dz;
        }
      }
    }
#pragma unroll
    for (int m = 0; m < 3; ++m) dyw[m][K - 1] = dy[m];
    // dx of token s = t - (K - 1): sum_j w_j dy_{s+K-1-j} = sum_j w_j dyw[K-1-j]
    const int s_ = t - (K - 1);
    if (s_ >= t0 && act) {   // s_ < t1 by the loop bound
      const long long drow = ((long long)b * f.T + s_) * a.dld;
#pragma unroll
      for (int m = 0; m < 3; ++m) {
        f32x4 acc = z4;
#pragma unroll
        for (int tap = 0; tap < K; ++tap) acc += w[m][tap] * dyw[m][K - 1 - tap];
#pragma unroll
        for (int u = 0; u < 4; ++u) a.dproj[drow + m * HD + ch + u] = acc[u];
      }
    }
    // slide the windows
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int i = 0; i + 1 < K; ++i) {
        x[m][i] = x[m][i + 1];
        dyw[m][i] = dyw[m][i + 1];
      }
  }
  // block partials: dw, db (per channel), dgb (per gate bias), dpoly (block sum)
  float* pt = a.part + (long long)blockIdx.x * a.part_len;
  if (act) {
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int tap = 0; tap < K; ++tap) pt[((long long)m * HD + ch + u) * f.K + tap] = dw[m][tap][u];
        pt[3LL * HD * f.K + m * HD + ch + u] = db[m][u];
      }
  }
  if (tid < ng) pt[3LL * HD * (f.K + 1) + tid] = dgb;
  __shared__ float red[8][4];
  for (int i = 0; i < f.P; ++i) {
    float v = act ? dpoly[i] : 0.f;
    for (int off = WAVE / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
    if (lane_id() == 0) red[i][wave_id()] = v;
  }
  __syncthreads();
  if (tid < f.P) {
    float v = 0.f;
    for (int wv = 0; wv < (int)(blockDim.x / WAVE); ++wv) v += red[tid][wv];
    pt[3LL * HD * (f.K + 1) + ng + tid] = v;
  }
}

// the block partials summed in block order into d_conv_w (3*HD*K), d_conv_b
// (3*HD), d_gate_b (NG*H) and d_poly (P), laid out consecutively in a partial
__global__ void __launch_bounds__(256) prologue_bwd_reduce_kernel(const float* part, int nblk, int len, int n_w,
                                                                  int n_b, int n_g, float* dw, float* db, float* dg,
                                                                  float* dp) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= len) return;
  float s = 0.f;
  for (int blk = 0; blk < nblk; ++blk) s += part[(long long)blk * len + i];
  if (i < n_w) dw[i] = s;
  else if (i < n_w + n_b) db[i - n_w] = s;
  else if (i < n_w + n_b + n_g) dg[i - n_w - n_b] = s;
  else dp[i - n_w - n_b - n_g] = s;
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

namespace {

// the backward's vector layout (every reference configuration): D 16/32/64,
// conv kernel <= 4, one block row of H*D/4 <= 256 threads that also covers
// the gate biases
bool prologue_bwd_supported(int H, int D, int K, int NG) {
  const int nthr = H * D / 4, threads = (nthr + WAVE - 1) / WAVE * WAVE;
  return (D == 16 || D == 32 || D == 64) && K >= 1 && K <= 4 && nthr <= 256 && NG * H <= threads;
}

}  // namespace

extern "C" size_t atlas_layer_prologue_bwd_workspace_size(int32_t B, int32_t T, int32_t H, int32_t D,
                                                          int32_t conv_kernel, int32_t poly_degree,
                                                          int32_t n_gates) {
  if (B < 1 || T < 1 || poly_degree < 0 || poly_degree > 8 || n_gates < 3 || n_gates > 4 ||
      !prologue_bwd_supported(H, D, conv_kernel, n_gates))
    return 0;
  const long long HD = (long long)H * D;
  const long long len = 3 * HD * (conv_kernel + 1) + (long long)n_gates * H + poly_degree;
  const long long nblk = (long long)B * ((T + PRO_BR - 1) / PRO_BR);
  return (size_t)(nblk * len) * sizeof(float);
}

extern "C" atlas_status atlas_layer_prologue_bwd(
    int32_t B, int32_t T, int32_t H, int32_t D, int32_t conv_kernel, int32_t poly_degree, int32_t n_gates,
    int32_t has_retrieve, const void* proj, int64_t proj_ld, int32_t proj_dtype, const float* conv_w,
    const float* conv_b, const float* poly, const float* gate_b, float max_lr, const void* dq, const void* dk,
    const void* dv, int32_t grad_dtype, const float* dgates, const float* dretrieve, float* dproj, int64_t dproj_ld,
    float* d_conv_w, float* d_conv_b, float* d_poly, float* d_gate_b, void* workspace, size_t workspace_bytes,
    void* stream) {
  clear_error();
  if (B < 1 || T < 1 || H < 1) return fail(ATLAS_ERR_INVALID_ARGUMENT, "B, T, H must be >= 1");
  if (n_gates < 3 || n_gates > 4) return fail(ATLAS_ERR_INVALID_ARGUMENT, "n_gates %d must be 3 or 4", n_gates);
  if (poly_degree < 0 || poly_degree > 8) return fail(ATLAS_ERR_INVALID_ARGUMENT, "poly_degree %d", poly_degree);
  if (!prologue_bwd_supported(H, D, conv_kernel, n_gates))
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "prologue backward compiled for D 16/32/64, conv kernel <= 4 and "
                "H*D <= 1024 (got H %d D %d K %d)", H, D, conv_kernel);
  if (proj_dtype < 0 || proj_dtype > 2 || grad_dtype < 0 || grad_dtype > 2)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad dtype");
  const long long ncols = 3LL * H * D + (long long)(n_gates + (has_retrieve ? 1 : 0)) * H;
  if (proj_ld < ncols || dproj_ld < ncols)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "proj_ld / dproj_ld below the %lld projection columns", ncols);
  if (!proj || !conv_w || !conv_b || !gate_b || !dq || !dk || !dv || !dgates || !dproj || !d_conv_w || !d_conv_b ||
      !d_gate_b || (poly_degree > 0 && (!poly || !d_poly)))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "null pointer");
  const size_t need = atlas_layer_prologue_bwd_workspace_size(B, T, H, D, conv_kernel, poly_degree, n_gates);
  if (!workspace || workspace_bytes < need)
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, need);
  const int esz = proj_dtype == 0 ? 4 : 2, gsz = grad_dtype == 0 ? 4 : 2;
  auto mis = [](const void* p, int al) { return reinterpret_cast<uintptr_t>(p) % al != 0; };
  (void)esz;
  if (mis(dq, 4 * gsz) || mis(dk, 4 * gsz) || mis(dv, 4 * gsz) || mis(workspace, 4))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "the q/k/v cotangents must be 4-element aligned");
  ProBwdArgs a;
  a.f = ProArgs{B, T, H, D, conv_kernel, poly_degree, n_gates, has_retrieve ? 1 : 0, proj, proj_ld, proj_dtype,
                conv_w, conv_b, poly, gate_b, max_lr, nullptr, nullptr, nullptr, 0, nullptr, nullptr};
  a.gq = dq; a.gk = dk; a.gv = dv; a.gdt = grad_dtype;
  a.ggates = dgates; a.gret = has_retrieve ? dretrieve : nullptr;
  a.dproj = dproj; a.dld = dproj_ld;
  a.part = static_cast<float*>(workspace);
  const long long HD = (long long)H * D;
  const int n_w = (int)(3 * HD * conv_kernel), n_b = (int)(3 * HD), n_g = n_gates * H;
  a.part_len = n_w + n_b + n_g + poly_degree;
  const int nthr = H * D / 4, threads = (nthr + WAVE - 1) / WAVE * WAVE;
  const long long nblk = (long long)B * ((T + PRO_BR - 1) / PRO_BR);
  if (nblk > 0x7fffffffLL) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "too many token rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (conv_kernel) {
    case 1: hipLaunchKernelGGL(prologue_bwd_kernel<1>, dim3((unsigned)nblk), dim3(threads), 0, st, a, nthr); break;
    case 2: hipLaunchKernelGGL(prologue_bwd_kernel<2>, dim3((unsigned)nblk), dim3(threads), 0, st, a, nthr); break;
    case 3: hipLaunchKernelGGL(prologue_bwd_kernel<3>, dim3((unsigned)nblk), dim3(threads), 0, st, a, nthr); break;
    default: hipLaunchKernelGGL(prologue_bwd_kernel<4>, dim3((unsigned)nblk), dim3(threads), 0, st, a, nthr); break;
  }
  hipLaunchKernelGGL(prologue_bwd_reduce_kernel, dim3((unsigned)((a.part_len + 255) / 256)), dim3(256), 0, st,
                     a.part, (int)nblk, a.part_len, n_w, n_b, n_g, d_conv_w, d_conv_b, d_gate_b, d_poly);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ATLAS_OK : fail_hip(e, "prologue backward launch");
}
