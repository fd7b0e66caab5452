// Device-side building blocks shared by the Atlas kernels (gfx950 / CDNA4).
//
// Matrix-core conventions used throughout
// ---------------------------------------
// All products use 32x32 output tiles.  A 32x32 fp32 accumulator (f32x16 per
// lane, "C layout") holds element (row, col) with
//     col = lane % 32,   row = 8*(r/4) + 4*(lane/32) + (r%4)   for register r.
// For C = P*Q the A operand fragment of lane l holds P[l%32][k-slots] and the
// B operand fragment holds Q[k-slots][l%32]; the hardware only requires that
// both operands use the same lane-half/element -> k assignment.  Hence a
// C-layout tile T whose ROWS run along the contraction index can feed an MFMA
// directly: as the B operand it supplies T itself, as the A operand it
// supplies T^T.  Symmetric Gram matrices therefore never need a transpose,
// and a chain X -> B*X keeps X in registers.  kslot() gives the row held by
// each fragment element under this C-layout assignment.
//
// Two arithmetic modes share the kernel code:
//   ModeF16: v_mfma_f32_32x32x16_f16, fp16 operands, fp32 accumulation.
//   ModeF32: v_mfma_f32_32x32x2f32, fp32 operands.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace atlas {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int WAVE = 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / WAVE; }

// Row of accumulator register r in lane-half h (C layout above).
__device__ __forceinline__ constexpr int crow(int r, int h) {
  return 8 * (r >> 2) + 4 * h + (r & 3);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

struct ModeF16 {
  using elem = _Float16;   // operand storage type in LDS
  using frag = f16x8;      // one MFMA operand fragment
  static constexpr int KB = 16;   // contraction depth of one MFMA
  static constexpr int KPT = 2;   // K-blocks per 32-row C tile

  __device__ __forceinline__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // Fragment kb of a C-layout tile whose rows are the contraction index.
  __device__ __forceinline__ static frag from_c(const f32x16& t, int kb) {
    frag f;
#pragma unroll
    for (int v = 0; v < 8; ++v) f[v] = (_Float16)t[8 * kb + v];
    return f;
  }
  // Row (within the 32-row tile) carried by element v of K-block kb, half h.
  __device__ __forceinline__ static constexpr int kslot(int kb, int h, int v) {
    return 16 * kb + 8 * (v >> 2) + 4 * h + (v & 3);
  }
  // Fragment from a contiguous LDS row: elements k = 16*kb + 8*h + (0..7).
  __device__ __forceinline__ static frag ld_contig(const elem* row, int kb, int h) {
    return *reinterpret_cast<const frag*>(row + 16 * kb + 8 * h);
  }
  // Fragment from an LDS row using the C-layout k assignment (kslot).
  __device__ __forceinline__ static frag ld_cslot(const elem* row, int kb, int h) {
    f16x4 lo = *reinterpret_cast<const f16x4*>(row + 16 * kb + 4 * h);
    f16x4 hi = *reinterpret_cast<const f16x4*>(row + 16 * kb + 8 + 4 * h);
    frag f;
#pragma unroll
    for (int v = 0; v < 4; ++v) { f[v] = lo[v]; f[4 + v] = hi[v]; }
    return f;
  }
  // Fragment gathered from a global fp32 row using the C-layout k assignment.
  __device__ __forceinline__ static frag gl_cslot(const float* row, int kb, int h) {
    f32x4 lo = *reinterpret_cast<const f32x4*>(row + 16 * kb + 4 * h);
    f32x4 hi = *reinterpret_cast<const f32x4*>(row + 16 * kb + 8 + 4 * h);
    frag f;
#pragma unroll
    for (int v = 0; v < 4; ++v) { f[v] = (_Float16)lo[v]; f[4 + v] = (_Float16)hi[v]; }
    return f;
  }
  // Fragment from a global fp32 row, contiguous k = 16*kb + 8*h + (0..7).
  __device__ __forceinline__ static frag gl_contig(const float* row, int kb, int h) {
    f32x4 lo = *reinterpret_cast<const f32x4*>(row + 16 * kb + 8 * h);
    f32x4 hi = *reinterpret_cast<const f32x4*>(row + 16 * kb + 8 * h + 4);
    frag f;
#pragma unroll
    for (int v = 0; v < 4; ++v) { f[v] = (_Float16)lo[v]; f[4 + v] = (_Float16)hi[v]; }
    return f;
  }
  __device__ __forceinline__ static frag scale(frag f, float s) {
    const _Float16 hs = (_Float16)s;
    return f * hs;
  }
  __device__ __forceinline__ static frag scale_v(frag f, frag s) { return f * s; }
  __device__ __forceinline__ static elem to_elem(float x) { return (_Float16)x; }
  // A-operand fragment of the 32x32 identity for K-block kb (row c, half h).
  __device__ __forceinline__ static frag identity(int kb, int c, int h) {
    frag f;
#pragma unroll
    for (int v = 0; v < 8; ++v) f[v] = (c == kslot(kb, h, v)) ? (_Float16)1.f : (_Float16)0.f;
    return f;
  }
  // Accumulation operands (acc += w * T via an identity MFMA) use bf16: fp32's
  // exponent range, so contributions far below fp16's range are not lost.
  using afrag = bf16x8;
  __device__ __forceinline__ static f32x16 amma(afrag a, afrag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static afrag a_from_c(const f32x16& t, int kb) {
    afrag f;
#pragma unroll
    for (int v = 0; v < 8; ++v) f[v] = (__bf16)t[8 * kb + v];
    return f;
  }
  __device__ __forceinline__ static afrag a_identity(int kb, int c, int h, float w) {
    afrag f;
    const __bf16 one = (__bf16)w, zero = (__bf16)0.f;
#pragma unroll
    for (int v = 0; v < 8; ++v) f[v] = (c == kslot(kb, h, v)) ? one : zero;
    return f;
  }
};

struct ModeF32 {
  using elem = float;
  using frag = float;
  static constexpr int KB = 2;
  static constexpr int KPT = 16;

  __device__ __forceinline__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag from_c(const f32x16& t, int kb) { return t[kb]; }
  __device__ __forceinline__ static constexpr int kslot(int kb, int h, int /*v*/) {
    return 8 * (kb >> 2) + 4 * h + (kb & 3);
  }
  __device__ __forceinline__ static frag ld_contig(const elem* row, int kb, int h) {
    return row[2 * kb + h];
  }
  __device__ __forceinline__ static frag ld_cslot(const elem* row, int kb, int h) {
    return row[kslot(kb, h, 0)];
  }
  __device__ __forceinline__ static frag gl_cslot(const float* row, int kb, int h) {
    return row[kslot(kb, h, 0)];
  }
  __device__ __forceinline__ static frag gl_contig(const float* row, int kb, int h) {
    return row[2 * kb + h];
  }
  __device__ __forceinline__ static frag scale(frag f, float s) { return f * s; }
  __device__ __forceinline__ static frag scale_v(frag f, frag s) { return f * s; }
  __device__ __forceinline__ static elem to_elem(float x) { return x; }
  __device__ __forceinline__ static frag identity(int kb, int c, int h) {
    return (c == kslot(kb, h, 0)) ? 1.f : 0.f;
  }
  using afrag = float;
  __device__ __forceinline__ static f32x16 amma(afrag a, afrag b, f32x16 c) { return mma(a, b, c); }
  __device__ __forceinline__ static afrag a_from_c(const f32x16& t, int kb) { return t[kb]; }
  __device__ __forceinline__ static afrag a_identity(int kb, int c, int h, float w) {
    return (c == kslot(kb, h, 0)) ? w : 0.f;
  }
};

// Polar-Express coefficient rows (a, b, c) of atlas_jax/memory_layer.py:34-40.
__constant__ static const float kPE[5][3] = {
    {8.156554524902461f, -22.48329292557795f, 15.878769915207462f},
    {4.042929935166739f, -2.808917465908714f, 0.5000178451051316f},
    {3.8916678022926607f, -2.772484153217685f, 0.5060648178503393f},
    {3.285753657755655f, -2.3681294933425376f, 0.46449024233003106f},
    {2.3465413258596377f, -1.7097828382687081f, 0.42323551169305323f},
};
// Per-step factors (a, b/c, c/a) of the fp16 Polar-Express update.
__constant__ static const float kPEd[5][3] = {
    {8.156554524902461f, -22.48329292557795f / 15.878769915207462f, 15.878769915207462f / 8.156554524902461f},
    {4.042929935166739f, -2.808917465908714f / 0.5000178451051316f, 0.5000178451051316f / 4.042929935166739f},
    {3.8916678022926607f, -2.772484153217685f / 0.5060648178503393f, 0.5060648178503393f / 3.8916678022926607f},
    {3.285753657755655f, -2.3681294933425376f / 0.46449024233003106f, 0.46449024233003106f / 3.285753657755655f},
    {2.3465413258596377f, -1.7097828382687081f / 0.42323551169305323f, 0.42323551169305323f / 2.3465413258596377f},
};

// Scaled fp16 Polar-Express (polar_express_wave_t): the iterate is carried
// as X_s = X / tau_st with tau_0 = 1/32 and tau_{st+1} = a_st tau_st, so the
// update X_s <- X_s + (B/a) X_s needs no a X multiply.  With G = X_s X_s^T:
// R = kappa G + G^2 and B/a = rho R, kappa = b / (c tau^2), rho = c tau^4 / a.
__constant__ static const float kPEt[5][2] = {
    {-1449.9165916965815f, 1.8565651707500468e-06f},
    {-86.464919938170382f, 0.00052205510948284965f},
    {-5.1588982945329462f, 0.1466500805871209f},
    {-0.31699423815939715f, 36.567608739989502f},
    {-0.023265445343007344f, 5438.1209129926056f},
};
// tau after ns steps (P = tau_ns X_s).
__constant__ static const float kPEtau[6] = {0.03125f, 0.2548923289032019f, 1.0305118267671212f,
                                             4.010409696111398f, 13.177218328096771f, 30.920887366754116f};

// acc += a * b on the matrix core with the accumulator in AGPRs.  (The
// compiler keeps a VGPR-form MFMA's accumulator in arch VGPRs; this form
// keeps long-lived accumulators out of the arch VGPR file.)  The compiler
// treats the asm as opaque and inserts no wait states around it, so they are
// provided here: two before the MFMA (its A/B operands are usually written by
// the VALU just before), agpr_init after the accumulators are zeroed (VALU
// writes of a SrcC), and agpr_mfma_drain before ordinary code reads acc.
__device__ __forceinline__ void agpr_mfma(f32x16& acc, f16x8 a, f16x8 b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Same with bf16 operands (fp32's exponent range).
__device__ __forceinline__ void agpr_mfma_bf16(f32x16& acc, bf16x8 a, bf16x8 b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Zeroes the accumulators and waits out the VALU-write -> MFMA-SrcC hazard.
template <int N>
__device__ __forceinline__ void agpr_init(f32x16 (&acc)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) acc[i] = zero16();
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+a"(acc[i]));
  asm volatile("s_nop 4" ::);
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+a"(acc[i]));
}
// Waits out the last agpr_mfma and pins every accumulator in acc after the
// wait, so that no read of them can be scheduled before it.
template <int N>
__device__ __forceinline__ void agpr_mfma_drain(f32x16 (&acc)[N]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::);
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+a"(acc[i]));
}

// Transposing LDS read (gfx950 ds_read_b64_tr_b16).  Within each group of 16
// lanes, lane i supplies the address of 4 consecutive 16-bit values; the
// group's 4x16 block comes back transposed: lane j receives element j % 4 of
// the values loaded by lanes 4k + j / 4, for k = 0..3.
typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 fp16x4_raw;
__device__ __forceinline__ f16x4 lds_read_tr16(const _Float16* p) {
  typedef __attribute__((address_space(3))) fp16x4_raw lds_fp16x4;
  const fp16x4_raw r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)(p));
  return __builtin_bit_cast(f16x4, r);
}

// Cross-lane reductions on the VALU instead of the LDS permute path: within
// 16-lane rows by DPP (quad_perm [1,0,3,2] and [2,3,0,1], then
// row_half_mirror and row_mirror -- a mirror pairs every lane with one of the
// other half once the halves hold their own reductions), across rows by
// gfx950's v_permlane16_swap / v_permlane32_swap of the value with itself (the
// two results hold, in every lane, the lane's own value and its partner's).
// Every lane of a group ends with the same bits (each pairwise step adds or
// compares the same two values).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// The lane's value and its partner's across 16-lane rows (XOR 16) or halves
// (XOR 32), in either order.  The swap exchanges rows between two registers,
// so the value is first copied into a second one (the asm keeps the compiler
// from folding the copy: a register swapped with itself only duplicates rows).
__device__ __forceinline__ void swap16(float x, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  unsigned v = u;
  asm volatile("" : "+v"(v));
  const auto r = __builtin_amdgcn_permlane16_swap(u, v, false, false);
  const unsigned r0 = r[0], r1 = r[1];   // (bit-casting the elements in place reads element 0 twice)
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void swap32(float x, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  unsigned v = u;
  asm volatile("" : "+v"(v));
  const auto r = __builtin_amdgcn_permlane32_swap(u, v, false, false);
  const unsigned r0 = r[0], r1 = r[1];   // (bit-casting the elements in place reads element 0 twice)
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
// Sum over each aligned group of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (G >= 2) x += dpp_f<0xB1>(x);
  if constexpr (G >= 4) x += dpp_f<0x4E>(x);
  if constexpr (G >= 8) x += dpp_f<0x141>(x);
  if constexpr (G >= 16) x += dpp_f<0x140>(x);
  float a, b;
  if constexpr (G >= 32) {
    swap16(x, a, b);
    x = a + b;
  }
  if constexpr (G >= 64) {
    swap32(x, a, b);
    x = a + b;
  }
  return x;
}
__device__ __forceinline__ float wave_sum(float x) { return group_sum<WAVE>(x); }
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f<0xB1>(x));
  x = fmaxf(x, dpp_f<0x4E>(x));
  x = fmaxf(x, dpp_f<0x141>(x));
  x = fmaxf(x, dpp_f<0x140>(x));
  float a, b;
  swap16(x, a, b);
  x = fmaxf(a, b);
  swap32(x, a, b);
  return fmaxf(a, b);
}

// Block-wide max over NW waves; `red` is an LDS array of >= NW floats.
template <int NW>
__device__ __forceinline__ float block_max(float x, float* red) {
  x = wave_max(x);
  __syncthreads();
  if (lane_id() == 0) red[wave_id()] = x;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = fmaxf(m, red[w]);
  return m;
}

// Block-wide maxima of two values with one barrier; `red` is an LDS array of
// >= 2 NW floats that no thread has read before the call.
template <int NW>
__device__ __forceinline__ void block_max2(float& x, float& y, float* red) {
  x = wave_max(x);
  y = wave_max(y);
  if (lane_id() == 0) {
    red[wave_id()] = x;
    red[NW + wave_id()] = y;
  }
  __syncthreads();
  x = red[0];
  y = red[NW];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    x = fmaxf(x, red[w]);
    y = fmaxf(y, red[NW + w]);
  }
}

// Power-of-two factor that brings max|x| = m into [1, 2); 1 for m == 0/inf/nan.
__device__ __forceinline__ float pow2_scale(float m) {
  if (!(m > 0.f) || !(m < 3.0e38f)) return 1.f;
  // capped at 2^126 so that a subnormal maximum cannot produce an infinite factor
  return ldexpf(1.f, min(-ilogbf(m), 126));
}

// GELU with the tanh approximation (jax.nn.gelu default, memory_layer.py:506,594).
// Evaluated through (1 + tanh(u)) / 2 = 1 / (1 + exp(-2u)), i.e. x * sigmoid(2u):
// one hardware exp and one reciprocal instead of tanhf (relative error of a
// few ulp; exp(-2u) -> inf for x << 0 gives -0, the limit).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  return __fdividef(x, 1.f + __expf(-2.f * u));
}
// Derivative of the exact erf GELU (memory_layer.py:225-230):
// Phi(x) + x phi(x).  Phi is evaluated branch-free with Abramowitz & Stegun
// 7.1.26 (|error of erf| <= 1.5e-7, so |error of Phi| <= 7.5e-8):
// erf(z) = 1 - (a1 t + ... + a5 t^5) exp(-z^2), t = 1 / (1 + p z), z >= 0,
// with z = |x| / sqrt(2); exp(-z^2) = exp(-x^2 / 2) is shared with phi.
__device__ __forceinline__ float gelu_erf_prime(float x) {
  const float ex = __expf(-0.5f * x * x);
  const float t = __frcp_rn(fmaf(0.3275911f * 0.7071067811865476f, fabsf(x), 1.f));
  float poly = 1.061405429f;
  poly = fmaf(poly, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f);
  const float tail = 0.5f * poly * t * ex;   // Phi(-|x|)
  const float cdf = (x >= 0.f) ? 1.f - tail : tail;
  return fmaf(x * 0.3989422804014327f, ex, cdf);
}

// Loads of the caller's activations/gates in any of the supported dtypes.
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dtype) {
  if (dtype == 0) return static_cast<const float*>(p)[i];
  if (dtype == 1) {
    const uint16_t u = static_cast<const uint16_t*>(p)[i];
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
  }
  return (float)static_cast<const _Float16*>(p)[i];
}
__device__ __forceinline__ void store_any(void* p, int64_t i, int dtype, float x) {
  if (dtype == 0) {
    static_cast<float*>(p)[i] = x;
  } else if (dtype == 1) {
    // round to nearest even
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u) {
      static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
      static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(u >> 16);
    }
  } else {
    static_cast<_Float16*>(p)[i] = (_Float16)x;
  }
}

// bf16 bits of x, round to nearest even (NaN/inf kept).
__device__ __forceinline__ uint16_t bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) return static_cast<uint16_t>((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Four consecutive elements at p[i..i+3] (i % 4 == 0, buffer 16-byte aligned).
__device__ __forceinline__ f32x4 load4_any(const void* p, int64_t i, int dtype) {
  if (dtype == 0) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  if (dtype == 1) {
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                 __uint_as_float(w.y & 0xffff0000u)};
  }
  const f16x4 h = *reinterpret_cast<const f16x4*>(static_cast<const _Float16*>(p) + i);
  return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}
__device__ __forceinline__ void store4_any(void* p, int64_t i, int dtype, f32x4 x) {
  if (dtype == 0) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = x;
  } else if (dtype == 1) {
    uint2 w;
    w.x = (uint32_t)bf16_bits(x[0]) | ((uint32_t)bf16_bits(x[1]) << 16);
    w.y = (uint32_t)bf16_bits(x[2]) | ((uint32_t)bf16_bits(x[3]) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = w;
  } else {
    *reinterpret_cast<f16x4*>(static_cast<_Float16*>(p) + i) =
        f16x4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
  }
}

}  // namespace atlas
