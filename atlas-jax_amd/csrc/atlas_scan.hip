// Host side of the chunk scan: validation, workspace layout, launch sequence
// and the C-ABI entry points declared in include/atlas_scan.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>

#include "atlas_scan.h"
#include "atlas_scan_kernels.hpp"
#include "atlas_scan_phase16.hpp"
#include "atlas_scan_tail8.hpp"
#include "atlas_scan_wide.hpp"
#include "atlas_profile.hpp"
#include "atlas_status.hpp"

namespace atlas {

namespace {

struct Plan {
  int streams, nsl, ts, n_chunks, cw;
  size_t off_W1b, off_W2b, off_S1b, off_S2b, off_kT, off_errT, off_actT, off_chainT, off_L1, off_L2,
      off_hloc, off_yloc, off_g, off_cmt, off_cm, off_thp, off_ap, off_am, off_S1T, total_floats;
};

bool supported_de(int D, int E) {
  return (D == 32 && (E == 32 || E == 64 || E == 128)) || (D == 64 && (E == 64 || E == 128 || E == 256));
}

// Slices per chunk: nsl = cs / ts with ts in {32, 16, 8, 4}, ts | cs.  One
// phase workgroup occupies a CU (256 on MI355X), so a launch of streams*nsl
// workgroups runs in ceil(streams*nsl / 256) rounds of ts tokens each plus a
// fixed staging/epilogue cost (about two tokens' worth); the count with the
// smallest estimate wins, the larger ts on ties.
int choose_slices(int streams, int cs, int requested) {
  if (requested > 0) return requested;
  constexpr long long kCUs = 256, kFixed = 2;
  int best = 0;
  long long best_cost = 0;
  for (int ts = 32; ts >= 4; ts /= 2) {
    if (cs % ts) continue;
    const int nsl = cs / ts;
    if (nsl > NSL_MAX) continue;
    const long long rounds = ((long long)streams * nsl + kCUs - 1) / kCUs;
    const long long cost = rounds * (ts + kFixed);
    if (best == 0 || cost < best_cost) {
      best = nsl;
      best_cost = cost;
    }
  }
  return best;
}

// Workspace layout for a gate-table window of cw chunks.
void layout(const atlas_scan_desc* d, Plan* P) {
  const size_t S = P->streams, DE = (size_t)d->D * d->E, cs = d->chunk_size;
  const int nsl = P->nsl;
  size_t o = 0;
  auto take = [&](size_t n) { size_t r = o; o += (n + 63) & ~size_t(63); return r; };
  P->off_W1b = take(S * DE);
  P->off_W2b = take(S * DE);
  P->off_S1b = take(S * DE);
  P->off_S2b = take(S * DE);
  P->off_kT = take(S * cs * d->D);
  P->off_errT = take(S * cs * d->D);
  P->off_actT = take(S * cs * d->E);
  P->off_chainT = take(S * cs * d->E);
  P->off_L1 = take(S * nsl * DE);
  P->off_L2 = take(S * nsl * DE);
  P->off_hloc = take(S * cs * d->E);
  P->off_yloc = take(S * cs * d->D);
  P->off_g = take(S * cs * d->E);
  const size_t SC = S * (size_t)P->cw;   // gate-only tables of one window of chunks
  P->off_cmt = take(SC * cs * cs);
  P->off_am = take(SC * cs * cs);
  P->off_cm = take(SC * cs);
  P->off_thp = take(SC * cs);
  P->off_ap = take(SC * cs);
  P->off_S1T = d->E > 128 ? take(2 * S * DE) : 0;
  P->total_floats = o;
}

// Whether the phase and prep kernels of (M, D, E) fit a CU's 160 KiB of LDS
// at this chunk and slice size (the same layouts run_scan / run_scan_wide
// launch with); a shape that does not takes the generic forward.
template <class M, int D, int E>
bool lds_fits_de(int cs, int ts, int nsl) {
  constexpr size_t LDS_MAX = 160 * 1024;
  constexpr bool kF16 = sizeof(typename M::elem) == 2;
  const size_t prep_lds = prep_lds_bytes<D, E>();
  if constexpr (E > 128) {
    const WideLayout<D, E> L(cs, ts, nsl);
    return L.total <= WIDE_LDS_MAX && prep_lds <= WIDE_LDS_MAX;
  } else {
    const PhaseLayout<M, D, E> L(cs);
    const Phase16Layout<D, E> L16(cs, ts);
    const size_t phase_lds = kF16 ? L16.total : (L.total_lsh <= LDS_MAX ? L.total_lsh : L.total);
    return phase_lds <= LDS_MAX && prep_lds <= LDS_MAX;
  }
}
template <class M>
bool lds_fits_mode(int D, int E, int cs, int ts, int nsl) {
  if constexpr (sizeof(typename M::elem) == 2) {
    if (D == 64 && E == 256) return lds_fits_de<M, 64, 256>(cs, ts, nsl);
  }
  if (D == 32 && E == 32) return lds_fits_de<M, 32, 32>(cs, ts, nsl);
  if (D == 32 && E == 64) return lds_fits_de<M, 32, 64>(cs, ts, nsl);
  if (D == 32 && E == 128) return lds_fits_de<M, 32, 128>(cs, ts, nsl);
  if (D == 64 && E == 64) return lds_fits_de<M, 64, 64>(cs, ts, nsl);
  if (D == 64 && E == 128) return lds_fits_de<M, 64, 128>(cs, ts, nsl);
  return false;
}

// Validates the descriptor and lays out the workspace.  The gate tables are
// held for a window of cw chunks, cw chosen so that one coef launch fills the
// GPU once (256 CUs times the blocks that fit a CU's LDS): the workspace then
// depends on B*H, D, E and cs but not on T.  With ws_cap > 0 the window is
// shrunk until the workspace fits ws_cap bytes (error if even one chunk's
// tables do not fit).
atlas_status make_plan(const atlas_scan_desc* d, Plan* P, size_t ws_cap = 0) {
  if (!d) return fail(ATLAS_ERR_INVALID_ARGUMENT, "desc is NULL");
  if (d->B < 1 || d->T < 1 || d->H < 1)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "B, T, H must be >= 1 (got %d, %d, %d)", d->B, d->T, d->H);
  if (!supported_de(d->D, d->E))
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE,
                "(D, E) = (%d, %d) not compiled; supported: D=32 with E in {32,64,128}, D=64 with E in "
                "{64,128,256}", d->D, d->E);
  if (d->E > 128 && d->compute != ATLAS_COMPUTE_F16)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "E = %d runs with fp16 matrix-core operands only (compute F16)", d->E);
  if (d->chunk_size < 4 || d->chunk_size > CS_MAX || d->chunk_size % 4)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "chunk_size %d must be a multiple of 4 in [4, %d]",
                d->chunk_size, CS_MAX);
  if (d->ns_steps < 0 || d->ns_steps > 5)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "ns_steps %d outside [0, 5]", d->ns_steps);
  if (d->io_dtype < 0 || d->io_dtype > 2 || d->gate_dtype < 0 || d->gate_dtype > 2)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad dtype (io %d, gate %d)", d->io_dtype, d->gate_dtype);
  if (d->compute != ATLAS_COMPUTE_F32 && d->compute != ATLAS_COMPUTE_F16)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad compute mode %d", d->compute);
  if (d->omega_window < 0) return fail(ATLAS_ERR_INVALID_ARGUMENT, "omega_window < 0");
  if ((d->x_stride_b | d->x_stride_t | d->x_stride_h) & 7)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "q/k/v/y strides must be multiples of 8 elements (vector loads)");
  const long long streams = (long long)d->B * d->H;
  if (streams > (1LL << 24)) return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "B*H too large");
  const int cs = d->chunk_size;
  const int nsl = choose_slices((int)streams, cs, d->n_slices);
  if (nsl < 1 || cs % nsl || nsl > NSL_MAX)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "n_slices %d does not divide chunk_size %d (max %d)", nsl, cs, NSL_MAX);
  const int ts = cs / nsl;
  if (ts % NW || ts > TS_MAX)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "tokens per slice %d must be a multiple of %d and <= %d", ts, NW,
                TS_MAX);
  const bool fits = d->compute == ATLAS_COMPUTE_F16 ? lds_fits_mode<ModeF16>(d->D, d->E, cs, ts, nsl)
                                                    : lds_fits_mode<ModeF32>(d->D, d->E, cs, ts, nsl);
  if (!fits)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "chunk_size %d (%d slices) needs more than 160 KiB of LDS in compute "
                "mode %d at D %d, E %d", cs, nsl, d->compute, d->D, d->E);
  P->streams = (int)streams;
  P->nsl = nsl;
  P->ts = ts;
  P->n_chunks = (d->T + cs - 1) / cs;
  const long long per_cu = std::max<long long>(1, (long long)(160 * 1024) / (long long)coef_lds_bytes(cs));
  const long long round = 256 * per_cu;
  P->cw = (int)std::min<long long>(P->n_chunks, std::max<long long>(1, (round + streams - 1) / streams));
  layout(d, P);
  while (ws_cap > 0 && P->total_floats * sizeof(float) > ws_cap && P->cw > 1) {
    P->cw = (P->cw + 1) / 2;
    layout(d, P);
  }
  if (ws_cap > 0 && P->total_floats * sizeof(float) > ws_cap)
    return fail(ATLAS_ERR_WORKSPACE, "scan needs %zu bytes of workspace, more than the %zu available",
                P->total_floats * sizeof(float), ws_cap);
  return ATLAS_OK;
}

template <class K>
hipError_t allow_lds(K kernel, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// A chunk-start state into the trace in one launch: the four n-float arrays
// (n a multiple of 4, 16-byte aligned; a null source is skipped) to dst +
// k n, k = 0..3 (four separate copies cost ~4x the launch gaps).
__global__ void __launch_bounds__(256) trace_copy_kernel(const float* s0, const float* s1, const float* s2,
                                                         const float* s3, float* dst, long long n4) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < 4 * n4; i += stride) {
    const int k = (int)(i / n4);
    const float* s = k == 0 ? s0 : k == 1 ? s1 : k == 2 ? s2 : s3;
    if (s) reinterpret_cast<f32x4*>(dst)[i] = reinterpret_cast<const f32x4*>(s)[i - k * n4];
  }
}
void launch_trace_copy(const float* s0, const float* s1, const float* s2, const float* s3, float* dst, size_t n,
                       hipStream_t st) {
  const long long n4 = (long long)(n / 4), blocks = std::min<long long>((4 * n4 + 255) / 256, 4096);
  hipLaunchKernelGGL(trace_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, st, s0, s1, s2, s3, dst, n4);
}

// Gate tables of the window of chunks starting at c0 (the previous window's
// tables are no longer read: every launch is on the same stream).
void launch_coef(const ScanArgs& a, const Plan& P, int c0, hipStream_t st) {
  const int nwin = std::min(P.cw, P.n_chunks - c0);
  hipLaunchKernelGGL(coef_kernel, dim3(P.streams * nwin), coef_block(a.cs), coef_lds_bytes(a.cs), st, a, c0, nwin);
}

template <class M, int D, int E>
atlas_status run_scan(const ScanArgs& base, const Plan& P, hipStream_t st) {
  constexpr bool kF16 = sizeof(typename M::elem) == 2;
  constexpr size_t LDS_MAX = 160 * 1024;
  const size_t prep_lds = prep_lds_bytes<D, E>();
  // fp16 mode: phase16_kernel (AGPR accumulation, LDS-transpose Polar-Express);
  // fp32 mode: phase_kernel, accumulating the slice memory partial in LDS
  // (exact fp32) when it fits, else in registers through an identity MFMA
  const PhaseLayout<M, D, E> L(base.cs);
  const Phase16Layout<D, E> L16(base.cs, base.ts);
  const bool lsh = L.total_lsh <= LDS_MAX;
  const size_t phase_lds = kF16 ? L16.total : (lsh ? L.total_lsh : L.total);
  if (phase_lds > LDS_MAX || prep_lds > LDS_MAX)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "LDS need %zu / %zu bytes exceeds 160 KiB", phase_lds, prep_lds);
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  static size_t tail_static = LDS_MAX;   // static LDS of tail_kernel (its finalize part)
  std::call_once(once, [&] {
    hipError_t e = allow_lds(prep_kernel<D, E>, prep_lds_bytes<D, E>());
    if (e == hipSuccess) e = allow_lds(coef_kernel, coef_lds_bytes());
    hipFuncAttributes fa;
    if (e == hipSuccess) e = hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(tail_kernel<M, D, E>));
    if (e == hipSuccess) {
      tail_static = fa.sharedSizeBytes;
      if (tail_static + prep_lds_bytes<D, E>() <= LDS_MAX) e = allow_lds(tail_kernel<M, D, E>, prep_lds_bytes<D, E>());
    }
    if constexpr (D == 64 && E <= 128) {
      if (e == hipSuccess) e = allow_lds(tail8_kernel<M, D, E>, Prep8L<D, E>::bytes());
    }
    if constexpr (kF16) {
      if (e == hipSuccess) e = allow_lds(phase16_kernel<D, E, 2>, LDS_MAX);
      if (e == hipSuccess) e = allow_lds(phase16_kernel<D, E, 1>, LDS_MAX);
    } else {
      if (e == hipSuccess) e = allow_lds(phase_kernel<M, D, E, 2, true>, LDS_MAX);
      if (e == hipSuccess) e = allow_lds(phase_kernel<M, D, E, 1, true>, LDS_MAX);
      if (e == hipSuccess) e = allow_lds(phase_kernel<M, D, E, 2, false>, LDS_MAX);
      if (e == hipSuccess) e = allow_lds(phase_kernel<M, D, E, 1, false>, LDS_MAX);
    }
    attr_err = e;
  });
  if (attr_err != hipSuccess) return fail_hip(attr_err, "hipFuncSetAttribute");

  ScanArgs a = base;
  const int nblk = (a.cs + 31) / 32;
  const dim3 pgrid(P.streams * P.nsl), pblock(NTHREADS);
  auto phase = [&](auto mat) {
    constexpr int MAT = decltype(mat)::value;
    if constexpr (kF16) {
      hipLaunchKernelGGL((phase16_kernel<D, E, MAT>), pgrid, pblock, phase_lds, st, a);
    } else if (lsh) {
      hipLaunchKernelGGL((phase_kernel<M, D, E, MAT, true>), pgrid, pblock, phase_lds, st, a);
    } else {
      hipLaunchKernelGGL((phase_kernel<M, D, E, MAT, false>), pgrid, pblock, phase_lds, st, a);
    }
  };
  // The next chunk's prep and this chunk's y are independent once W_end is
  // formed, so they share one launch (tail_kernel).  W_end comes from the
  // slice-prefix kernels when there are more than 4 slices, else from its
  // own launch (fin_wend_kernel).
  const bool tail = tail_static + prep_lds <= LDS_MAX;
  // D = 64, E <= 128 with the slice partials summed directly: the tail on
  // eight-wave blocks whose prep forms W_end itself (atlas_scan_tail8.hpp),
  // no W_end launch; the last chunk's W_end and y take fin_kernel
  const bool tail8 = (D == 64 && E <= 128) && !a.use_prefix;
  for (int c = 0; c < P.n_chunks; ++c) {
    a.chunk = c;
    a.cur = c & 1;
    if (a.trace) {   // this chunk's start state, after the previous chunk's kernels (stream order)
      const size_t n = (size_t)P.streams * D * E;
      float* dst = a.trace + (size_t)c * 4 * n;
      launch_trace_copy(a.W1[a.cur], a.W2[a.cur], a.S1[a.cur], a.S2[a.cur], dst, n, st);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return fail_hip(e, "state trace copy");
    }
    if (c % P.cw == 0) launch_coef(a, P, c, st);
    if (!(tail || tail8) || c == 0) {
      profile_begin(ATLAS_KERNEL_PREP, st);
      hipLaunchKernelGGL((prep_kernel<D, E>), dim3(P.streams * nblk), dim3(NTHREADS), prep_lds, st, a);
      profile_end(ATLAS_KERNEL_PREP, st);
    }
    profile_begin(ATLAS_KERNEL_PHASE2, st);
    phase(std::integral_constant<int, 2>{});
    profile_end(ATLAS_KERNEL_PHASE2, st);
    if (a.use_prefix) {
      profile_begin(ATLAS_KERNEL_PREFIX, st);
      hipLaunchKernelGGL((prefix_kernel<D, E>), dim3(P.streams * kPrefixParts<D, E>), dim3(NTHREADS), 0, st, a, 2);
      profile_end(ATLAS_KERNEL_PREFIX, st);
    }
    profile_begin(ATLAS_KERNEL_PHASE1, st);
    phase(std::integral_constant<int, 1>{});
    profile_end(ATLAS_KERNEL_PHASE1, st);
    if (a.use_prefix) {
      profile_begin(ATLAS_KERNEL_PREFIX, st);
      hipLaunchKernelGGL((prefix_kernel<D, E>), dim3(P.streams * kPrefixParts<D, E>), dim3(NTHREADS), 0, st, a, 1);
      profile_end(ATLAS_KERNEL_PREFIX, st);
    }
    if constexpr (D == 64 && E <= 128) {
      if (tail8) {
        if (c + 1 < P.n_chunks) {
          ScanArgs an = a;
          an.chunk = c + 1;
          an.cur = (c + 1) & 1;
          const int n_prep = P.streams * nblk, n_y = P.streams * ((P.nsl + 1) / 2);
          profile_begin(ATLAS_KERNEL_TAIL, st);
          hipLaunchKernelGGL((tail8_kernel<M, D, E>), dim3(n_prep + n_y), dim3(NT8), (Prep8L<D, E>::bytes()), st, an,
                             n_prep);
          profile_end(ATLAS_KERNEL_TAIL, st);
        } else {
          profile_begin(ATLAS_KERNEL_FIN, st);
          hipLaunchKernelGGL((fin_kernel<M, D, E>), dim3(P.streams * P.nsl), dim3(NTHREADS), 0, st, a);
          profile_end(ATLAS_KERNEL_FIN, st);
        }
        continue;
      }
    }
    if (tail) {
      if (!a.use_prefix) {
        profile_begin(ATLAS_KERNEL_FIN, st);
        hipLaunchKernelGGL((fin_wend_kernel<M, D, E>), dim3(P.streams * P.nsl), dim3(NTHREADS), 0, st, a);
        profile_end(ATLAS_KERNEL_FIN, st);
      }
      ScanArgs an = a;
      an.chunk = c + 1;
      an.cur = (c + 1) & 1;
      const int n_prep = (c + 1 < P.n_chunks) ? P.streams * nblk : 0;
      // one slice per finalize block: a block holds the prep's LDS (63 KiB
      // at D64 E128) and 142 VGPRs per lane, so two blocks share a CU and
      // the y blocks run beside the prep blocks instead of after each other
      // (C2: 14.4 us per tail launch instead of 15.4 with two slices per block)
      const int per = 1, n_fin = P.streams * P.nsl;
      profile_begin(ATLAS_KERNEL_TAIL, st);
      hipLaunchKernelGGL((tail_kernel<M, D, E>), dim3(n_prep + n_fin), dim3(NTHREADS), n_prep > 0 ? prep_lds : 0, st,
                         an, n_prep, per);
      profile_end(ATLAS_KERNEL_TAIL, st);
    } else {
      profile_begin(ATLAS_KERNEL_FIN, st);
      hipLaunchKernelGGL((fin_kernel<M, D, E>), dim3(P.streams * P.nsl), dim3(NTHREADS), 0, st, a);
      profile_end(ATLAS_KERNEL_FIN, st);
    }
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "kernel launch");
  return ATLAS_OK;
}

// Wide memories (E > 128): prep with sequential weight staging, the pair
// phase kernels, the common finalize kernel.
template <int D, int E>
atlas_status run_scan_wide(const ScanArgs& base, const Plan& P, hipStream_t st) {
  using M = ModeF16;
  const WideLayout<D, E> L(base.cs, base.ts, base.nsl);
  const size_t prep_lds = prep_lds_bytes<D, E>();
  constexpr size_t LDS_MAX = WIDE_LDS_MAX;
  if (L.total > LDS_MAX || prep_lds > LDS_MAX)
    return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "LDS need %zu / %zu bytes exceeds 160 KiB", L.total, prep_lds);
  static std::once_flag once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(once, [&] {
    hipError_t e = allow_lds(prep_kernel<D, E>, prep_lds_bytes<D, E>());
    if (e == hipSuccess) e = allow_lds(coef_kernel, coef_lds_bytes());
    if (e == hipSuccess) e = allow_lds(phase_wide_kernel<D, E, 2, false, true>, LDS_MAX);
    if (e == hipSuccess) e = allow_lds(phase_wide_kernel<D, E, 1, false, true>, LDS_MAX);
    if (e == hipSuccess) e = allow_lds(phase_wide_kernel<D, E, 2, false, false>, LDS_MAX);
    if (e == hipSuccess) e = allow_lds(phase_wide_kernel<D, E, 1, false, false>, LDS_MAX);
    if (e == hipSuccess) e = allow_lds(phase_wide_kernel<D, E, 2, true, false>, LDS_MAX);
    if (e == hipSuccess) e = allow_lds(phase_wide_kernel<D, E, 1, true, false>, LDS_MAX);
    attr_err = e;
  });
  if (attr_err != hipSuccess) return fail_hip(attr_err, "hipFuncSetAttribute");

  ScanArgs a = base;
  const int nblk = (a.cs + 31) / 32;
  const dim3 grid(P.streams * P.nsl), block(NTHREADS);
  const dim3 tgrid(P.streams * (D / 32) * (E / 32));
  hipLaunchKernelGGL((transpose_kernel<D, E>), tgrid, dim3(256), 0, st, a.S1[0], a.S1T[0]);
  for (int c = 0; c < P.n_chunks; ++c) {
    a.chunk = c;
    a.cur = c & 1;
    if (a.trace) {   // this chunk's start state in the callers' layouts (S1 from its [e][d] copy)
      const size_t n = (size_t)P.streams * D * E;
      float* dst = a.trace + (size_t)c * 4 * n;
      launch_trace_copy(a.W1[a.cur], a.W2[a.cur], nullptr, a.S2[a.cur], dst, n, st);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return fail_hip(e, "state trace copy");
      hipLaunchKernelGGL((transpose_kernel<E, D>), tgrid, dim3(256), 0, st, a.S1T[a.cur], dst + 2 * n);
    }
    if (c % P.cw == 0) launch_coef(a, P, c, st);
    profile_begin(ATLAS_KERNEL_PREP, st);
    hipLaunchKernelGGL((prep_kernel<D, E>), dim3(P.streams * nblk), dim3(NTHREADS), prep_lds, st, a);
    profile_end(ATLAS_KERNEL_PREP, st);
    profile_begin(ATLAS_KERNEL_PHASE2, st);
    if (L.seq) hipLaunchKernelGGL((phase_wide_kernel<D, E, 2, true, false>), grid, block, L.total, st, a);
    else if (L.s0l) hipLaunchKernelGGL((phase_wide_kernel<D, E, 2, false, true>), grid, block, L.total, st, a);
    else hipLaunchKernelGGL((phase_wide_kernel<D, E, 2, false, false>), grid, block, L.total, st, a);
    profile_end(ATLAS_KERNEL_PHASE2, st);
    if (a.use_prefix) {
      profile_begin(ATLAS_KERNEL_PREFIX, st);
      hipLaunchKernelGGL((prefix_kernel<D, E>), dim3(P.streams * kPrefixParts<D, E>), dim3(NTHREADS), 0, st, a, 2);
      profile_end(ATLAS_KERNEL_PREFIX, st);
    }
    profile_begin(ATLAS_KERNEL_PHASE1, st);
    if (L.seq) hipLaunchKernelGGL((phase_wide_kernel<D, E, 1, true, false>), grid, block, L.total, st, a);
    else if (L.s0l) hipLaunchKernelGGL((phase_wide_kernel<D, E, 1, false, true>), grid, block, L.total, st, a);
    else hipLaunchKernelGGL((phase_wide_kernel<D, E, 1, false, false>), grid, block, L.total, st, a);
    profile_end(ATLAS_KERNEL_PHASE1, st);
    if (a.use_prefix) {
      profile_begin(ATLAS_KERNEL_PREFIX, st);
      hipLaunchKernelGGL((prefix_kernel<D, E>), dim3(P.streams * kPrefixParts<D, E>), dim3(NTHREADS), 0, st, a, 1);
      profile_end(ATLAS_KERNEL_PREFIX, st);
    }
    profile_begin(ATLAS_KERNEL_FIN, st);
    hipLaunchKernelGGL((fin_kernel<M, D, E>), grid, block, 0, st, a);
    profile_end(ATLAS_KERNEL_FIN, st);
  }
  // the final S1 lives in its transposed copy: back into the caller's buffer
  hipLaunchKernelGGL((transpose_kernel<E, D>), tgrid, dim3(256), 0, st, a.S1T[P.n_chunks & 1], a.S1[0]);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, "kernel launch");
  return ATLAS_OK;
}

template <class M>
atlas_status dispatch_de(int D, int E, const ScanArgs& a, const Plan& P, hipStream_t st) {
  if constexpr (sizeof(typename M::elem) == 2) {
    if (D == 64 && E == 256) return run_scan_wide<64, 256>(a, P, st);
  }
  if (D == 32 && E == 32) return run_scan<M, 32, 32>(a, P, st);
  if (D == 32 && E == 64) return run_scan<M, 32, 64>(a, P, st);
  if (D == 32 && E == 128) return run_scan<M, 32, 128>(a, P, st);
  if (D == 64 && E == 64) return run_scan<M, 64, 64>(a, P, st);
  if (D == 64 && E == 128) return run_scan<M, 64, 128>(a, P, st);
  return fail(ATLAS_ERR_UNSUPPORTED_SHAPE, "(D, E) = (%d, %d) not compiled", D, E);
}

}  // namespace
}  // namespace atlas

using namespace atlas;

namespace atlas {
// The generic forward (csrc/atlas_scan_bwd.hip): the shapes and chunk sizes
// the phase kernels are not built for.
bool generic_fwd_supported(const atlas_scan_desc* d);
size_t generic_fwd_workspace(const atlas_scan_desc* d);
atlas_status generic_fwd(const atlas_scan_desc* d, const void* q, const void* k, const void* v, const void* alpha,
                         const void* eta, const void* theta, const void* gamma, float* W1, float* W2, float* S1,
                         float* S2, void* y, float* trace, void* workspace, hipStream_t st);

namespace {
atlas_status generic_entry(const atlas_scan_desc* d, const void* q, const void* k, const void* v, const void* alpha,
                           const void* eta, const void* theta, const void* gamma, float* W1, float* W2, float* S1,
                           float* S2, void* y, float* trace, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (!q || !k || !v || !alpha || !eta || !theta || !W1 || !W2 || !S1 || !S2 || !y)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL tensor pointer (only gamma may be NULL)");
  const size_t need = generic_fwd_workspace(d);
  if (!workspace || workspace_bytes < need)
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes, need);
  auto mis = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; };
  if (mis(W1) || mis(W2) || mis(S1) || mis(S2) || mis(trace) || mis(workspace))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "the states, the trace and the workspace must be 16-byte aligned");
  return generic_fwd(d, q, k, v, alpha, eta, theta, gamma, W1, W2, S1, S2, y, trace, workspace,
                     static_cast<hipStream_t>(stream));
}
}  // namespace
}  // namespace atlas

extern "C" size_t atlas_scan_workspace_size(const atlas_scan_desc* desc) {
  Plan P;
  const atlas_status s = make_plan(desc, &P);
  if (s != ATLAS_OK) {
    if (s != ATLAS_ERR_UNSUPPORTED_SHAPE || !generic_fwd_supported(desc)) return 0;
    clear_error();
    return generic_fwd_workspace(desc);
  }
  return P.total_floats * sizeof(float);
}

namespace atlas {
namespace {

// Scratch of the allocation-free entry point: a file-scope device array, one
// copy per GPU, addressed from the host through the pointer that
// hipGetSymbolAddress returns on that GPU (the array's name is a host-side
// stand-in that must never reach a kernel or a copy).
constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's scratch (looked up once per device, with that
// device current).
atlas_status scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(ATLAS_ERR_INVALID_ARGUMENT, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(ATLAS_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ATLAS_OK;
}

bool misaligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

// The chunk loop for a validated plan and a workspace of at least
// P.total_floats floats (shared by both entry points).
atlas_status scan_fwd_impl(const atlas_scan_desc* d, const Plan& P, const void* q, const void* k, const void* v,
                           const void* alpha, const void* eta, const void* theta, const void* gamma, float* W1,
                           float* W2, float* S1, float* S2, void* y, void* workspace, void* stream,
                           float* trace = nullptr) {
  if (!q || !k || !v || !alpha || !eta || !theta || !W1 || !W2 || !S1 || !S2 || !y)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL tensor pointer (only gamma may be NULL)");
  // q/k/v/y rows and the state are read and written with 16-byte vector
  // accesses
  if (misaligned16(q) || misaligned16(k) || misaligned16(v) || misaligned16(y))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "q, k, v and y must be 16-byte aligned");
  if (misaligned16(W1) || misaligned16(W2) || misaligned16(S1) || misaligned16(S2))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "W1, W2, S1 and S2 must be 16-byte aligned");
  if (misaligned16(workspace)) return fail(ATLAS_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  const long long D = d->D, H = d->H, T = d->T;
  ScanArgs a;
  std::memset(&a, 0, sizeof(a));
  a.B = d->B; a.T = d->T; a.H = d->H; a.D = d->D; a.E = d->E;
  a.cs = d->chunk_size;
  a.use_omega = (d->omega_window > 1 && gamma != nullptr) ? 1 : 0;
  a.w_eff = a.use_omega ? d->omega_window : 1;
  a.ns = d->ns_steps;
  a.nsl = P.nsl; a.ts = P.ts; a.n_chunks = P.n_chunks; a.cw = P.cw;
  // cross-slice sums: direct for few slices (fewer launches), through the
  // slice-prefix kernel when their count would grow quadratically
  a.use_prefix = P.nsl > 4 ? 1 : 0;
  a.io_dtype = d->io_dtype; a.gate_dtype = d->gate_dtype;
  a.xsh = d->x_stride_h ? d->x_stride_h : D;
  a.xst = d->x_stride_t ? d->x_stride_t : H * D;
  a.xsb = d->x_stride_b ? d->x_stride_b : T * H * D;
  a.gst = d->g_stride_t ? d->g_stride_t : H;
  a.gsb = d->g_stride_b ? d->g_stride_b : T * H;
  a.q = q; a.k = k; a.v = v; a.alpha = alpha; a.eta = eta; a.theta = theta; a.gamma = gamma;
  a.y = y;
  float* ws = static_cast<float*>(workspace);
  a.W1[0] = W1; a.W1[1] = ws + P.off_W1b;
  a.W2[0] = W2; a.W2[1] = ws + P.off_W2b;
  a.S1[0] = S1; a.S1[1] = ws + P.off_S1b;
  a.S2[0] = S2; a.S2[1] = ws + P.off_S2b;
  a.kT = ws + P.off_kT; a.errT = ws + P.off_errT; a.actT = ws + P.off_actT; a.chainT = ws + P.off_chainT;
  a.cmt = ws + P.off_cmt; a.cm = ws + P.off_cm; a.thp = ws + P.off_thp; a.ap = ws + P.off_ap; a.am = ws + P.off_am;
  a.L1 = ws + P.off_L1; a.L2 = ws + P.off_L2;
  a.hloc = ws + P.off_hloc; a.yloc = ws + P.off_yloc; a.g = ws + P.off_g;
  a.trace = trace;
  a.S1T[0] = d->E > 128 ? ws + P.off_S1T : nullptr;
  a.S1T[1] = d->E > 128 ? ws + P.off_S1T + (size_t)P.streams * d->D * d->E : nullptr;

  hipStream_t st = static_cast<hipStream_t>(stream);
  atlas_status s = (d->compute == ATLAS_COMPUTE_F16) ? dispatch_de<ModeF16>(d->D, d->E, a, P, st)
                                                     : dispatch_de<ModeF32>(d->D, d->E, a, P, st);
  if (s != ATLAS_OK) return s;
  if (P.n_chunks & 1) {
    // final state landed in the workspace copies
    const size_t bytes = (size_t)P.streams * d->D * d->E * sizeof(float);
    hipError_t e = hipMemcpyAsync(W1, a.W1[1], bytes, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(W2, a.W2[1], bytes, hipMemcpyDeviceToDevice, st);
    // (wide memories: S1 was already written back from its transposed copy)
    if (e == hipSuccess && d->E <= 128) e = hipMemcpyAsync(S1, a.S1[1], bytes, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(S2, a.S2[1], bytes, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return fail_hip(e, "state copy-back");
  }
  return ATLAS_OK;
}

}  // namespace
}  // namespace atlas

extern "C" atlas_status atlas_scan_fwd(const atlas_scan_desc* d, const void* q, const void* k,
                                       const void* v, const void* alpha, const void* eta,
                                       const void* theta, const void* gamma, float* W1, float* W2,
                                       float* S1, float* S2, void* y, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  clear_error();
  Plan P;
  atlas_status s = make_plan(d, &P);
  if (s != ATLAS_OK) {
    if (s == ATLAS_ERR_UNSUPPORTED_SHAPE && generic_fwd_supported(d))
      return generic_entry(d, q, k, v, alpha, eta, theta, gamma, W1, W2, S1, S2, y, nullptr, workspace,
                           workspace_bytes, stream);
    return s;
  }
  if (!q || !k || !v || !alpha || !eta || !theta || !W1 || !W2 || !S1 || !S2 || !y)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL tensor pointer (only gamma may be NULL)");
  if (!workspace || workspace_bytes < P.total_floats * sizeof(float))
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes,
                P.total_floats * sizeof(float));
  return scan_fwd_impl(d, P, q, k, v, alpha, eta, theta, gamma, W1, W2, S1, S2, y, workspace, stream);
}

extern "C" atlas_status atlas_scan_fwd_trace(const atlas_scan_desc* d, const void* q, const void* k,
                                             const void* v, const void* alpha, const void* eta,
                                             const void* theta, const void* gamma, float* W1, float* W2,
                                             float* S1, float* S2, void* y, float* state_trace, void* workspace,
                                             size_t workspace_bytes, void* stream) {
  clear_error();
  Plan P;
  atlas_status s = make_plan(d, &P);
  if (!state_trace || misaligned16(state_trace))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "state_trace must be a non-NULL 16-byte aligned pointer");
  if (s == ATLAS_ERR_UNSUPPORTED_SHAPE && generic_fwd_supported(d))
    return generic_entry(d, q, k, v, alpha, eta, theta, gamma, W1, W2, S1, S2, y, state_trace, workspace,
                         workspace_bytes, stream);
  if (s != ATLAS_OK) return s;
  if (!state_trace || misaligned16(state_trace))
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "state_trace must be a non-NULL 16-byte aligned pointer");
  if (!q || !k || !v || !alpha || !eta || !theta || !W1 || !W2 || !S1 || !S2 || !y)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "NULL tensor pointer (only gamma may be NULL)");
  if (!workspace || workspace_bytes < P.total_floats * sizeof(float))
    return fail(ATLAS_ERR_WORKSPACE, "workspace %zu bytes < required %zu", workspace_bytes,
                P.total_floats * sizeof(float));
  return scan_fwd_impl(d, P, q, k, v, alpha, eta, theta, gamma, W1, W2, S1, S2, y, workspace, stream, state_trace);
}

extern "C" size_t atlas_scan_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" atlas_status atlas_scan_fwd_noalloc(const atlas_scan_desc* d, const void* q, const void* k,
                                               const void* v, const void* alpha, const void* eta,
                                               const void* theta, const void* gamma, float* W1, float* W2,
                                               float* S1, float* S2, void* y, void* stream) {
  clear_error();
  Plan P;
  atlas_status s = make_plan(d, &P, kScratchBytes);
  if (s != ATLAS_OK) return s;
  void* ws = nullptr;
  s = scratch_ptr(&ws);
  if (s != ATLAS_OK) return s;
  return scan_fwd_impl(d, P, q, k, v, alpha, eta, theta, gamma, W1, W2, S1, S2, y, ws, stream);
}
