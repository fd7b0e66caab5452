// Event-based kernel timing used by measurement tools (bench.py).
#include "atlas_profile.hpp"

#include <mutex>
#include <vector>

#include "atlas_common.hpp"
#include "atlas_status.hpp"

namespace atlas {
namespace {

constexpr int KINDS = 6;
struct Rec {
  hipEvent_t a, b;
};
std::mutex mu;
bool enabled = false;
std::vector<Rec> recs[KINDS];
std::vector<hipEvent_t> pool;
hipEvent_t pending[KINDS];

hipEvent_t take() {
  if (!pool.empty()) {
    hipEvent_t e = pool.back();
    pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  // no system-scope release on record: the timed kernels exchange no data
  // with the host, and the fence would add several microseconds per event
  (void)hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
  return e;
}

}  // namespace

bool profile_on() { return enabled; }

void profile_begin(int kind, hipStream_t st) {
  if (!enabled) return;
  std::lock_guard<std::mutex> g(mu);
  hipEvent_t e = take();
  (void)hipEventRecord(e, st);
  pending[kind] = e;
}

void profile_end(int kind, hipStream_t st) {
  if (!enabled) return;
  std::lock_guard<std::mutex> g(mu);
  hipEvent_t e = take();
  (void)hipEventRecord(e, st);
  recs[kind].push_back({pending[kind], e});
}

// Matrix-core calibration: independent accumulator chains of the fp16 32x32x16
// MFMA the phase kernels use, with pseudo-random operands rotated every
// product (the part's power draw, and with it the sustained clock, depends on
// how many operand bits toggle: constant operands run far faster than real
// data).  Writes nothing unless `sink_flag` equals a value no caller passes,
// so that the products are not eliminated.
__global__ void __launch_bounds__(1024) mfma_rate_kernel(int iters, int sink_flag, float* sink) {
  f16x8 a[4], b[4];
  unsigned x = 2654435761u * (blockIdx.x * blockDim.x + threadIdx.x + 1);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x ^= x << 13;
      x ^= x >> 17;
      x ^= x << 5;
      a[j][i] = (_Float16)((float)(x & 0xffff) / 65536.f - 0.5f);
      x ^= x << 13;
      x ^= x >> 17;
      x ^= x << 5;
      b[j][i] = (_Float16)((float)(x & 0xffff) / 65536.f - 0.5f);
    }
  f32x16 acc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) acc[k] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k)
        acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[k], b[(k + u) & 3], acc[k], 0, 0, 0);
  }
  if (sink_flag == 0x5eed) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[k][r];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
  }
}

}  // namespace atlas

using namespace atlas;

extern "C" atlas_status atlas_profile_mfma_rate(int32_t waves_per_simd, double* tflops, void* stream) {
  clear_error();
  if (waves_per_simd < 1 || waves_per_simd > 4 || !tflops)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "waves_per_simd must be 1..4 and tflops non-NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return fail_hip(e, "device query");
  const int threads = 256 * waves_per_simd, iters = 12000;   // ~25 ms at the sustained rate
  hipEvent_t e0 = nullptr, e1 = nullptr;
  e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e != hipSuccess) return fail_hip(e, "hipEventCreate");
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus), dim3(threads), 0, st, iters / 8, 0, nullptr);   // clocks up
  (void)hipEventRecord(e0, st);
  hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus), dim3(threads), 0, st, iters, 0, nullptr);
  (void)hipEventRecord(e1, st);
  e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) return fail_hip(e, "mfma calibration timing");
  const double flops = (double)cus * threads / 64 * iters * 16.0 * 32 * 32 * 16 * 2;
  *tflops = flops / (ms * 1e-3) / 1e12;
  return ATLAS_OK;
}

extern "C" atlas_status atlas_profile_enable(int32_t enable) {
  clear_error();
  std::lock_guard<std::mutex> g(mu);
  for (auto& v : recs) {
    for (auto& r : v) {
      pool.push_back(r.a);
      pool.push_back(r.b);
    }
    v.clear();
  }
  enabled = enable != 0;
  return ATLAS_OK;
}

extern "C" atlas_status atlas_profile_read(int32_t kind, int64_t* launches, double* total_ms) {
  clear_error();
  if (kind < 0 || kind >= KINDS || !launches || !total_ms)
    return fail(ATLAS_ERR_INVALID_ARGUMENT, "bad profile query");
  std::lock_guard<std::mutex> g(mu);
  double tot = 0.0;
  for (auto& r : recs[kind]) {
    hipError_t e = hipEventSynchronize(r.b);
    if (e != hipSuccess) return fail_hip(e, "hipEventSynchronize");
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) return fail_hip(e, "hipEventElapsedTime");
    tot += ms;
  }
  *launches = (int64_t)recs[kind].size();
  *total_ms = tot;
  return ATLAS_OK;
}
