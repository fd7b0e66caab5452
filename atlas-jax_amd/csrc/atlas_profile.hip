// Event-based kernel timing used by measurement tools (bench.py).
#include "atlas_profile.hpp"

#include <mutex>
#include <vector>

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

}  // namespace atlas

using namespace atlas;

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
