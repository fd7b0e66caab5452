// Opt-in per-kernel timing with HIP events (atlas_profile_enable/read).
#pragma once

#include <hip/hip_runtime.h>

namespace atlas {

bool profile_on();
// Records an event pair around one launch of `kind`; call begin() before the
// launch and end() after it.  No-ops when profiling is off.
void profile_begin(int kind, hipStream_t st);
void profile_end(int kind, hipStream_t st);

}  // namespace atlas
