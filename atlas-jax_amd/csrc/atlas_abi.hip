// Library-wide C-ABI entry points: version and error message.
#include "atlas_status.hpp"

namespace atlas {

char* error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}

}  // namespace atlas

extern "C" const char* atlas_last_error(void) { return atlas::error_buffer(); }

extern "C" int32_t atlas_abi_version(void) { return ATLAS_ABI_VERSION; }
