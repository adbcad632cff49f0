// Error reporting shared by every C-ABI entry point.
#include <cstdarg>

#include "common.hpp"

namespace gdn {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return GDN_OK;
  set_error("%s: %s", what, hipGetErrorString(err));
  return GDN_ERR_HIP;
}

}  // namespace gdn

extern "C" const char* gdn_last_error(void) { return gdn::g_last_error; }

extern "C" int gdn_abi_version(void) { return 6; }
