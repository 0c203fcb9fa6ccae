// Error state and version query of the C ABI.
#include "capi.hpp"

namespace shrimp {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

}  // namespace shrimp

extern "C" const char* shrimp_last_error(void) { return shrimp::g_last_error.c_str(); }

extern "C" int shrimp_abi_version(void) { return SHRIMP_ABI_VERSION; }
