// Error state and version query of the C ABI.
#include "capi.hpp"

#include <atomic>

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

std::atomic<int> g_conv_variant{0};
std::atomic<int> g_attn_variant{0};

int max_lds_per_block() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        v <= 0)
      v = 64 * 1024;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace shrimp

extern "C" const char* shrimp_last_error(void) { return shrimp::g_last_error.c_str(); }

extern "C" int shrimp_abi_version(void) { return SHRIMP_ABI_VERSION; }

extern "C" int shrimp_conv_variant(int variant) {
  if (variant < 0 || variant > 3) return shrimp::g_conv_variant.load();
  return shrimp::g_conv_variant.exchange(variant);
}

extern "C" int shrimp_attn_variant(int variant) {
  if (variant < 0 || variant > 3) return shrimp::g_attn_variant.load();
  return shrimp::g_attn_variant.exchange(variant);
}

extern "C" int shrimp_max_lds_per_block(void) { return shrimp::max_lds_per_block(); }
