// Library-wide host helpers: device properties cache, error strings, ABI version.
#include <atomic>

#include "common.h"

namespace bytes_amd {

int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace bytes_amd

extern "C" {

const char* bytes_error_string(int code) { return hipGetErrorString(static_cast<hipError_t>(code)); }

int bytes_abi_version(void) { return 1; }

}  // extern "C"
