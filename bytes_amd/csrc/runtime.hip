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

// Kernel timing hook: when a caller has set a (start, stop) event pair for a
// kernel family, the entry points of that family launch their main kernel
// with that pair (hipExtLaunchKernel stamps it with the dispatch's own start
// and end), or, for the multi-kernel top-k, record it around their launches.
// Used by the benchmark to time the dominant kernel of a step with HIP
// events; no effect otherwise.
static std::atomic<hipEvent_t> g_prof_start{nullptr};
static std::atomic<hipEvent_t> g_prof_stop{nullptr};
static std::atomic<int> g_prof_family{0};

void prof_begin(int family, hipStream_t st) {
  if (g_prof_family.load(std::memory_order_relaxed) != family) return;
  hipEvent_t e = g_prof_start.load(std::memory_order_relaxed);
  if (e) (void)hipEventRecord(e, st);
}

void prof_end(int family, hipStream_t st) {
  if (g_prof_family.load(std::memory_order_relaxed) != family) return;
  hipEvent_t e = g_prof_stop.load(std::memory_order_relaxed);
  if (e) (void)hipEventRecord(e, st);
}

bool prof_events(int family, hipEvent_t* start, hipEvent_t* stop) {
  if (g_prof_family.load(std::memory_order_relaxed) != family) return false;
  *start = g_prof_start.load(std::memory_order_relaxed);
  *stop = g_prof_stop.load(std::memory_order_relaxed);
  return *start && *stop;
}

}  // namespace bytes_amd

extern "C" {

int bytes_set_kernel_events(int family, void* start, void* stop) {
  using namespace bytes_amd;
  if (family < 0 || family > kProfFamilies || (family > 0 && (!start || !stop))) return (int)hipErrorInvalidValue;
  g_prof_family.store(0);
  g_prof_start.store(static_cast<hipEvent_t>(start));
  g_prof_stop.store(static_cast<hipEvent_t>(stop));
  g_prof_family.store(family);
  return 0;
}

const char* bytes_error_string(int code) { return hipGetErrorString(static_cast<hipError_t>(code)); }

int bytes_abi_version(void) { return 1; }

}  // extern "C"
