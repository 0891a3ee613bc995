// C-ABI housekeeping: thread-local last-error string, library version, and
// the per-device property cache (the only state the library keeps between
// calls besides the thread-local decode-family switch of hn_gemv.hip).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

static thread_local char g_hn_err[512] = "";

extern "C" void hn_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_hn_err, sizeof(g_hn_err), fmt, ap);
  va_end(ap);
}

extern "C" const char* hn_last_error_string(void) { return g_hn_err; }

extern "C" int hn_abi_version(void) { return 1; }

// CU count of the current device, queried once per device.  Concurrent first
// calls may both query; they store the same value.
namespace {
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];
}  // namespace

// Launch tags of the last-arriver counters (hn_common.h, hn_arrive).
extern "C" unsigned long long hn_next_tag(void) {
  static std::atomic<unsigned long long> tag{0};
  const unsigned long long t = (tag.fetch_add(1, std::memory_order_relaxed) + 1) &
                               ((1ull << 48) - 1);
  return t ? t : 1;
}

extern "C" int hn_device_cus(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int n = g_cus[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      v <= 0)
    v = 256;
  g_cus[dev].store(v, std::memory_order_relaxed);
  return v;
}

extern "C" int hn_current_device(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  return dev;
}
