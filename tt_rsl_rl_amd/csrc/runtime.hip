// Error reporting shared by every entry point of libppo_hip.so.
#include <atomic>

#include "common.hpp"

namespace ppo {

namespace {
thread_local char g_error[1024] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PPO_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PPO_OK;
}

DeviceInfo device_info() {
  static std::atomic<int> cus_cache[kMaxDevices], xcds_cache[kMaxDevices];  // value + 1; 0 = not queried yet
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return {0, 0};
  }
  int c = cus_cache[dev].load(std::memory_order_relaxed);
  int x = xcds_cache[dev].load(std::memory_order_relaxed);
  if (c == 0 || x == 0) {
    int cus = 0, xcds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) xcds = 0;
    (void)hipGetLastError();
    c = std::max(cus, 0) + 1;
    x = std::max(xcds, 1) + 1;
    cus_cache[dev].store(c, std::memory_order_relaxed);
    xcds_cache[dev].store(x, std::memory_order_relaxed);
  }
  return {c - 1, x - 1};
}

}  // namespace ppo

extern "C" const char* ppo_last_error(void) { return ppo::g_error; }

extern "C" int ppo_abi_version(void) { return 8; }
