// Error reporting shared by every entry point of libppo_hip.so.
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

}  // namespace ppo

extern "C" const char* ppo_last_error(void) { return ppo::g_error; }

extern "C" int ppo_abi_version(void) { return 5; }
