// Error reporting and versioning shared by every entry point of the C ABI.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace yapd {

namespace {
thread_local char g_last_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return YAPD_OK;
  set_error("%s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
  return YAPD_EHIP;
}

}  // namespace yapd

extern "C" const char* yapd_last_error(void) { return yapd::g_last_error; }

extern "C" int yapd_abi_version(void) { return 4; }
