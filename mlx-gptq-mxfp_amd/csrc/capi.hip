// Library-wide C-ABI plumbing: version, per-thread error message, launch
// checks.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "mgq_capi.h"

namespace mgq {
namespace {
thread_local char g_last_error[1024] = {0};
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return MGQ_OK;
  set_error("%s: HIP error %d (%s)", what, static_cast<int>(e), hipGetErrorString(e));
  return MGQ_ERR_HIP;
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

}  // namespace mgq

extern "C" int mgq_version(void) { return 100; }

extern "C" const char* mgq_last_error(void) { return mgq::g_last_error; }
