// Error state of the C-ABI: every entry point returns 0 on success and a
// non-zero status otherwise; moba_hip_last_error() gives the message of the
// last failure on the calling thread.
#include <cstdarg>
#include <cstdio>
#include "common.h"
#include "../../include/moba_hip.h"

static thread_local char g_err[512] = "";

void moba_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int moba_launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    moba_set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MOBA_ERR_LAUNCH;
  }
  return MOBA_OK;
}

extern "C" const char* moba_hip_last_error(void) { return g_err; }

extern "C" int moba_hip_version(void) { return MOBA_HIP_ABI_VERSION; }
