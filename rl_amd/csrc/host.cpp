// Host-side support shared by every entry point: per-thread error messages,
// launch checking and the version string.
#include "common.h"

namespace mirl {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MIRL_ERR_HIP;
  }
  return MIRL_OK;
}

}  // namespace mirl

extern "C" const char* mirl_last_error(void) { return mirl::g_last_error.c_str(); }

extern "C" const char* mirl_version(void) { return "mirl 0.1.0 gfx950"; }
