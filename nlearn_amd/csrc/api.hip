// api.hip — status codes, per-thread error messages and small utilities of
// the C ABI declared in include/nlearn_hip.h.
#include <string>

#include "common.h"

namespace {
thread_local std::string g_last_error;
}

int nl_set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int nl_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return nl_set_error(NL_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  }
  return NL_OK;
}

extern "C" const char* nl_strerror(int status) {
  switch (status) {
    case NL_OK: return "ok";
    case NL_EINVAL: return "invalid argument";
    case NL_EALIGN: return "misaligned pointer or leading dimension";
    case NL_EUNSUPPORTED: return "unsupported configuration";
    case NL_ELAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

extern "C" const char* nl_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* nl_version(void) { return "nlearn_hip 0.1 gfx950"; }
