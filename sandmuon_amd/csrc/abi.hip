// Library-wide ABI plumbing: version and thread-local error reporting.
#include "common.h"

#include <cstdio>

namespace smx {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    std::snprintf(buf, sizeof(buf), "%s: launch failed: %s", what, hipGetErrorString(e));
    g_last_error = buf;
    return SMX_ELAUNCH;
  }
  return SMX_OK;
}

}  // namespace smx

extern "C" int smx_abi_version(void) { return SMX_ABI_VERSION; }

extern "C" const char *smx_last_error(void) { return smx::g_last_error.c_str(); }
