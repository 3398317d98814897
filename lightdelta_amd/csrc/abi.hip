// Error reporting and version entry points of the C ABI.
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace ld {

int fail(int code, const char* msg) {
  snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
  return code;
}

int launch_failed(const char* what, hipError_t err) {
  snprintf(g_last_error, sizeof(g_last_error), "%s: kernel launch failed: %s", what,
           hipGetErrorString(err));
  return LD_ERR_LAUNCH;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return launch_failed(what, err);
  return LD_OK;
}

}  // namespace ld

extern "C" const char* ld_last_error(void) { return g_last_error; }

extern "C" int ld_abi_version(void) { return LD_ABI_VERSION; }
