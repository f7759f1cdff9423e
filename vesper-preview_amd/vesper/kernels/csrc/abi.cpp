// The C ABI's shared pieces: the per-thread last-error string and the version query.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "common.h"
#include "vesper_kernels.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace vsp {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  g_last_error[0] = '\0';
  return OK;
}

}  // namespace vsp

extern "C" const char* vsp_last_error(void) { return g_last_error; }

extern "C" int vsp_abi_version(void) { return VSP_ABI_VERSION; }
