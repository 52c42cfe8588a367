// Error reporting for the C-ABI: every entry point returns an int status; the message of the last
// failure on the calling thread is available through sd_last_error().
#include <stdarg.h>
#include <stdio.h>

#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(kLaunchFailed, "%s: launch failed: %s", what, hipGetErrorString(err));
  return kOk;
}

}  // namespace sd

extern "C" const char* sd_last_error(void) { return sd::g_last_error; }

extern "C" int sd_abi_version(void) { return SD_ABI_VERSION; }
