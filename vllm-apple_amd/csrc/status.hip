// Error reporting shared by every entry point of the library.
#include "common.h"

namespace vaa {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(VAA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return VAA_OK;
}

}  // namespace vaa

extern "C" const char* vaa_last_error(void) { return vaa::g_last_error; }
extern "C" int vaa_abi_version(void) { return VAA_ABI_VERSION; }
