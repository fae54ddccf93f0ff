// Version query and the thread-local error channel of the libivakv C ABI.
#include "ivakv_internal.h"

namespace ivakv {

namespace {
thread_local char g_last_error[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(IVAKV_E_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return IVAKV_OK;
}

}  // namespace ivakv

extern "C" int ivakv_abi_version(void) { return IVAKV_ABI_VERSION; }

extern "C" const char* ivakv_last_error(void) { return ivakv::g_last_error; }
