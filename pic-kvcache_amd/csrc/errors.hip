// Error reporting shared by every entry point of libcacheblend_hip.so.
#include "cbk_common.hpp"

namespace cbk {

namespace {
thread_local char g_last_error[512] = {0};
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

int launch_status(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(CBK_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(err));
  }
  return CBK_OK;
}

}  // namespace cbk

extern "C" {

int cbk_abi_version(void) { return 1; }

const char* cbk_error_string(int code) {
  switch (code) {
    case CBK_OK: return "ok";
    case CBK_ERR_INVALID: return "invalid argument";
    case CBK_ERR_UNSUPPORTED: return "unsupported";
    case CBK_ERR_LAUNCH: return "HIP launch failure";
    case CBK_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown error";
  }
}

const char* cbk_last_error(void) { return cbk::g_last_error; }

}  // extern "C"
