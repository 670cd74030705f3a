// Status codes and the thread-local error message of the C ABI.
#include "zmoe_internal.h"

namespace zmoe {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(ZMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ZMOE_OK;
}

}  // namespace zmoe

extern "C" int zmoe_abi_version(void) { return ZMOE_ABI_VERSION; }

extern "C" const char* zmoe_status_string(int status) {
  switch (status) {
    case ZMOE_OK: return "ok";
    case ZMOE_ERR_NULL: return "null pointer";
    case ZMOE_ERR_SHAPE: return "bad shape";
    case ZMOE_ERR_DTYPE: return "unsupported dtype";
    case ZMOE_ERR_ALIGN: return "misaligned pointer or stride";
    case ZMOE_ERR_WORKSPACE: return "workspace too small";
    case ZMOE_ERR_HIP: return "HIP error";
    default: return "unknown status";
  }
}

extern "C" const char* zmoe_last_error(void) { return zmoe::g_last_error; }
