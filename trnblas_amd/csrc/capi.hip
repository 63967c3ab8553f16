// Error reporting and version of the C ABI (include/trnblas_hip.h).
#include <stdarg.h>

#include "common.hpp"

namespace trnblas {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TRNBLAS_E_LAUNCH;
  }
  return TRNBLAS_OK;
}

}  // namespace trnblas

extern "C" int trnblas_hip_abi_version(void) { return 11; }

extern "C" const char* trnblas_hip_last_error(void) { return trnblas::g_last_error; }
