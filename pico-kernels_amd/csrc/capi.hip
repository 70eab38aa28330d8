// Library-level C ABI: version and error reporting.
#include "pk_common.h"

#include <cstdarg>
#include <cstdio>

namespace pk {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
  set_error("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return PK_EHIP;
}

}  // namespace pk

extern "C" int pk_version(void) { return 100; }

extern "C" const char* pk_last_error(void) { return pk::g_last_error; }
