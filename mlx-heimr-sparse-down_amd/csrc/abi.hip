// Error state and version of the libhsd C ABI.
#include "hsd_common.h"

#include <string>

namespace hsd {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(HSD_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return HSD_OK;
}

}  // namespace hsd

extern "C" const char* hsd_last_error(void) { return hsd::g_last_error.c_str(); }

extern "C" int hsd_abi_version(void) { return 1; }
