// Error state and version of the libhsd C ABI.
#include "hsd_common.h"

#include <map>
#include <mutex>
#include <string>
#include <tuple>

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

static std::mutex g_occ_mu;
static std::map<std::tuple<const void*, int, size_t, int>, int> g_occ;

int resident_workgroups(const void* kernel, int threads, size_t lds, int fallback) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fallback;
  std::lock_guard<std::mutex> lock(g_occ_mu);
  auto key = std::make_tuple(kernel, threads, lds, dev);
  auto it = g_occ.find(key);
  if (it != g_occ.end()) return it->second;
  int per_cu = 0, cus = 0;
  int r = fallback;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && per_cu > 0 && cus > 0)
    r = per_cu * cus;
  g_occ[key] = r;
  return r;
}

}  // namespace hsd

extern "C" const char* hsd_last_error(void) { return hsd::g_last_error.c_str(); }

extern "C" int hsd_abi_version(void) { return 1; }
