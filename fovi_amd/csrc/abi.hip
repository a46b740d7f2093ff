// Library-wide C-ABI entry points: version and error reporting.
#include <map>
#include <mutex>
#include <utility>

#include "common.h"

namespace fovi {

static thread_local std::string g_last_error;
static thread_local const char* g_last_path = "";

void note_path(const char* name) { g_last_path = name; }

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

hipError_t reserve_dynamic_lds(const void* kernel, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, size_t> done;   // (kernel, device) -> bytes reserved
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  size_t& have = done[std::make_pair(kernel, dev)];
  if (have >= bytes) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  if (e == hipSuccess) have = bytes;
  return e;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return 1;
  }
  return 0;
}

}  // namespace fovi

extern "C" int fovi_abi_version(void) { return FOVI_ABI_VERSION; }

extern "C" const char* fovi_last_error(void) { return fovi::g_last_error.c_str(); }

extern "C" const char* fovi_knnconv_last_path(void) { return fovi::g_last_path; }
