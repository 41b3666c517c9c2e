// Status / error objects of the C ABI and small device queries.  The error objects
// are this library's own (am_gfx950_error_*): the reference library keeps the
// am_error_* names of its c_api.h:82-88.

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <unordered_map>

#include "am_c_api.h"
#include "am_gfx950.h"

namespace {
thread_local std::string g_last_error;

struct ErrorObject {
  am_status_code code;
  std::string message;
};
}  // namespace

namespace am {
am_status_code SetLastError(am_status_code code, const char* msg) {
  g_last_error = msg ? msg : "";
  return code;
}

int DeviceCUs() {
  static std::mutex mu;
  static std::unordered_map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  cache[dev] = cus;
  return cus;
}
}  // namespace am

extern "C" {

am_error_handle am_gfx950_error_create(am_status_code code, const char* message) {
  return new ErrorObject{code, message ? message : ""};
}

void am_gfx950_error_destroy(am_error_handle e) { delete static_cast<ErrorObject*>(e); }

am_status_code am_gfx950_error_code(am_error_handle e) {
  return e ? static_cast<ErrorObject*>(e)->code : AM_STATUS_INVALID_ARGUMENT;
}

const char* am_gfx950_error_message(am_error_handle e) { return e ? static_cast<ErrorObject*>(e)->message.c_str() : ""; }

const char* am_last_error_message(void) { return g_last_error.c_str(); }

int32_t am_gfx950_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

const char* am_gfx950_version(void) { return "aethermind-gfx950 0.1 (gfx950, HIP)"; }

}  // extern "C"
