// Error state of the C ABI: every entry point returns an es_status code and leaves a message that
// es_last_error_string() returns (per host thread).
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/echosparse_hip.h"
#include "common.h"

namespace es {
static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": HIP launch failed: " + hipGetErrorString(e));
    return ES_ERR_LAUNCH;
  }
  return ES_OK;
}
}  // namespace es

extern "C" const char* es_last_error_string(void) { return es::g_last_error.c_str(); }

extern "C" int es_abi_version(void) { return ES_ABI_VERSION; }
