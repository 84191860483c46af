// fgs_capi.cpp -- error reporting and version query of the C ABI.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "fgs_common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace fgs {

int32_t set_error(int32_t code, const char* msg) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s", msg ? msg : "");
  return code;
}

int32_t check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s", what, hipGetErrorString(e));
    return FGS_ERR_LAUNCH;
  }
  return FGS_OK;
}

}  // namespace fgs

extern "C" const char* fgs_last_error(void) { return g_last_error; }

extern "C" int32_t fgs_abi_version(void) { return 9; }
