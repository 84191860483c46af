// fgs_capi.cpp -- error reporting, version query and launch events of the C ABI.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>

#include "fgs_common.hpp"

namespace {
thread_local char g_last_error[512] = "";

// Caller events per launch kind: [kind][0] before, [kind][1] after.
std::atomic<void*> g_launch_events[fgs::kLaunchKinds][2];
constexpr const char* kLaunchNames[fgs::kLaunchKinds] = {
    "preprocess_fwd", "rasterize_fwd", "rasterize_bwd", "preprocess_bwd", "loss_fwd", "loss_bwd",
    "preprocess_colour"};
}  // namespace

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

int32_t launch_mark(LaunchKind k, hipStream_t st, int after) {
  void* ev = g_launch_events[k][after ? 1 : 0].load(std::memory_order_acquire);
  if (!ev) return FGS_OK;
  const hipError_t e = hipEventRecord((hipEvent_t)ev, st);
  if (e != hipSuccess) {
    std::snprintf(g_last_error, sizeof(g_last_error), "launch event of %s: %s", kLaunchNames[k],
                  hipGetErrorString(e));
    return FGS_ERR_LAUNCH;
  }
  return FGS_OK;
}

}  // namespace fgs

extern "C" const char* fgs_last_error(void) { return g_last_error; }

extern "C" int32_t fgs_abi_version(void) { return 16; }

extern "C" int32_t fgs_set_launch_events(const char* kernel, void* start, void* stop) {
  if (!kernel) return fgs::set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_set_launch_events: null name");
  if (!start != !stop)
    return fgs::set_error(FGS_ERR_INVALID_ARGUMENT,
                          "fgs_set_launch_events: give both events or neither");
  for (int k = 0; k < fgs::kLaunchKinds; ++k) {
    if (std::strcmp(kernel, kLaunchNames[k]) == 0) {
      g_launch_events[k][0].store(start, std::memory_order_release);
      g_launch_events[k][1].store(stop, std::memory_order_release);
      return FGS_OK;
    }
  }
  return fgs::set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_set_launch_events: unknown kernel name");
}
