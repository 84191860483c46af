// fgs_common.hpp -- host-side helpers shared by the C-ABI entry points:
// thread-local error message and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fastgs_hip.h"
#include "fgs_device.hpp"

namespace fgs {

// Records msg as the calling thread's last error and returns code.
int32_t set_error(int32_t code, const char* msg);

// Checks hipGetLastError() after a launch; returns FGS_OK or FGS_ERR_LAUNCH.
int32_t check_launch(const char* what);

inline unsigned ceil_div_u(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// Up to kFillSpans 32-bit arrays set to one value by a single kernel launch
// (no hipMemsetAsync: callers may capture these calls in HIP graphs).
constexpr int kFillSpans = 4;
struct FillSpans {
  uint32_t* p[kFillSpans];
  int64_t n[kFillSpans];
  int count;
  uint32_t value;
};
void launch_fill_spans(const FillSpans& f, hipStream_t st);

}  // namespace fgs
