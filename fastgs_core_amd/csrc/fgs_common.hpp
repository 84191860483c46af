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

// Main kernels whose launches can be bracketed by caller events
// (fgs_set_launch_events); launch_mark(k, st, 0) goes directly before the
// launch, launch_mark(k, st, 1) directly after it.  Returns FGS_OK, or an
// error code when recording an event fails.
enum LaunchKind {
  kLaunchPreprocessFwd,
  kLaunchRasterFwd,
  kLaunchRasterBwd,
  kLaunchPreprocessBwd,
  kLaunchLossFwd,
  kLaunchLossBwd,
  kLaunchPreprocessColour,
  kLaunchKinds
};
int32_t launch_mark(LaunchKind k, hipStream_t st, int after);

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

// The fill of FillSpans by thread tid of nthreads: a head of single words up
// to 16-byte alignment, 16-byte stores, then the tail.
__device__ __forceinline__ void fill_spans_body(const FillSpans& f, int64_t tid,
                                                int64_t nthreads) {
  const uint4 v4 = make_uint4(f.value, f.value, f.value, f.value);
  for (int s = 0; s < f.count; ++s) {
    uint32_t* p = f.p[s];
    const int64_t n = f.n[s];
    int64_t head = (int64_t)(((16u - (uint32_t)(reinterpret_cast<uintptr_t>(p) & 15u)) & 15u) >> 2);
    if (head > n) head = n;
    if (tid < head) p[tid] = f.value;
    const int64_t nv = (n - head) >> 2;
    uint4* q = reinterpret_cast<uint4*>(p + head);
    for (int64_t i = tid; i < nv; i += nthreads) q[i] = v4;
    const int64_t done = head + nv * 4;
    if (tid < n - done) p[done + tid] = f.value;
  }
}

}  // namespace fgs
