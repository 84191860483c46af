// Exhaustive check of the two instructions blend_exp2f (fgs_device.hpp) takes
// its reduction from: for every float t in [-126, 8],
//   v_fract_f32(t)        == fminf(t - floorf(t), 0x1.fffffep-1f)
//   v_cvt_flr_i32_f32(t)  == (int)floorf(t)
// (the values the CPU oracle computes with floorf and the IEEE subtraction).
// Prints the count of floats checked and of mismatches; exit status 0 when
// there are none.  Built beside the library; run by
// tests/test_gpu_fract_floor.py.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

__global__ void check_kernel(uint32_t hi_neg, uint32_t hi_pos, unsigned long long* bad,
                             uint32_t* first) {
  // negative patterns 0x80000000 (-0) .. hi_neg, then positive 0 .. hi_pos
  const uint64_t n_neg = (uint64_t)(hi_neg - 0x80000000u) + 1;
  const uint64_t total = n_neg + (uint64_t)hi_pos + 1;
  unsigned long long local = 0;
  uint32_t fb = 0xFFFFFFFFu;
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < total;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t bits = i < n_neg ? 0x80000000u + (uint32_t)i : (uint32_t)(i - n_neg);
    const float t = __uint_as_float(bits);
    const float fr = __builtin_amdgcn_fractf(t);
    int e;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(e) : "v"(t));
    const float fl = __builtin_floorf(t);
    const float want = fminf(t - fl, 0x1.fffffep-1f);
    if (__float_as_uint(fr) != __float_as_uint(want) || e != (int)fl) {
      ++local;
      fb = bits < fb ? bits : fb;
    }
  }
  if (local) {
    atomicAdd(bad, local);
    atomicMin(first, fb);
  }
}

int main() {
  const uint32_t hi_neg = 0xC2FC0000u;  // -126
  const uint32_t hi_pos = 0x41000000u;  // 8
  unsigned long long* d_bad = nullptr;
  uint32_t* d_first = nullptr;
  unsigned long long bad = 0;
  uint32_t first = 0xFFFFFFFFu;
  if (hipMalloc(&d_bad, sizeof bad) != hipSuccess || hipMalloc(&d_first, sizeof first) != hipSuccess ||
      hipMemcpy(d_bad, &bad, sizeof bad, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(d_first, &first, sizeof first, hipMemcpyHostToDevice) != hipSuccess) {
    std::printf("allocation failed\n");
    return 2;
  }
  hipLaunchKernelGGL(check_kernel, dim3(4096), dim3(256), 0, 0, hi_neg, hi_pos, d_bad, d_first);
  if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(&bad, d_bad, sizeof bad, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&first, d_first, sizeof first, hipMemcpyDeviceToHost) != hipSuccess) {
    std::printf("launch failed\n");
    return 3;
  }
  const unsigned long long n = (unsigned long long)(hi_neg - 0x80000000u) + 1ull + hi_pos + 1ull;
  std::printf("checked %llu floats, mismatches %llu, first 0x%08x\n", n, bad, first);
  hipFree(d_bad);
  hipFree(d_first);
  return bad ? 1 : 0;
}
