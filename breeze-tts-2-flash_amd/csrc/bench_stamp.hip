// Measurement helper for bench.py (libbz_bench_stamp.so, not part of the decode-attention C ABI): a one-thread kernel
// that writes the GPU's constant-rate wall clock (s_memrealtime, 100 MHz on MI355X) to a device word. Two of them
// captured into a HIP graph around the timed calls measure those calls alone on the GPU: events recorded outside the
// graph would also hold the replay's own fixed cost (about 8 us per replay), and ROCm does not allow timing events
// inside a captured graph.
//
//   int bz_bench_stamp(uint64_t* dst, hipStream_t stream)   enqueue the stamp kernel; 0 or -1 (launch error)
//   int bz_bench_stamp_rate_khz(int* khz)                    the wall clock's rate of the current device; 0 or -1
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace {

__global__ void __launch_bounds__(64) stamp_kernel(uint64_t* dst) {
  if (threadIdx.x == 0) *dst = wall_clock64();
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int bz_bench_stamp(uint64_t* dst, hipStream_t stream) {
  if (dst == nullptr) return -1;
  hipLaunchKernelGGL(stamp_kernel, dim3(1), dim3(64), 0, stream, dst);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

__attribute__((visibility("default"))) int bz_bench_stamp_rate_khz(int* khz) {
  int dev = 0;
  if (khz == nullptr || hipGetDevice(&dev) != hipSuccess) return -1;
  return hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess ? 0 : -1;
}

}  // extern "C"
