// Measurement helpers for bench.py (libbz_bench_stamp.so, not part of the decode-attention C ABI). A one-thread kernel
// that writes the GPU's constant-rate wall clock (s_memrealtime, 100 MHz on MI355X) to a device word. Two of them
// captured into a HIP graph around the timed calls measure those calls alone on the GPU: events recorded outside the
// graph would also hold the replay's own fixed cost (about 8 us per replay), and ROCm does not allow timing events
// inside a captured graph.
//
//   int bz_bench_stamp(uint64_t* dst, hipStream_t stream)   enqueue the stamp kernel; 0 or -1 (launch error)
//   int bz_bench_stamp_rate_khz(int* khz)                    the wall clock's rate of the current device; 0 or -1
//   int bz_bench_stream_read(const void* data, uint64_t bytes_per_wg, int workgroups, uint32_t* sink,
//                            hipStream_t stream)
//       enqueue a pure streaming read of workgroups * bytes_per_wg bytes from data (workgroup i reads its own
//       contiguous bytes_per_wg, a multiple of 16, with 256 threads and eight 16-byte non-temporal loads per thread
//       in flight, as the attention kernel streams its K/V), doing nothing with the bytes: the floor that the
//       memory system and one launch set for reading that much. sink: one word, written only if the data XOR to a
//       marker value (so that no load can be dropped); 0 or -1 (bad argument or launch error)
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace {

__global__ void __launch_bounds__(64) stamp_kernel(uint64_t* dst) {
  if (threadIdx.x == 0) *dst = wall_clock64();
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kStreamThreads = 256, kStreamDepth = 8;
constexpr uint32_t kMarker = 0x9e3779b9u;

__global__ void __launch_bounds__(kStreamThreads) stream_read_kernel(const u32x4* __restrict__ data, uint64_t vec_per_wg,
                                                                     uint32_t* sink) {
  const u32x4* src = data + (uint64_t)blockIdx.x * vec_per_wg;
  uint32_t acc = 0;
  for (uint64_t i = threadIdx.x; i < vec_per_wg; i += (uint64_t)kStreamThreads * kStreamDepth) {
    u32x4 r[kStreamDepth];
#pragma unroll
    for (int u = 0; u < kStreamDepth; ++u) {
      const uint64_t j = i + (uint64_t)u * kStreamThreads;
      r[u] = j < vec_per_wg ? __builtin_nontemporal_load(src + j) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kStreamDepth; ++u) acc ^= r[u][0] ^ r[u][1] ^ r[u][2] ^ r[u][3];
  }
  if (acc == kMarker) *sink = acc;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int bz_bench_stamp(uint64_t* dst, hipStream_t stream) {
  if (dst == nullptr) return -1;
  hipLaunchKernelGGL(stamp_kernel, dim3(1), dim3(64), 0, stream, dst);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

__attribute__((visibility("default"))) int bz_bench_stream_read(const void* data, uint64_t bytes_per_wg, int workgroups,
                                                                uint32_t* sink, hipStream_t stream) {
  if (data == nullptr || sink == nullptr || workgroups <= 0 || bytes_per_wg % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(data) & 15) != 0)
    return -1;
  hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(kStreamThreads), 0, stream,
                     static_cast<const u32x4*>(data), bytes_per_wg / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

__attribute__((visibility("default"))) int bz_bench_stamp_rate_khz(int* khz) {
  int dev = 0;
  if (khz == nullptr || hipGetDevice(&dev) != hipSuccess) return -1;
  return hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess ? 0 : -1;
}

}  // extern "C"
