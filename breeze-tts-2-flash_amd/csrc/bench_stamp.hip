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
//
//   int bz_bench_kv_pattern(const bz_bench_kv_args* a, hipStream_t stream)
//       enqueue the split kernel's memory traffic without its arithmetic, for a contiguous [rows, kv heads, capacity,
//       128] bf16 cache: grid (splits, kv heads, rows) of 256 threads, the arguments of the stream preloaded into
//       SGPRs as the kernel's are; each workgroup reads the row length from seq_lens, cuts the row into chunks by the
//       split kernel's rule and streams its chunk of K and V as the split kernel does (16 lanes per 256-byte row, two
//       tiles of 32 positions in flight, non-temporal loads through buffer resources cut at the chunk's end), folding
//       the bytes by XOR. With exchange != 0 it then runs the split kernel's exchange on a 1 KB partial per workgroup
//       (agent-scope stores, store wait, barrier, agent-scope arrival counter; the last workgroup of each (row, kv
//       head) reads every partial with sc1 loads, all in flight, and writes 256 bf16 values), so its time is the
//       floor that one launch, the K/V stream and the exchange protocol set for the kernel. Every partial holds 1.0
//       (unless the row's data XOR to the marker), so each output value is the row's chunk count (1 without
//       exchange). 0 or -1 (bad argument or launch error)
//   int bz_bench_kv_pattern_workspace(int32_t rows, int32_t num_kv_heads, int32_t splits, size_t* bytes)
//       bytes of a->workspace (zero-filled before the first call; the calls leave the counters at zero)
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

// ---- the split kernel's traffic without its arithmetic (head_dim 128)
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int kPatD = 128, kPatRowLanes = 16, kPatRows = kStreamThreads / kPatRowLanes;  // 16 rows per load
constexpr int kPatTile = 2 * kPatRows;                                                  // 32 positions per tile
constexpr int kPatMinChunk = 16 * 1024 / (4 * kPatD);                                   // 16 KB of K+V
constexpr int kPatOneSplit = 64 * 1024 / (4 * kPatD);                                   // 64 KB of K+V
constexpr int kPatCounterStride = 64;                                                   // ints per counter line
constexpr int kPatPartial = 256;                                                        // floats per partial

__device__ __forceinline__ Rsrc pat_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

struct PatTile {
  u32x4 k[2], v[2];
};

__device__ __forceinline__ void pat_load(PatTile& t, Rsrc rk, Rsrc rv, int pos0, int c) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t off = (uint32_t)(pos0 + kPatRows * i) * (2 * kPatD) + 16 * c;
    t.k[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 2));
    t.v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 2));
  }
}

__device__ __forceinline__ uint32_t pat_fold(const PatTile& t) {
  uint32_t a = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) a ^= t.k[i][0] ^ t.k[i][1] ^ t.k[i][2] ^ t.k[i][3] ^ t.v[i][0] ^ t.v[i][1] ^ t.v[i][2] ^ t.v[i][3];
  return a;
}

// ceil(n / d) for 0 <= n < 2^24, d >= 1, from a float reciprocal and one correction step (no integer division)
__device__ __forceinline__ int pat_ceil_div(int n, int d, float inv_d) {
  int q = (int)((float)n * inv_d);
  int r = n - q * d;
  q = r < 0 ? q - 1 : (r >= d ? q + 1 : q);
  r = n - q * d;
  return q + (r > 0);
}

__device__ __forceinline__ uint16_t pat_bf16(float x) { return (uint16_t)(__float_as_uint(x) >> 16); }  // exact here

// The arguments the stream needs come first, so that they are preloaded into SGPRs with the launch (the library is
// built with 14 dwords of kernel-argument preloading): the only memory access before the first K/V load is the
// row's length. The cache is [rows, nkv, cap, 128] bf16, contiguous.
template <bool XCH>
__global__ void __launch_bounds__(kStreamThreads) kv_pattern_kernel(const uint8_t* k, const uint8_t* v,
                                                                    const int32_t* lens, int cap, int splits,
                                                                    float inv_splits, int nkv, int* counters,
                                                                    float* partials,
                                                                    uint16_t* out, uint32_t* sink) {
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, r = tid / kPatRowLanes, c = tid % kPatRowLanes;
  const int len = min(max(lens[b], 0), cap);  // no access past the capacity
  const int chunk = len <= kPatOneSplit ? max(len, kPatMinChunk) : max(pat_ceil_div(len, splits, inv_splits), kPatMinChunk);
  if (split > 0 && split * chunk >= len) return;
  const int lo = split * chunk, hi = min(lo + chunk, len);
  const int64_t unit = (int64_t)b * nkv + h;
  const int64_t head = unit * cap * (2 * kPatD);
  const Rsrc rk = pat_rsrc(k + head, hi * 2 * kPatD), rv = pat_rsrc(v + head, hi * 2 * kPatD);
  PatTile ta, tb;
  pat_load(ta, rk, rv, lo + r, c);
  pat_load(tb, rk, rv, lo + kPatTile + r, c);
  const int nact = len > 0 ? pat_ceil_div(len, chunk, __builtin_amdgcn_rcpf((float)chunk)) : 1;
  uint32_t acc = 0;
  for (int t0 = lo; t0 < hi; t0 += 2 * kPatTile) {
    acc ^= pat_fold(ta);
    if (t0 + kPatTile >= hi) break;
    pat_load(ta, rk, rv, t0 + 2 * kPatTile + r, c);
    acc ^= pat_fold(tb);
    pat_load(tb, rk, rv, t0 + 3 * kPatTile + r, c);
  }
  uint16_t* const o = out + unit * kPatPartial;
  if (!XCH || nact == 1) {
    if (acc == kMarker) *sink = acc;
    if (split == 0) o[tid] = pat_bf16(1.f);
    return;
  }
  float* const part = partials + unit * splits * kPatPartial;
  // the partial carries the fold, so that no load can be dropped; it is 1.0 unless the data XOR to the marker
  __hip_atomic_store(part + split * kPatPartial + tid, acc == kMarker ? 2.f : 1.f, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's partial stores have completed
  __syncthreads();
  if (tid == 0) {
    int* const cnt = counters + unit * kPatCounterStride;
    const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == nact - 1;
    if (s_last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  const Rsrc rp = pat_rsrc(part, nact * kPatPartial * 4);
  float sum = 0.f;
  for (int s0 = 0; s0 < nact; s0 += 16) {
    float x[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      x[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rp, ((s0 + u) * kPatPartial + tid) * 4, 0, 16));
#pragma unroll
    for (int u = 0; u < 16; ++u) sum += x[u];  // 0 past nact (outside the resource)
  }
  o[tid] = pat_bf16(sum);
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

typedef struct bz_bench_kv_args {
  const void* k_cache;  // [rows, num_kv_heads, capacity, 128] bf16, strides in elements, head_dim contiguous
  const void* v_cache;
  int64_t kv_stride_b, kv_stride_h, kv_stride_s;
  const int32_t* seq_lens;  // [rows]
  int32_t rows, num_kv_heads, head_dim, capacity, splits, exchange;
  void* workspace;
  size_t workspace_bytes;
  uint16_t* out;  // [rows, num_kv_heads, 256]
  uint32_t* sink;
} bz_bench_kv_args;

__attribute__((visibility("default"))) int bz_bench_kv_pattern_workspace(int32_t rows, int32_t num_kv_heads,
                                                                         int32_t splits, size_t* bytes) {
  if (bytes == nullptr || rows <= 0 || num_kv_heads <= 0 || splits <= 0 || splits > 256) return -1;
  const size_t units = (size_t)rows * num_kv_heads;
  *bytes = units * kPatCounterStride * 4 + units * splits * kPatPartial * 4;
  return 0;
}

__attribute__((visibility("default"))) int bz_bench_kv_pattern(const bz_bench_kv_args* a, hipStream_t stream) {
  size_t need = 0;
  if (a == nullptr || a->k_cache == nullptr || a->v_cache == nullptr || a->seq_lens == nullptr ||
      a->workspace == nullptr || a->out == nullptr || a->sink == nullptr || a->head_dim != kPatD ||
      a->capacity <= 0 || bz_bench_kv_pattern_workspace(a->rows, a->num_kv_heads, a->splits, &need) != 0 ||
      a->workspace_bytes < need || a->num_kv_heads > 65535 || a->rows > 65535)
    return -1;
  if ((reinterpret_cast<uintptr_t>(a->k_cache) | reinterpret_cast<uintptr_t>(a->v_cache)) & 15) return -1;
  // contiguous [rows, num_kv_heads, capacity, 128] only, spans addressable with 31-bit byte offsets
  if (a->kv_stride_s != kPatD || a->kv_stride_h != (int64_t)a->capacity * kPatD ||
      a->kv_stride_b != (int64_t)a->num_kv_heads * a->kv_stride_h)
    return -1;
  if ((int64_t)(a->capacity + 1024) * kPatD * 2 >= ((int64_t)1 << 31)) return -1;
  int* const counters = static_cast<int*>(a->workspace);
  float* const partials = reinterpret_cast<float*>(static_cast<uint8_t*>(a->workspace) +
                                                   (size_t)a->rows * a->num_kv_heads * kPatCounterStride * 4);
  const dim3 grid(a->splits, a->num_kv_heads, a->rows);
  const float inv = 1.f / (float)a->splits;
  const uint8_t* k = static_cast<const uint8_t*>(a->k_cache);
  const uint8_t* v = static_cast<const uint8_t*>(a->v_cache);
  if (a->exchange)
    hipLaunchKernelGGL(kv_pattern_kernel<true>, grid, dim3(kStreamThreads), 0, stream, k, v, a->seq_lens,
                       a->capacity, a->splits, inv, a->num_kv_heads, counters, partials, a->out, a->sink);
  else
    hipLaunchKernelGGL(kv_pattern_kernel<false>, grid, dim3(kStreamThreads), 0, stream, k, v, a->seq_lens,
                       a->capacity, a->splits, inv, a->num_kv_heads, counters, partials, a->out, a->sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

__attribute__((visibility("default"))) int bz_bench_stamp_rate_khz(int* khz) {
  int dev = 0;
  if (khz == nullptr || hipGetDevice(&dev) != hipSuccess) return -1;
  return hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess ? 0 : -1;
}

}  // extern "C"
