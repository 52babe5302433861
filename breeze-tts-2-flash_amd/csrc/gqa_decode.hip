// Host side of libbz_gqa_decode.so: the C ABI of include/bz_gqa_decode.h (argument checks, workspace layout, split
// and tiling heuristics, launches) and the kernel table of the plain (non-fused) attention. The device code is in
// gqa_kernels.cuh; the fused-prologue kernels are instantiated in gqa_fused.hip.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <atomic>
#include <mutex>

#include "bz_gqa_decode.h"
#include "gqa_kernels.cuh"
#include "gqa_wave.cuh"

namespace {

SplitFn pick_split(int D, int G, int mk, int ppt, int nt, bool fused) {
  if (fused) return bz::pick_split_fused(D, G, mk, ppt, nt);
  if (nt != kSplitThreads) return nullptr;
  if (D == 128) return pick_group<128, kSplitThreads, false>(G, mk, ppt);
  if (D == 64) return pick_group<64, kSplitThreads, false>(G, mk, ppt);
  return nullptr;
}

CombineFn pick_combine(int D, int G) {
#define BZ_COMBINE_CASE(DD, GG) \
  if (D == DD && G == GG) return gqa_combine_kernel<DD, GG>;
  BZ_COMBINE_CASE(128, 1) BZ_COMBINE_CASE(128, 2) BZ_COMBINE_CASE(128, 4) BZ_COMBINE_CASE(128, 8)
  BZ_COMBINE_CASE(64, 1) BZ_COMBINE_CASE(64, 2) BZ_COMBINE_CASE(64, 4) BZ_COMBINE_CASE(64, 8)
#undef BZ_COMBINE_CASE
  return nullptr;
}

using WaveFn = void (*)(const int32_t*, const int32_t*, const uint16_t*, const uint16_t*, int64_t, int64_t, int32_t,
                        int32_t, const Params);

WaveFn pick_wave(int D) {
  if (D == 128) return gqa_wave_kernel<128>;
  if (D == 64) return gqa_wave_kernel<64>;
  return nullptr;
}

using ProbsFn = void (*)(const Params, float*);

template <bool FUSED>
ProbsFn pick_probs(int D, int mk) {
  if (D == 128) {
    if (mk == BZ_MASK_BF16) return gqa_probs_kernel<128, BZ_MASK_BF16, FUSED>;
    if (mk == BZ_MASK_F32) return gqa_probs_kernel<128, BZ_MASK_F32, FUSED>;
    return gqa_probs_kernel<128, BZ_MASK_NONE, FUSED>;
  }
  if (D == 64 && !FUSED) {
    if (mk == BZ_MASK_BF16) return gqa_probs_kernel<64, BZ_MASK_BF16, false>;
    if (mk == BZ_MASK_F32) return gqa_probs_kernel<64, BZ_MASK_F32, false>;
    return gqa_probs_kernel<64, BZ_MASK_NONE, false>;
  }
  return nullptr;
}

bool supported_group(int G) { return G == 1 || G == 2 || G == 4 || G == 8; }
bool supported_dim(int D) { return D == 64 || D == 128; }

// Smallest chunk a split gets: 16 KB of K+V (32 positions at head_dim 128, 64 at head_dim 64).
int min_chunk_for(int D) { return (16 * 1024) / (4 * D); }

// Positions per thread per tile: 1 when two one-position tiles cover the expected chunk, else 2. Two tiles (A, B) are
// in flight from the start, so the first tile's arithmetic overlaps the second tile's arrival. Tiles of more
// positions (4 was measured) leave more arithmetic exposed after the last tile arrives: config 3 +2%, config 4 +6%.
int ppt_for(int D, int G, int chunk, int nt) {
  (void)G;
  const int rows = nt / (D / 8);
  return 2 * rows >= chunk ? 1 : 2;
}


std::atomic<int> g_cu_count[kMaxDevices];

int device_cus(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return BZ_ERR_DEVICE;
  if (dev >= 0 && dev < kMaxDevices) {
    const int cached = g_cu_count[dev].load(std::memory_order_relaxed);
    if (cached > 0) {
      *cus = cached;
      return BZ_OK;
    }
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return BZ_ERR_DEVICE;
  if (dev >= 0 && dev < kMaxDevices) g_cu_count[dev].store(n, std::memory_order_relaxed);
  *cus = n;
  return BZ_OK;
}

int effective_len(int capacity, int max_seq_len) {
  return (max_seq_len > 0 && max_seq_len < capacity) ? max_seq_len : capacity;
}

// Split count: enough workgroups to give every CU one (cus / units splits), and no chunk longer than kMaxChunk
// positions even in the longest row (a chunk streams through one workgroup two tiles at a time, so its latency grows
// with its length), but no split shorter than min_chunk positions. When the whole K+V span of the longest row fits
// kOneSplitBytes there is one split (the kernels apply the same bound to each row's actual length): the
// cross-workgroup merge of two or more splits costs about 2 us, more than one workgroup takes to stream 64 KB (cold,
// B2 16/8: head_dim 128, 128 positions 4.45 against 5.42 us; head_dim 64, 256 positions 4.47 against 5.17; at 128 KB
// one split is slower: 6.23 against 5.47).
int default_splits_for(int units, int D, int len, int cus) {
  constexpr int kMaxChunk = 256;
  if ((int64_t)len * 4 * D <= kOneSplitBytes) return 1;
  const int min_chunk = min_chunk_for(D);
  const int useful = len > 0 ? (len + min_chunk - 1) / min_chunk : 1;
  int s = (cus + units - 1) / units;
  const int by_len = (len + kMaxChunk - 1) / kMaxChunk;
  if (s < by_len) s = by_len;
  if (s > useful) s = useful;
  if (s > kMaxSplits) s = kMaxSplits;
  return s < 1 ? 1 : s;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace: the arrival counters of every (row, kv head), one 256-byte line each, first, then the split partials:
// (m, l) pairs and the G * D accumulators of each split. The counters are zero between calls (the merging workgroup
// resets its counter) and sit at the same place whatever the split count or length, so one zero-filled workspace
// serves every call with the same rows * kv heads that it is large enough for. The partials are written before they
// are read in every call.
struct WsLayout {
  size_t counters, ml, acc, total;
};

WsLayout ws_layout(int rows, int NH, int NKV, int D, int splits) {
  WsLayout w;
  w.counters = 0;
  w.ml = (size_t)rows * NKV * kCounterStride * sizeof(int);
  w.acc = align256(w.ml + (size_t)rows * NH * splits * sizeof(float2));
  w.total = align256(w.acc + (size_t)rows * NH * splits * D * sizeof(float));
  return w;
}

int check_sizes(int B, int NH, int NKV, int D, int cap) {
  if (B <= 0 || NH <= 0 || NKV <= 0 || cap <= 0 || D <= 0) return BZ_ERR_SHAPE;
  if (NH % NKV != 0) return BZ_ERR_SHAPE;
  if (B > 65535 || NKV > 65535) return BZ_ERR_SHAPE;  // grid.z / grid.y limits
  if (!supported_dim(D) || !supported_group(NH / NKV)) return BZ_ERR_UNSUPPORTED;
  return BZ_OK;
}

// Query tokens per row (0 in the struct means 1) and the number of (row, token) pairs, the kernels' grid rows.
int tokens_of(const bz_gqa_decode_args* a) { return a->tokens_per_row > 1 ? a->tokens_per_row : 1; }
int rows_of(const bz_gqa_decode_args* a) { return a->batch * tokens_of(a); }

int resolve_splits(const bz_gqa_decode_args* a, int* splits) {
  if (a->num_splits < 0 || a->num_splits > kMaxSplits) return BZ_ERR_SHAPE;
  if (a->num_splits > 0) {
    *splits = a->num_splits;
    return BZ_OK;
  }
  int cus = 0;
  const int rc = device_cus(&cus);
  if (rc != BZ_OK) return rc;
  *splits = default_splits_for(rows_of(a) * a->num_kv_heads, a->head_dim,
                               effective_len(a->capacity, a->max_seq_len), cus);
  return BZ_OK;
}

// The kernel parameters every entry shares: pointers, strides, sizes and the rows' range arrays.
Params base_params(const bz_gqa_decode_args* a, const int32_t* seq_lens, const int32_t* kv_start) {
  Params p{};
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_sb = a->q_stride_b;
  p.q_sh = a->q_stride_h;
  p.q_st = a->q_stride_t;
  p.T = tokens_of(a);
  p.k = static_cast<const uint16_t*>(a->k_cache);
  p.v = static_cast<const uint16_t*>(a->v_cache);
  p.kv_sb = a->kv_stride_b;
  p.kv_sh = a->kv_stride_h;
  p.kv_ss = a->kv_stride_s;
  p.seq_lens = seq_lens;
  p.kv_start = kv_start;
  p.mask = a->mask;
  p.m_sb = a->mask_stride_b;
  p.scale_log2 = a->scale * kLog2e;
  p.out = static_cast<uint16_t*>(a->out);
  p.o_sb = a->out_stride_b;
  p.o_sh = a->out_stride_h;
  p.o_st = a->out_stride_t;
  p.B = a->batch;
  p.NH = a->num_q_heads;
  p.NKV = a->num_kv_heads;
  p.G = a->num_q_heads / a->num_kv_heads;
  p.cap = a->capacity;
  p.splits = 1;
  p.inv_splits = 1.0f;
  return p;
}

// One wave per (row, token, q head): the device function attend_wave launched alone (bz_gqa_decode_wave, and the
// automatic route below). out and its strides must be 16-byte aligned.
bool wave_out_aligned(const bz_gqa_decode_args* a) {
  return !((reinterpret_cast<uintptr_t>(a->out) & 15) || ((a->out_stride_b | a->out_stride_h) & 7) ||
           (tokens_of(a) > 1 && (a->out_stride_t & 7)));
}

int launch_wave(const bz_gqa_decode_args* a, hipStream_t stream, const int32_t* seq_lens, const int32_t* kv_start) {
  const WaveFn fn = pick_wave(a->head_dim);
  if (fn == nullptr) return BZ_ERR_UNSUPPORTED;
  if (rows_of(a) > 65535) return BZ_ERR_SHAPE;  // one workgroup per wave: grid (G, NKV, rows), grid.z <= 65535
  const Params p = base_params(a, seq_lens, kv_start);
  hipLaunchKernelGGL(fn, dim3(a->num_q_heads / a->num_kv_heads, a->num_kv_heads, rows_of(a)), dim3(kWave), 0, stream,
                     p.seq_lens, p.kv_start, p.k, p.v, p.kv_sb, p.kv_sh, (int32_t)p.kv_ss, p.cap, p);
  return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

// The automatic route to the wave kernel: groups of two or more q heads over short rows, with nothing asked explicitly
// (split count, combine mode) and no mask. The split kernel's waves each run the dot products and softmax of all G
// heads in series, while the wave kernel gives each q head a wave whose first two K/V tiles (2 * 2048 / D positions)
// are loaded before its range is known. Measured per launch, 16 launches in a HIP graph over rows in the L2 (as a
// depth step's freshly written rows are), B2, 2 or 8 kv heads:
//   D 128, G 2: 17 positions 2.52 against 2.65 us, 32: 2.69 / 2.70, 48: 3.32 / 2.98 (the split kernel wins)
//   D 128, G 4: 17 positions 2.55 / 3.43, 32: 2.71 / 3.53, 64: 3.94 / 4.09, 128: 6.43 / 5.46
//   D 64,  G 2: 32 positions 2.17 / 2.51, 64: 2.65 / 2.75, 128: 3.74 / 3.12
//   D 64,  G 4: 64 positions 2.66 / 3.29, 128: 3.79 / 3.80
//   G 1: the split kernel from 17 positions on (D 128: 2.51 / 2.38)
// so the route takes rows of at most two tiles for G = 2 and four tiles for G >= 4 (positions: max_seq_len, else the
// capacity). The reference's depth transformer (8 q / 2 KV heads, D 128, at most 17 positions) is on it.
int wave_route_len(int D, int G) {
  const int tile = 2048 / D;  // positions per K/V tile of attend_wave
  return G >= 4 ? 4 * tile : (G >= 2 ? 2 * tile : 0);
}

bool wave_route(const bz_gqa_decode_args* a, int mask_kind, const bz_gqa_decode_fused_args* f) {
  return f == nullptr && mask_kind == BZ_MASK_NONE && a->num_splits == 0 && a->combine == BZ_COMBINE_AUTO &&
         effective_len(a->capacity, a->max_seq_len) <= wave_route_len(a->head_dim, a->num_q_heads / a->num_kv_heads) &&
         wave_out_aligned(a);
}

// The static scratch of bz_gqa_decode_noalloc, for callers that cannot allocate (code under HIP graph capture,
// torch.compile's CUDA-graph trees, serving loops that forbid allocation): device memory of the library itself, one
// copy per device, held until the process ends. Its layout differs from a workspace's: the arrival counters of up to
// kScratchGroups (row, kv head) groups sit at fixed places at its start whatever the call's sizes, so calls of any
// sizes can follow one another on it (a workspace's counter region follows the call's own group count); the split
// partials follow. The counters start at zero (a __device__ array is zero-initialised when the library is loaded)
// and every call leaves them at zero (the merging workgroup resets its counter); the partials are written before
// they are read. In host code `scratch` only names the symbol: its device address comes from hipGetSymbolAddress,
// per device (scratch_address below).
constexpr int kScratchGroups = 1024;
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices];

// Device address of the current device's scratch, looked up once per device with that device current.
int scratch_address(void** addr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return BZ_ERR_DEVICE;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return BZ_ERR_DEVICE;
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return BZ_OK;
}

// Picks the kernels, checks the workspace and launches the split kernel (and, when asked, the merge kernel), or the
// wave kernel where wave_route says so (it needs no workspace).
// seq_lens NULL: each row's range comes from the mask, scanned by the kernels themselves. f != nullptr selects the
// fused-prologue variant. scratch_base != nullptr: the static scratch (its address on the current device) instead of
// a->workspace.
int launch(const bz_gqa_decode_args* a, hipStream_t stream, const int32_t* seq_lens, const int32_t* kv_start,
           int mask_kind, const bz_gqa_decode_fused_args* f, void* scratch_base = nullptr) {
  const int NH = a->num_q_heads, NKV = a->num_kv_heads, D = a->head_dim, cap = a->capacity;
  const int G = NH / NKV, R = rows_of(a);
  if (a->combine < BZ_COMBINE_AUTO || a->combine > BZ_COMBINE_KERNEL) return BZ_ERR_COMBINE_MODE;
  // the split kernels built without a mask take each row's range from seq_lens alone
  if (mask_kind == BZ_MASK_NONE && seq_lens == nullptr) return BZ_ERR_NULL;
  if (seq_lens != nullptr && wave_route(a, mask_kind, f)) return launch_wave(a, stream, seq_lens, kv_start);
  int splits = 0;
  int rc = resolve_splits(a, &splits);
  if (rc != BZ_OK) return rc;
  WsLayout ws;
  char* wsb = nullptr;
  if (scratch_base == nullptr) {
    ws = ws_layout(R, NH, NKV, D, splits);
    if (a->workspace == nullptr || a->workspace_bytes < ws.total) return BZ_ERR_WORKSPACE;
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255) != 0) return BZ_ERR_ALIGNMENT;
    wsb = static_cast<char*>(a->workspace);
  } else {
    if ((long long)R * NKV > kScratchGroups) return BZ_ERR_SCRATCH;
    ws.counters = 0;
    ws.ml = (size_t)kScratchGroups * kCounterStride * sizeof(int);
    ws.acc = align256(ws.ml + (size_t)R * NH * splits * sizeof(float2));
    ws.total = align256(ws.acc + (size_t)R * NH * splits * D * sizeof(float));
    if (ws.total > kScratchBytes) return BZ_ERR_SCRATCH;
    wsb = static_cast<char*>(scratch_base);
  }

  const int min_chunk = min_chunk_for(D);
  const int len = effective_len(cap, a->max_seq_len);
  int chunk = (len + splits - 1) / splits;
  if (chunk < min_chunk) chunk = min_chunk;
  const int nt = kSplitThreads;
  const int ppt = ppt_for(D, G, chunk, nt);
  SplitFn split_fn = pick_split(D, G, mask_kind, ppt, nt, f != nullptr);
  CombineFn comb_fn = pick_combine(D, G);
  if (split_fn == nullptr || comb_fn == nullptr) return BZ_ERR_UNSUPPORTED;
  // One launch needs no residency of the whole grid: no workgroup waits for another (the last to count in merges,
  // the others leave), so grids larger than the device runs at once merge in the same launch.
  const bool two_kernels = a->combine == BZ_COMBINE_KERNEL;

  Params p = base_params(a, seq_lens, kv_start);
  p.splits = splits;
  p.inv_splits = 1.0f / (float)splits;
  p.min_chunk = min_chunk;
  p.mask_kind = mask_kind;
  p.combine_last = two_kernels ? 0 : 1;
  p.counters = reinterpret_cast<int*>(wsb + ws.counters);
  p.part_ml = reinterpret_cast<float2*>(wsb + ws.ml);
  p.part_acc = reinterpret_cast<float*>(wsb + ws.acc);
  p.qkv = nullptr;
  p.qkv_sb = 0;
  p.qn_w = p.kn_w = p.cos = p.sin = nullptr;
  p.eps = 0.f;
  p.cs_sb = 0;
  p.cache_pos = nullptr;
  p.k_out = p.v_out = nullptr;
  if (f != nullptr) {
    p.qkv = static_cast<const uint16_t*>(f->qkv);
    p.qkv_sb = f->qkv_stride_b;
    p.qn_w = static_cast<const uint16_t*>(f->q_norm_weight);
    p.kn_w = static_cast<const uint16_t*>(f->k_norm_weight);
    p.eps = f->eps;
    p.cos = static_cast<const uint16_t*>(f->cos);
    p.sin = static_cast<const uint16_t*>(f->sin);
    p.cs_sb = f->rope_stride_b;
    p.cache_pos = f->cache_pos;
    p.k_out = const_cast<uint16_t*>(p.k);
    p.v_out = const_cast<uint16_t*>(p.v);
  }

  hipLaunchKernelGGL(split_fn, dim3(splits, NKV, R), dim3(nt), 0, stream, p.seq_lens, p.kv_start, p.T, p);
  if (hipGetLastError() != hipSuccess) return BZ_ERR_LAUNCH;
  if (two_kernels && splits > 1) {
    hipLaunchKernelGGL(comb_fn, dim3(NKV, R), dim3(kThreads), 0, stream, p);
    if (hipGetLastError() != hipSuccess) return BZ_ERR_LAUNCH;
  }
  return BZ_OK;
}

int check_common(const bz_gqa_decode_args* a, bool need_q) {
  if (a == nullptr) return BZ_ERR_NULL;
  if ((need_q && a->q == nullptr) || a->k_cache == nullptr || a->v_cache == nullptr || a->out == nullptr)
    return BZ_ERR_NULL;
  int rc = check_sizes(a->batch, a->num_q_heads, a->num_kv_heads, a->head_dim, a->capacity);
  if (rc != BZ_OK) return rc;
  const uintptr_t kp = reinterpret_cast<uintptr_t>(a->k_cache), vp = reinterpret_cast<uintptr_t>(a->v_cache);
  if ((kp | vp) & 15) return BZ_ERR_ALIGNMENT;
  if (need_q && ((reinterpret_cast<uintptr_t>(a->q) & 15) || ((a->q_stride_b | a->q_stride_h) & 7) ||
                 (tokens_of(a) > 1 && (a->q_stride_t & 7))))
    return BZ_ERR_ALIGNMENT;
  if ((a->kv_stride_b | a->kv_stride_h | a->kv_stride_s) & 7) return BZ_ERR_ALIGNMENT;
  if (a->kv_stride_s < a->head_dim) return BZ_ERR_SHAPE;
  if (a->tokens_per_row < 0 || (int64_t)a->batch * tokens_of(a) > 65535) return BZ_ERR_SHAPE;  // grid.z limit
  // K/V are read through buffer resources with 32-bit byte offsets per (row, kv head): every offset the kernel forms
  // (positions below capacity + 1024, the largest read-ahead) must stay below 2^31
  if (((int64_t)a->capacity + 1024) * a->kv_stride_s * 2 > INT32_MAX) return BZ_ERR_SHAPE;
  if (a->mask_dtype < BZ_MASK_NONE || a->mask_dtype > BZ_MASK_F32) return BZ_ERR_MASK_DTYPE;
  return BZ_OK;
}

int check_fused(const bz_gqa_decode_fused_args* f) {
  if (f == nullptr) return BZ_ERR_NULL;
  const bz_gqa_decode_args* a = &f->base;
  int rc = check_common(a, false);
  if (rc != BZ_OK) return rc;
  if (f->qkv == nullptr || f->q_norm_weight == nullptr || f->k_norm_weight == nullptr || f->cos == nullptr ||
      f->sin == nullptr || f->cache_pos == nullptr)
    return BZ_ERR_NULL;
  if (a->head_dim != 128 || tokens_of(a) != 1) return BZ_ERR_UNSUPPORTED;
  if (f->qkv_stride_b < (int64_t)(a->num_q_heads + 2 * a->num_kv_heads) * a->head_dim) return BZ_ERR_SHAPE;
  if (f->rope_stride_b < a->head_dim) return BZ_ERR_SHAPE;
  const uintptr_t ptrs = reinterpret_cast<uintptr_t>(f->qkv) | reinterpret_cast<uintptr_t>(f->q_norm_weight) |
                         reinterpret_cast<uintptr_t>(f->k_norm_weight) | reinterpret_cast<uintptr_t>(f->cos) |
                         reinterpret_cast<uintptr_t>(f->sin);
  if ((ptrs & 15) || ((f->qkv_stride_b | f->rope_stride_b) & 7)) return BZ_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(f->cache_pos) & 7)) return BZ_ERR_ALIGNMENT;
  return BZ_OK;
}

// The probabilities of bz_gqa_decode / bz_gqa_decode_fused (f != nullptr) with these arguments.
int launch_probs(const bz_gqa_decode_args* a, const bz_gqa_decode_fused_args* f, float* probs, hipStream_t stream) {
  if (probs == nullptr || (a->seq_lens == nullptr && a->mask == nullptr)) return BZ_ERR_NULL;
  if (tokens_of(a) != 1) return BZ_ERR_UNSUPPORTED;
  if (reinterpret_cast<uintptr_t>(probs) & 3) return BZ_ERR_ALIGNMENT;
  const int mk = (a->mask == nullptr) ? BZ_MASK_NONE : a->mask_dtype;
  if (a->mask != nullptr && mk != BZ_MASK_BF16 && mk != BZ_MASK_F32) return BZ_ERR_MASK_DTYPE;
  const ProbsFn fn = f != nullptr ? pick_probs<true>(a->head_dim, mk) : pick_probs<false>(a->head_dim, mk);
  if (fn == nullptr) return BZ_ERR_UNSUPPORTED;
  Params p = base_params(a, a->seq_lens, a->seq_lens != nullptr ? a->kv_start : nullptr);
  p.mask_kind = mk;
  if (f != nullptr) {
    p.qkv = static_cast<const uint16_t*>(f->qkv);
    p.qkv_sb = f->qkv_stride_b;
    p.qn_w = static_cast<const uint16_t*>(f->q_norm_weight);
    p.eps = f->eps;
    p.cos = static_cast<const uint16_t*>(f->cos);
    p.sin = static_cast<const uint16_t*>(f->sin);
    p.cs_sb = f->rope_stride_b;
  }
  hipLaunchKernelGGL(fn, dim3(a->num_q_heads, a->batch), dim3(kThreads), 0, stream, p, probs);
  return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

}  // namespace

namespace bz {
// The CU count of the current device (cached per device), for the GEMVs' launch choices in gemv.hip.
int device_cu_count(int* cus) { return device_cus(cus); }
}  // namespace bz

extern "C" {

__attribute__((visibility("default"))) int bz_gqa_decode(const bz_gqa_decode_args* a, hipStream_t stream) {
  int rc = check_common(a, true);
  if (rc != BZ_OK) return rc;
  if (a->seq_lens == nullptr) return BZ_ERR_NULL;
  const int mk = (a->mask == nullptr) ? BZ_MASK_NONE : a->mask_dtype;
  if (a->mask != nullptr && mk == BZ_MASK_NONE) return BZ_ERR_MASK_DTYPE;
  return launch(a, stream, a->seq_lens, a->kv_start, mk, nullptr);
}

__attribute__((visibility("default"))) int bz_gqa_decode_noalloc(const bz_gqa_decode_args* a, hipStream_t stream) {
  int rc = check_common(a, true);
  if (rc != BZ_OK) return rc;
  void* sc = nullptr;
  if (a->seq_lens != nullptr) {
    const int mk = (a->mask == nullptr) ? BZ_MASK_NONE : a->mask_dtype;
    if (a->mask != nullptr && mk == BZ_MASK_NONE) return BZ_ERR_MASK_DTYPE;
    rc = scratch_address(&sc);
    if (rc != BZ_OK) return rc;
    return launch(a, stream, a->seq_lens, a->kv_start, mk, nullptr, sc);
  }
  if (a->mask == nullptr) return BZ_ERR_NULL;
  if (a->mask_dtype != BZ_MASK_BF16 && a->mask_dtype != BZ_MASK_F32) return BZ_ERR_MASK_DTYPE;
  rc = scratch_address(&sc);
  if (rc != BZ_OK) return rc;
  return launch(a, stream, nullptr, nullptr, a->mask_dtype, nullptr, sc);
}

__attribute__((visibility("default"))) int bz_gqa_decode_masked(const bz_gqa_decode_args* a, hipStream_t stream) {
  int rc = check_common(a, true);
  if (rc != BZ_OK) return rc;
  if (a->mask == nullptr) return BZ_ERR_NULL;
  if (a->mask_dtype != BZ_MASK_BF16 && a->mask_dtype != BZ_MASK_F32) return BZ_ERR_MASK_DTYPE;
  return launch(a, stream, nullptr, nullptr, a->mask_dtype, nullptr);
}

__attribute__((visibility("default"))) int bz_gqa_decode_fused(const bz_gqa_decode_fused_args* f,
                                                               hipStream_t stream) {
  int rc = check_fused(f);
  if (rc != BZ_OK) return rc;
  const bz_gqa_decode_args* a = &f->base;
  if (a->seq_lens != nullptr) {
    const int mk = (a->mask == nullptr) ? BZ_MASK_NONE : a->mask_dtype;
    if (a->mask != nullptr && mk == BZ_MASK_NONE) return BZ_ERR_MASK_DTYPE;
    return launch(a, stream, a->seq_lens, a->kv_start, mk, f);
  }
  if (a->mask == nullptr) return BZ_ERR_NULL;
  if (a->mask_dtype != BZ_MASK_BF16 && a->mask_dtype != BZ_MASK_F32) return BZ_ERR_MASK_DTYPE;
  return launch(a, stream, nullptr, nullptr, a->mask_dtype, f);
}

__attribute__((visibility("default"))) int bz_gqa_decode_wave(const bz_gqa_decode_args* a, hipStream_t stream) {
  int rc = check_common(a, true);
  if (rc != BZ_OK) return rc;
  if (a->seq_lens == nullptr) return BZ_ERR_NULL;
  if (a->mask != nullptr) return BZ_ERR_UNSUPPORTED;
  if (!wave_out_aligned(a)) return BZ_ERR_ALIGNMENT;
  return launch_wave(a, stream, a->seq_lens, a->kv_start);
}

__attribute__((visibility("default"))) int bz_gqa_decode_probs(const bz_gqa_decode_args* a, float* probs,
                                                               hipStream_t stream) {
  const int rc = check_common(a, true);
  return rc != BZ_OK ? rc : launch_probs(a, nullptr, probs, stream);
}

__attribute__((visibility("default"))) int bz_gqa_decode_fused_probs(const bz_gqa_decode_fused_args* f, float* probs,
                                                                     hipStream_t stream) {
  const int rc = check_fused(f);
  return rc != BZ_OK ? rc : launch_probs(&f->base, f, probs, stream);
}

__attribute__((visibility("default"))) int bz_mask_interval(const void* mask, int32_t mask_dtype,
                                                            int64_t mask_stride_b, int32_t batch, int32_t capacity,
                                                            int32_t* seq_lens, int32_t* kv_start, hipStream_t stream) {
  if (mask == nullptr || seq_lens == nullptr || kv_start == nullptr) return BZ_ERR_NULL;
  if (mask_dtype != BZ_MASK_BF16 && mask_dtype != BZ_MASK_F32) return BZ_ERR_MASK_DTYPE;
  if (batch <= 0 || capacity <= 0 || mask_stride_b < 0 || (batch > 1 && mask_stride_b > 0 && mask_stride_b < capacity))
    return BZ_ERR_SHAPE;
  const size_t esize = mask_dtype == BZ_MASK_BF16 ? 2 : 4;
  if ((reinterpret_cast<uintptr_t>(mask) % esize) || (reinterpret_cast<uintptr_t>(seq_lens) & 3) ||
      (reinterpret_cast<uintptr_t>(kv_start) & 3))
    return BZ_ERR_ALIGNMENT;
  if (mask_dtype == BZ_MASK_BF16)
    hipLaunchKernelGGL(mask_range_kernel<BZ_MASK_BF16>, dim3(batch), dim3(kThreads), 0, stream, mask, mask_stride_b,
                       capacity, kv_start, seq_lens);
  else
    hipLaunchKernelGGL(mask_range_kernel<BZ_MASK_F32>, dim3(batch), dim3(kThreads), 0, stream, mask, mask_stride_b,
                       capacity, kv_start, seq_lens);
  return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

__attribute__((visibility("default"))) int bz_gqa_decode_workspace_size(int32_t batch, int32_t num_q_heads,
                                                                        int32_t num_kv_heads, int32_t head_dim,
                                                                        int32_t capacity, int32_t num_splits,
                                                                        int32_t max_seq_len, size_t* bytes) {
  if (bytes == nullptr) return BZ_ERR_NULL;
  int rc = check_sizes(batch, num_q_heads, num_kv_heads, head_dim, capacity);
  if (rc != BZ_OK) return rc;
  if (num_splits < 0 || num_splits > kMaxSplits) return BZ_ERR_SHAPE;
  int splits = num_splits;
  if (splits == 0) {
    int cus = 0;
    rc = device_cus(&cus);
    if (rc != BZ_OK) return rc;
    splits = default_splits_for(batch * num_kv_heads, head_dim, effective_len(capacity, max_seq_len), cus);
  }
  *bytes = ws_layout(batch, num_q_heads, num_kv_heads, head_dim, splits).total;
  return BZ_OK;
}

__attribute__((visibility("default"))) int bz_gqa_decode_default_splits(int32_t batch, int32_t num_kv_heads,
                                                                        int32_t head_dim, int32_t capacity,
                                                                        int32_t max_seq_len, int32_t* num_splits) {
  if (num_splits == nullptr) return BZ_ERR_NULL;
  if (batch <= 0 || num_kv_heads <= 0 || capacity <= 0) return BZ_ERR_SHAPE;
  if (!supported_dim(head_dim)) return BZ_ERR_UNSUPPORTED;
  int cus = 0;
  const int rc = device_cus(&cus);
  if (rc != BZ_OK) return rc;
  *num_splits = default_splits_for(batch * num_kv_heads, head_dim, effective_len(capacity, max_seq_len), cus);
  return BZ_OK;
}

__attribute__((visibility("default"))) const char* bz_status_string(int status) {
  switch (status) {
    case BZ_OK: return "ok";
    case BZ_ERR_NULL: return "a required pointer is NULL";
    case BZ_ERR_SHAPE: return "a size is out of range (or num_q_heads is not a multiple of num_kv_heads)";
    case BZ_ERR_UNSUPPORTED:
      return "unsupported head_dim (64, 128; 128 for the fused prologue) or GQA group size (1, 2, 4, 8)";
    case BZ_ERR_ALIGNMENT: return "K/V pointers and strides must be 16-byte aligned, workspace 256-byte aligned";
    case BZ_ERR_WORKSPACE: return "workspace missing or smaller than bz_gqa_decode_workspace_size()";
    case BZ_ERR_MASK_DTYPE: return "mask_dtype must be BZ_MASK_BF16 or BZ_MASK_F32 when a mask is given";
    case BZ_ERR_LAUNCH: return "kernel launch failed";
    case BZ_ERR_DEVICE: return "HIP device query failed";
    case BZ_ERR_COMBINE_MODE: return "combine must be BZ_COMBINE_AUTO, _LAST_BLOCK or _KERNEL";
    case BZ_ERR_SCRATCH:
      return "bz_gqa_decode_noalloc: more than 1024 (row, kv head) groups or 8 MiB of split partials for its static "
             "scratch; use bz_gqa_decode with a workspace";
    default: return "unknown status";
  }
}

__attribute__((visibility("default"))) int bz_gqa_decode_abi_version(void) { return BZ_GQA_DECODE_ABI_VERSION; }

#ifndef BZ_BUILD_ID
#define BZ_BUILD_ID "unknown"
#endif
__attribute__((visibility("default"))) const char* bz_gqa_decode_build_id(void) { return BZ_BUILD_ID; }

}  // extern "C"
