// Device code of the MI355X (gfx950) GQA flash-decoding attention, shared by the translation units of
// libbz_gqa_decode.so (gqa_decode.hip: C ABI and plain kernels; gqa_fused.hip: kernels with the fused prologue).
//
// What it computes is the reference's decode attention (flash/csrc/bb_attn.cu:1-17, the eager chain of
// third_party/breeze-tts/models/breeze.py:259-286 with the head map of repeat_kv, :245-256): for each row b and
// q head h, softmax(scale * q . K^T + mask) . V over the KV positions [kv_start[b], seq_lens[b]) of KV head
// h / G, in fp32 (the north-star oracle), not the reference's bf16 rounding chain. The fused variant first applies
// the reference's prologue (bb_attn.cu:78-149): q_norm / k_norm (Qwen3 RMSNorm) and RoPE on the raw projections at
// the eager bf16 rounding points, and writes the new k and v into cache slot cache_pos.
//
// Work decomposition (split-K over the KV length, "flash-decoding"):
//   grid (splits, num_kv_heads, batch), NT = 256 threads (4 wave64) per workgroup.
//   Each row's valid length is cut on the device into nact <= splits chunks of
//   chunk = max(min_chunk, ceil(len / splits)) positions (one chunk for a row whose K+V span is at most 64 KB), so a
//   fixed grid serves every length (HIP-graph safe) and the work follows the real length: workgroups past nact exit
//   at once.
//   A workgroup streams its chunk in tiles of ROWS * PPT positions, two tiles in flight (ping-pong). A KV row of
//   head_dim bf16 is read by LPR = head_dim / 8 consecutive lanes, 16 bytes each, so one wave64 load instruction
//   covers 64 * 16 B of consecutive positions and every K/V byte is read once, by one lane, straight into VGPRs.
//   All G q heads of the GQA group use the same K/V registers.
//   q . k: four v_dot2c_f32_bf16 per head on the packed bf16 words, then a 16- (or 8-) lane DPP row sum.
//   Softmax: online, base 2 (scale * log2(e) applied to the score), one running max per wave (the rows of a wave
//   take the tile max across rows with lane swaps), per-row running sums and accumulators. At the end of the chunk
//   the rows of a wave are summed with lane swaps and the waves are merged through LDS (log-sum-exp rule).
//   One chunk (nact == 1): the workgroup writes the bf16 output directly. Several: each writes (acc[D], max, sum) in
//   fp32 to the workspace and the last workgroup of the (batch, kv head) to arrive merges them in split order (or,
//   on request, a second kernel does).
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "bz_gqa_decode.h"
#include "device_common.cuh"

namespace bz {

struct Params {
  const uint16_t* q;
  int64_t q_sb, q_sh, q_st;  // batch, head and token strides of q
  int T;                     // query tokens per row (the last T positions of the row, causal among themselves)
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sb, kv_sh, kv_ss;
  const int32_t* seq_lens;
  const int32_t* kv_start;
  const void* mask;
  int64_t m_sb;
  float scale_log2;  // scale * log2(e)
  uint16_t* out;
  int64_t o_sb, o_sh, o_st;
  int B, NH, NKV, cap, splits, min_chunk;
  float inv_splits;  // 1 / splits rounded to float (split_chunk's quotient estimate)
  int G;             // NH / NKV
  int mask_kind;     // bz_mask_dtype of mask (for the merge kernel, which is not templated on it)
  int combine_last;  // 1: last workgroup of each (b, kv head) merges the splits
  float* part_acc;   // [B * T, NKV, splits, G * D]  unnormalised sum_p 2^(s_p - m) v_p
  float2* part_ml;   // [B * T, NKV, splits, G]      (m, sum_p 2^(s_p - m))
  int* counters;     // [B * T, NKV] x kCounterStride arrivals, reset by the merging workgroup
  // fused prologue only
  const uint16_t* qkv;  // [B, (NH + 2 NKV) * D] raw projections: q heads | k heads | v heads
  int64_t qkv_sb;
  const uint16_t* qn_w;  // [D]
  const uint16_t* kn_w;  // [D]
  float eps;
  const uint16_t* cos;  // [B, D]
  const uint16_t* sin;
  int64_t cs_sb;
  const int64_t* cache_pos;  // device scalar: cache slot of the new k / v
  uint16_t* k_out;  // the caches, written at cache_pos
  uint16_t* v_out;
};

// The split kernels take the rows' range arrays (seq_lens, kv_start) as leading kernel arguments ahead of the
// parameter block, and so does the number of query tokens per row, which the row index (and so the address of its
// range) depends on: built with kernel-argument preloading (-mllvm -amdgpu-kernarg-preload-count), the leading
// scalar arguments of a kernel (up to 56 bytes; a struct argument is never preloaded) arrive in SGPRs with the wave,
// so the range loads go out at once, together with the loads of the argument buffer rather than after one. Without
// preloading they are read from the argument buffer like the rest.
using SplitFn = void (*)(const int32_t*, const int32_t*, int, const Params);
using CombineFn = void (*)(const Params);

// Kernel tables (gqa_fused.hip defines the fused one).
SplitFn pick_split_fused(int D, int G, int mk, int ppt, int nt);

}  // namespace bz

namespace {

using bz::Params;
using bz::SplitFn;
using bz::CombineFn;


constexpr int kThreads = 256;  // 4 wave64 (merge and mask kernels)
// Threads per split workgroup: four waves. Eight (two per SIMD, one workgroup per CU at B = 2) measured slower once
// the loads, reductions and merge took their present form: config 2 6.45 against 6.39 us, config 3 9.84 against 9.62.
constexpr int kSplitThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxSplits = 256;
constexpr int kMaxDevices = 64;
constexpr int kCounterStride = 64;  // ints: one 256-byte line per arrival counter (atomics to one line serialize)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kExcluded = -1e30f;  // mask values <= this exclude the position (bb_attn.cu:9-11, :115)

// ---------------------------------------------------------------------------------------------- helpers

// Value of the lane holding the same 8 dims +/- head_dim / 2 (rotate_half's partner): LPR / 2 lanes away inside the
// row; row_ror:8 for head_dim 128, a bpermute for head_dim 64.
template <int LPR>
__device__ __forceinline__ float half_partner(float x) {
  if constexpr (LPR == 16) return lane_xor8(x);
  else return __shfl_xor(x, LPR / 2);
}

// Qwen3 per-head RMSNorm then RoPE on this lane's 8 dims (dims 8c .. 8c + 7 of a head spread over LPR lanes), at the
// eager rounding points of transformers' Qwen3RMSNorm + apply_rotary_pos_emb, which bb_attn.cu:78-100 reproduces:
//   h = bf16(x * rsqrt(mean(x^2) + eps));  y = bf16(w * h);
//   out = bf16(bf16(y * cos) + bf16(rotate_half(y) * sin)),  rotate_half(y) = [-y[D/2:], y[:D/2]].
// Returns the 8 results as packed bf16 pairs.
template <int LPR>
__device__ __forceinline__ uint4 norm_rope8(const uint4& xr, const uint4& wr, const uint4& cr, const uint4& sr,
                                            float eps, int c) {
  float x[8], w[8], cs[8], sn[8];
  unpack8(xr, x);
  unpack8(wr, w);
  unpack8(cr, cs);
  unpack8(sr, sn);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss = fmaf(x[j], x[j], ss);
  ss = row_sum<LPR>(ss);
  const float inv_rms = rsqrtf(ss * (1.f / (8 * LPR)) + eps);
  float y[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = x[j] * inv_rms;
  round8(y);
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] *= w[j];
  round8(y);
  const bool first_half = c < LPR / 2;
  float yc[8], ys[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float partner = half_partner<LPR>(y[j]);
    yc[j] = y[j] * cs[j];
    ys[j] = (first_half ? -partner : partner) * sn[j];
  }
  round8(yc);
  round8(ys);
  return make_uint4(pack_bf16x2(yc[0] + ys[0], yc[1] + ys[1]), pack_bf16x2(yc[2] + ys[2], yc[3] + ys[3]),
                    pack_bf16x2(yc[4] + ys[4], yc[5] + ys[5]), pack_bf16x2(yc[6] + ys[6], yc[7] + ys[7]));
}

// The four dwords of x from lane src_lane of the wave (ds_bpermute through the LDS crossbar; no LDS storage).
__device__ __forceinline__ uint4 lane_fetch4(const uint4& x, int src_lane) {
  const int a = src_lane * 4;
  return make_uint4((uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)x.x), (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)x.y),
                    (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)x.z), (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)x.w));
}

// The row's range from its raw seq_lens / kv_start values, clamped so that no access can leave [0, capacity).
__device__ __forceinline__ void clamp_range(const Params& p, int e_raw, int s_raw, int& start, int& end) {
  const int e = e_raw < 0 ? 0 : (e_raw > p.cap ? p.cap : e_raw);
  start = p.kv_start == nullptr || s_raw < 0 ? 0 : (s_raw > e ? e : s_raw);
  end = e;
}

__device__ __forceinline__ void row_range(const Params& p, int b, int& start, int& end) {
  // both loads are issued before either is waited for: without kv_start the second one reads seq_lens again and its
  // value is dropped (a conditional load would wait for the first before issuing the second)
  const int32_t* ks = p.kv_start ? p.kv_start : p.seq_lens;
  clamp_range(p, p.seq_lens[b], ks[b], start, end);
}

// Range of query token t of a row whose range is [start, end): the row's tokens are its last T positions, each
// attending up to itself, so token t ends T - 1 - t positions before the row (flash/csrc/depth_frame.cu:221-227:
// token t of step 0 attends 0..t).
__device__ __forceinline__ int token_end(const Params& p, int t, int start, int end) {
  return max(start, end - (p.T - 1 - t));
}

// A row whose K+V span is at most kOneSplitBytes runs as one split whatever the grid: the cross-workgroup merge of two
// or more splits (partials stored, counted, reloaded: about 2 us) costs more than one workgroup takes to stream that
// much. The host's default split count applies the same bound to the capacity (or max_seq_len); here it applies to
// each row's actual length, so a captured grid sized for the capacity serves the early, short steps too.
constexpr int kOneSplitBytes = 64 * 1024;
template <int D>
constexpr int one_split_len() { return kOneSplitBytes / (4 * D); }

// Positions per split and number of non-empty splits for a row of length len (>= 1 split even when empty, so
// that someone writes the row's output).
// ceil(n / d) for 0 <= n < 2^24 without an integer division (about 30 dependent instructions): inv_d is 1 / d within
// one ulp (rounded, or v_rcp_f32), and d >= 2 or inv_d exactly 1, so the float quotient is within one of floor(n / d)
// and one correction step makes it exact (checked on the CPU against integer division for d up to 4096 with both
// neighbours of the rounded 1 / d)
__device__ __forceinline__ int ceil_div_est(int n, int d, float inv_d) {
  int q = (int)((float)n * inv_d);
  int r = n - q * d;
  q = r < 0 ? q - 1 : (r >= d ? q + 1 : q);
  r = n - q * d;
  return q + (r > 0);
}

template <int D>
__device__ __forceinline__ int split_chunk(int len, int splits, float inv_splits, int min_chunk) {
  if (len <= one_split_len<D>()) return len > min_chunk ? len : min_chunk;
  const int c = ceil_div_est(len, splits, inv_splits);
  return c > min_chunk ? c : min_chunk;
}
__device__ __forceinline__ int split_count(int len, int chunk) { return len > 0 ? (len + chunk - 1) / chunk : 1; }

template <int MK>
__device__ __forceinline__ float load_mask(const void* m, int64_t off) {
  if (MK == BZ_MASK_BF16) return bf16_to_f32(static_cast<const uint16_t*>(m)[off]);
  return static_cast<const float*>(m)[off];
}

// Split partials cross workgroups (and XCDs, each with its own L2) inside one launch, so they are written and read
// as agent-scope relaxed atomics: on gfx950 these are sc1 accesses that write through to, and read from, the level
// where all XCDs are coherent, with no L2 writeback or invalidate of the whole cache.
__device__ __forceinline__ void st_agent(float* ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge the nact split partials of the G q heads of kv head h in split order and write the bf16 output. tpr: query
// tokens per row (p.T; the split kernel has it in an SGPR from the launch, so a row index needs no division at T = 1).
// The partials of one (row, kv head) are read through buffer resources cut at nact splits, with the sc1 cache policy
// (bit 4 of the buffer instruction's cache-policy operand on gfx940 and later: the cache behaviour of an agent-scope
// relaxed atomic load), so every load is unconditional and splits past nact read 0 without a memory access. All loads
// are issued before anything waits: each thread's first kBatch partials for its kOut (q head, dim) outputs, and the
// (max, sum) pairs of q head `wave` (one lane per split). Split weights w_s = 2^(m_s - M) / sum_s 2^(m_s - M) l_s are
// reduced over the wave and stored to LDS zero-padded, so the weighted sum needs no per-split condition.
// The partials are left in place: each is written before it is read in every call, and only the counters need to
// start at zero (clearing the partials as well, so that the whole workspace is zero between calls, cost 0.26 us per
// call at the serving shape and 0.5 us on the ragged batch).
template <int D, int G, int NT>
__device__ void merge_splits(const Params& p, int z, int h, int nact, int tpr) {
  constexpr int kBatch = 16;
  constexpr int NW = NT / kWave;
  constexpr int kOut = (G * D + NT - 1) / NT;
  constexpr int kPerLane = kMaxSplits / kWave;
  constexpr int GD = G * D;
  __shared__ __align__(16) float s_w[G][kMaxSplits];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int64_t unit = (int64_t)z * p.NKV + h;
  const Rsrc racc = span_rsrc(p.part_acc + unit * p.splits * GD, nact * GD * 4);
  const Rsrc rml = span_rsrc(p.part_ml + unit * p.splits * G, nact * G * 8);
  const int b = tpr == 1 ? z : z / tpr, tok = z - b * tpr;
  uint16_t* const orow = p.out + (int64_t)b * p.o_sb + (int64_t)tok * p.o_st;

  // The (max, sum) pairs of q head wave % G first, by every wave and without a condition (a wave past the group's
  // heads works a head out again and stores nothing): loads complete in issue order, so the split weights are
  // worked out while the accumulators are still on their way.
  using Pair = decltype(__builtin_amdgcn_raw_buffer_load_b64(rml, 0, 0, kSc1));
  Pair raw[kPerLane];
  auto load_ml = [&](int g) {
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      raw[j] = __builtin_amdgcn_raw_buffer_load_b64(rml, ((lane + kWave * j) * G + g) * 8, 0, kSc1);
  };
  load_ml(wave % G);
  // the accumulators, also unconditionally: threads past the group's G * D values (G * D < NT) load one of them
  // again and drop it, so that the compiler's count of loads in flight stays exact
  float t[kOut][kBatch];
#pragma unroll
  for (int k = 0; k < kOut; ++k) {
    const int o = (tid + k * NT) % GD;
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      t[k][u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(racc, (u * GD + o) * 4, 0, kSc1));
  }

  // split weights w_s = 2^(m_s - M) / sum_s 2^(m_s - M) l_s of head g, from the pairs in raw
  auto weights = [&](int g) {
    float mv[kPerLane], lv[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      mv[j] = lane + kWave * j < nact ? __uint_as_float(raw[j][0]) : -INFINITY;
      lv[j] = __uint_as_float(raw[j][1]);  // 0 past nact
    }
    float mloc = mv[0];
#pragma unroll
    for (int j = 1; j < kPerLane; ++j) mloc = fmaxf(mloc, mv[j]);
    const float M = wave_max(mloc);
    const float mu = (M == -INFINITY) ? 0.f : M;
    float lloc = 0.f;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      mv[j] = fast_exp2(mv[j] - mu);  // 0 for the padding (-inf)
      lloc = fmaf(mv[j], lv[j], lloc);
    }
    const float L = wave_sum(lloc);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (wave < G) {  // waves past the group's heads only followed along
#pragma unroll
      for (int j = 0; j < kPerLane; ++j) s_w[g][lane + kWave * j] = mv[j] * inv;
    }
  };
  weights(wave % G);
  for (int g = wave + NW; g < G; g += NW) {  // groups of more q heads than waves
    load_ml(g);
    weights(g);
  }
  __syncthreads();

#pragma unroll
  for (int k = 0; k < kOut; ++k) {
    const int o = tid + k * NT;
    if (o >= GD) continue;
    const int g = o / D;
    float a = 0.f;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) a = fmaf(s_w[g][u], t[k][u], a);
    for (int s0 = kBatch; s0 < nact; s0 += kBatch) {
      float x[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        x[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(racc, ((s0 + u) * GD + o) * 4, 0, kSc1));
#pragma unroll
      for (int u = 0; u < kBatch; ++u) a = fmaf(s_w[g][s0 + u], x[u], a);
    }
    orow[(int64_t)(h * G + g) * p.o_sh + o % D] = f32_to_bf16(a);
  }
}

// Blocks of positions with at least one attended position, recorded while a mask row is scanned: bit i of the
// kValidWords words covers positions [i << shift, (i + 1) << shift), shift >= 6 chosen so that the capacity fits.
constexpr int kValidWords = 64;
__device__ __forceinline__ int valid_shift(int cap) {
  int s = 6;
  while (((cap - 1) >> s) >= 32 * kValidWords) ++s;
  return s;
}
// Whether [lo, hi) holds a block with an attended position (uniform over the workgroup: every thread reads the same
// LDS words).
__device__ __forceinline__ bool any_valid(const uint32_t* bits, int shift, int lo, int hi) {
  if (hi <= lo) return false;
  for (int blk = lo >> shift; blk <= (hi - 1) >> shift; ++blk)
    if (bits[blk >> 5] & (1u << (blk & 31))) return true;
  return false;
}

// [start, end) of mask row b: the first and last position below capacity whose mask value is > -1e30, or [0, 0) if
// there is none (what mask_range_kernel computes, and bz_mask_interval returns). All NT threads of the workgroup
// take part, and all get the result. With bits (kValidWords words of LDS), the blocks holding attended positions are
// recorded there too (valid_shift(cap)), so a workgroup can skip a chunk the mask excludes entirely, as the
// reference skips its fully masked 64-position chunks (bb_attn.cu:9-11, :151-154).
template <int NT, int MK>
__device__ void mask_row_range_t(const Params& p, int b, int& start, int& end, uint32_t* bits) {
  constexpr int kUnroll = 8;  // mask values per thread loaded before any is compared: one round trip per 8 NT
  __shared__ int s_lo[NT / kWave], s_hi[NT / kWave];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int shift = valid_shift(p.cap);
  if (bits != nullptr) {
    for (int i = tid; i < kValidWords; i += NT) bits[i] = 0;
    __syncthreads();
  }
  // the row through a buffer resource cut at the capacity: every load is unconditional (loads past it read 0 and
  // touch no memory), so the compiler issues the kUnroll loads together
  constexpr int kBytes = MK == BZ_MASK_BF16 ? 2 : 4;
  const Rsrc rm = span_rsrc(static_cast<const char*>(p.mask) + (int64_t)b * p.m_sb * kBytes, p.cap * kBytes);
  int lo = p.cap, hi = -1;
  for (int base = 0; base < p.cap; base += kUnroll * NT) {
    float m[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t off = (uint32_t)(base + u * NT + tid) * kBytes;
      m[u] = MK == BZ_MASK_BF16 ? bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(rm, off, 0, 0))
                                : __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, off, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int pos = base + u * NT + tid;
      const bool keep = pos < p.cap && m[u] > kExcluded;
      if (keep) {
        lo = min(lo, pos);
        hi = max(hi, pos);
      }
      // a wave's 64 positions here are one aligned run of 64, inside one block (shift >= 6): one LDS OR per wave
      if (bits != nullptr && __ballot(keep) != 0 && lane == 0) {
        const int blk = (base + u * NT + wave * kWave) >> shift;
        atomicOr(&bits[blk >> 5], 1u << (blk & 31));
      }
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    lo = min(lo, __shfl_xor(lo, off));
    hi = max(hi, __shfl_xor(hi, off));
  }
  if (lane == 0) {
    s_lo[wave] = lo;
    s_hi[wave] = hi;
  }
  __syncthreads();
  lo = s_lo[0];
  hi = s_hi[0];
#pragma unroll
  for (int u = 1; u < NT / kWave; ++u) {
    lo = min(lo, s_lo[u]);
    hi = max(hi, s_hi[u]);
  }
  start = hi >= 0 ? lo : 0;
  end = hi >= 0 ? hi + 1 : 0;
}

// MK: the mask's dtype when the caller is built for one, BZ_MASK_NONE to take it from p.mask_kind.
template <int NT, int MK = BZ_MASK_NONE>
__device__ __forceinline__ void mask_row_range(const Params& p, int b, int& start, int& end, uint32_t* bits = nullptr) {
  if (MK == BZ_MASK_BF16 || (MK == BZ_MASK_NONE && p.mask_kind == BZ_MASK_BF16))
    mask_row_range_t<NT, BZ_MASK_BF16>(p, b, start, end, bits);
  else
    mask_row_range_t<NT, BZ_MASK_F32>(p, b, start, end, bits);
}

// Range of query token t of row b, from seq_lens / kv_start or, when seq_lens is NULL, from the mask row (all NT
// threads of the workgroup must call it then; bits as in mask_row_range).
template <int NT, int MK = BZ_MASK_NONE>
__device__ __forceinline__ void unit_range(const Params& p, int b, int t, int& start, int& end,
                                           uint32_t* bits = nullptr) {
  if (p.seq_lens != nullptr) {
    row_range(p, b, start, end);
  } else {
    mask_row_range<NT, MK>(p, b, start, end, bits);
  }
  end = token_end(p, t, start, end);
}

// One tile of KV rows held in VGPRs: position pos0 + ROWS * i for i < PPT (pos0 = tile start + this lane's row).
template <int PPT>
struct Tile {
  uint4 k[PPT], v[PPT];
  float m[PPT];
};

// The K, V (and mask) spans of one (row, kv head), each cut at position hi: positions >= hi are outside the resource,
// so their loads return zero without reading memory (NaN tails and slots past the row stay unread).
struct Spans {
  Rsrc k, v, m;
  uint32_t row_bytes;  // bytes between consecutive positions of K / V
  uint32_t lane_off;   // this lane's 16 bytes inside a row
};

// Issue every K and V load of a tile (and its mask values) before any arithmetic. K and V are read once per call, so
// their loads carry the non-temporal hint (kStream): the streamed bytes do not push the lengths, q and the split
// workspace out of the L2. The loads are unconditional (the
// resource bounds do the cut at hi), so the compiler's vmcnt accounting stays exact and earlier loads (q, the fused
// prologue's inputs) can be consumed while the tile is still in flight.
template <int ROWS, int PPT, int MK>
__device__ __forceinline__ void load_tile(Tile<PPT>& t, const Spans& sp, int pos0) {
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const uint32_t pos = (uint32_t)(pos0 + ROWS * i);
    const uint32_t off = pos * sp.row_bytes + sp.lane_off;
    t.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(sp.k, off, 0, kStream));
    t.v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(sp.v, off, 0, kStream));
    if (MK == BZ_MASK_BF16) t.m[i] = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(sp.m, pos * 2, 0, 0));
    if (MK == BZ_MASK_F32)
      t.m[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(sp.m, pos * 4, 0, 0));
  }
}

// Fold one tile into the running (max m, sum l, acc) per q head: q.k as four bf16 dot2 per head plus a DPP row sum,
// scaled by scale * log2(e); online softmax in base 2 with one max per wave (m is wave-uniform, l and acc per row);
// then P.V in fp32 on the unpacked V registers.
// A slot whose row lies past hi (or, with LO, before lo) is dropped (the condition is uniform over the row's lanes, and
// the DPP sum reads only lanes of the same row, so whatever the dropped slot holds stays in its own row).
// Fused prologue: the slot newpos (>= 0 only in the workgroup whose chunk holds it) takes the new k / v computed in
// registers; the cache write of this call is not read back.
template <int LPR, int ROWS, int G, int PPT, int MK, bool FUSED, bool LO = false>
__device__ __forceinline__ void consume_tile(Tile<PPT>& t, const uint4 (&qp)[G], float scale_log2, float (&m)[G],
                                             float (&l)[G], float (&acc)[G][8], int pos0, int hi, int newpos,
                                             const uint4& knew, const uint4& vnew, int lo = 0) {
  // No branch: every slot's products are computed and a slot outside the range (or excluded by the mask) is dropped
  // by selects, its score to -inf and its V to 0 (so NaN there reaches neither the sums nor the accumulator through
  // 0 * V). Branches here would also make the compiler's waits for the tile's loads conservative.
  auto sel = [](bool c, const uint4& a, const uint4& b) {
    return make_uint4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
  };
  float s[G][PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int pos = pos0 + ROWS * i;
    bool inc = pos < hi && (!LO || pos >= lo);
    if (FUSED) {
      const bool fresh = pos == newpos;
      t.k[i] = sel(fresh, knew, t.k[i]);
      t.v[i] = sel(fresh, vnew, t.v[i]);
    }
    if (MK != BZ_MASK_NONE) inc = inc && t.m[i] > kExcluded;
    t.v[i] = sel(inc, t.v[i], make_uint4(0, 0, 0, 0));
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float d = dot2_bf16(qp[g].x, t.k[i].x, 0.f);
      d = dot2_bf16(qp[g].y, t.k[i].y, d);
      d = dot2_bf16(qp[g].z, t.k[i].z, d);
      d = dot2_bf16(qp[g].w, t.k[i].w, d);
      d = row_sum<LPR>(d) * scale_log2;
      if (MK != BZ_MASK_NONE) d = fmaf(t.m[i], kLog2e, d);
      s[g][i] = inc ? d : -INFINITY;
    }
  }
  // one running max per wave: the rows of a wave can then be merged by plain sums
  float mt[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mt[g] = s[g][0];
#pragma unroll
    for (int i = 1; i < PPT; ++i) mt[g] = fmaxf(mt[g], s[g][i]);
    if (LPR == 8) mt[g] = fmaxf(mt[g], lane_xor8(mt[g]));
  }
  rows_max<G>(mt);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mn = fmaxf(m[g], mt[g]);
    const float mu = (mn == -INFINITY) ? 0.f : mn;
    const float alpha = fast_exp2(m[g] - mu);
    l[g] *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] *= alpha;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      s[g][i] = fast_exp2(s[g][i] - mu);
      l[g] += s[g][i];
    }
    m[g] = mn;
  }
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    float vf[8];
    unpack8(t.v[i], vf);
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(s[g][i], vf[j], acc[g][j]);
  }
}

// ---------------------------------------------------------------------------------------------- kernels

// lens, starts: p.seq_lens and p.kv_start again, as leading (preloaded) arguments.
template <int D, int G, int PPT, int MK, int NT, bool FUSED>
__global__ void __launch_bounds__(NT) gqa_split_kernel(const int32_t* lens, const int32_t* starts, const int tpr,
                                                       const Params p) {
  constexpr int NW = NT / kWave;        // waves per workgroup
  constexpr int LPR = D / 8;            // lanes per KV row, 16 B (8 bf16) each
  constexpr int ROWS = NT / LPR;        // KV rows per load instruction across the workgroup
  constexpr int TP = ROWS * PPT;        // positions per tile
  constexpr int RPW = kWave / LPR;      // rows per wave
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");

  const int split = blockIdx.x, h = blockIdx.y, z = blockIdx.z;  // z = row * T + token
  // tpr = p.T, preloaded: T = 1 but in the depth step's two-token first step
  const int b = tpr == 1 ? z : z / tpr, tok = z - b * tpr;
  const int tid = threadIdx.x, c = tid % LPR, r = tid / LPR;

  // q of the G heads of this group, this lane's 8 dims, issued first, since none of it depends on the row's length.
  // Fused: the prologue's inputs instead. Its NE = G + 1 heads (the G q heads, then the new k) are spread over the
  // RPW rows of each wave, head e on row e % RPW (slot e / RPW), so a row normalises and rotates NS heads rather than
  // all NE; the results are then fetched across rows.
  constexpr int NE = G + 1;
  constexpr int NS = (NE + RPW - 1) / RPW;
  static_assert(!FUSED || D == 128, "the fused prologue is built for head_dim 128");
  const int rw = (tid % kWave) / LPR;  // row inside the wave
  uint4 qr[G];
  uint4 xe[NS], we[NS], xv, rc, rs;
  int64_t newpos64 = -1;
  // The row's length and start first, ahead of every vector load of the workgroup: the CU's vector memory queue is
  // shared with the workgroups already streaming there (four per CU on a 1024-workgroup grid), and a q load waiting
  // for room in it would hold up these scalar loads behind it in program order. Their addresses come from the
  // preloaded leading arguments (the range arrays, and the token count that gives the row index), so the loads go
  // out together with those of the argument buffer instead of one round trip after them.
  int e_raw = 0, s_raw = 0;
  if (MK == BZ_MASK_NONE) {
    e_raw = lens[b];
    s_raw = (starts ? starts : lens)[b];  // without kv_start: read again and dropped
    __builtin_amdgcn_sched_barrier(0);
  }
  if (FUSED) {
    const uint16_t* row = p.qkv + (int64_t)b * p.qkv_sb + 8 * c;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int e = min(s * RPW + rw, G);  // rows past the last head redo the k head (result unused)
      const int64_t col = e < G ? (int64_t)(h * G + e) * D : (int64_t)(p.NH + h) * D;
      xe[s] = *reinterpret_cast<const uint4*>(row + col);
      we[s] = *reinterpret_cast<const uint4*>((e < G ? p.qn_w : p.kn_w) + 8 * c);
    }
    xv = *reinterpret_cast<const uint4*>(row + (int64_t)(p.NH + p.NKV + h) * D);
    rc = *reinterpret_cast<const uint4*>(p.cos + (int64_t)b * p.cs_sb + 8 * c);
    rs = *reinterpret_cast<const uint4*>(p.sin + (int64_t)b * p.cs_sb + 8 * c);
    newpos64 = p.cache_pos[0];
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint16_t* qsrc = p.q + (int64_t)b * p.q_sb + (int64_t)tok * p.q_st + (int64_t)(h * G + g) * p.q_sh + 8 * c;
      qr[g] = *reinterpret_cast<const uint4*>(qsrc);  // 16-byte aligned: the host checks q and its strides
    }
  }

  int start, end;
  __shared__ uint32_t s_valid[MK != BZ_MASK_NONE ? kValidWords : 1];
  if (MK == BZ_MASK_NONE) {
    // without a mask the row's range always comes from seq_lens (the host passes it); keeping the mask scan out of
    // this instantiation takes 2.3 KB of never-run code out of the kernel (5.9 KB instead of 8.2 at the serving
    // shape), which measured 2-4% faster
    clamp_range(p, e_raw, s_raw, start, end);
    end = token_end(p, tok, start, end);
  } else {
    unit_range<NT, MK>(p, b, tok, start, end, s_valid);
  }
  const int len = end - start;
  const int chunk = split_chunk<D>(len, p.splits, p.inv_splits, p.min_chunk);
  if (split > 0 && split * chunk >= len) return;  // past the row's last non-empty chunk (split 0 always stays)
  const int lo = start + split * chunk;
  const int hi_chunk = min(lo + chunk, end);
  // A chunk whose every position the mask excludes streams nothing (its partial is empty: max -inf, sum 0); the
  // scan of the mask row recorded which blocks of positions hold an attended one. hi_chunk still decides which
  // workgroup owns the fused step's cache slot.
  const bool skip = MK != BZ_MASK_NONE && p.seq_lens == nullptr &&
                    !any_valid(s_valid, valid_shift(p.cap), lo, hi_chunk);
  const int hi = skip ? lo : hi_chunk;

  Spans sp;
  {
    const int64_t head_off = (int64_t)b * p.kv_sb + (int64_t)h * p.kv_sh;
    sp.row_bytes = (uint32_t)p.kv_ss * 2;
    sp.lane_off = 16 * c;
    const int span = hi * (int)sp.row_bytes;  // < 2^31: the host bounds (capacity + 1024) * kv_stride_s * 2
    sp.k = span_rsrc(p.k + head_off, span);
    sp.v = span_rsrc(p.v + head_off, span);
    if (MK == BZ_MASK_BF16) sp.m = span_rsrc(static_cast<const uint16_t*>(p.mask) + (int64_t)b * p.m_sb, 2 * hi);
    if (MK == BZ_MASK_F32) sp.m = span_rsrc(static_cast<const float*>(p.mask) + (int64_t)b * p.m_sb, 4 * hi);
  }

  // The first two tiles' K/V loads go out before q is converted, so no wave waits on
  // q before streaming. Tiles A and B ping-pong without register copies: while one is consumed the other's loads
  // are in flight. Loads of positions >= hi fall outside the spans and make no memory access, so a one-tile chunk
  // issues no extra traffic.
  Tile<PPT> ta, tb;
  load_tile<ROWS, PPT, MK>(ta, sp, lo + r);
  load_tile<ROWS, PPT, MK>(tb, sp, lo + TP + r);
  // keep the machine scheduler from sinking the tile loads below the q / prologue arithmetic (which would make that
  // arithmetic wait for its own inputs before any K/V load is in flight)
  __builtin_amdgcn_sched_barrier(0);
  // non-empty chunks of the row (1 for an empty row); without a branch, which would make the compiler wait for the
  // tiles before the q / prologue arithmetic below (chunk >= min_chunk >= 32)
  const int nact = ceil_div_est(max(len, 1), chunk, __builtin_amdgcn_rcpf((float)chunk));

  uint4 qp[G], knew = make_uint4(0, 0, 0, 0), vnew = make_uint4(0, 0, 0, 0);
  int newpos = -1;
  if (FUSED) {
    uint4 ye[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) ye[s] = norm_rope8<LPR>(xe[s], we[s], rc, rs, p.eps, c);
    static_assert(RPW * LPR == kWave, "a wave holds whole rows");
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const uint4 y = lane_fetch4(ye[e / RPW], (e % RPW) * LPR + c);  // head e from lane c of row e % RPW
      if (e < G) qp[e] = y;
      else knew = y;
    }
    vnew = xv;
    if (newpos64 >= 0 && newpos64 < p.cap) {
      const int pos = (int)newpos64;
      // one writer per (row, kv head): the workgroup whose chunk holds the slot, or split 0 when the slot lies
      // outside the row's attended range; only that workgroup can read the slot in this call, from registers
      const bool in_range = pos >= start && pos < end;
      const bool owner = in_range ? (pos >= lo && pos < hi_chunk) : (split == 0);
      if (owner) {
        if (in_range) newpos = pos;
        if (tid < LPR) {
          const int64_t off = (int64_t)b * p.kv_sb + (int64_t)h * p.kv_sh + (int64_t)pos * p.kv_ss + 8 * c;
          *reinterpret_cast<uint4*>(p.k_out + off) = knew;
          *reinterpret_cast<uint4*>(p.v_out + off) = vnew;
        }
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) qp[g] = qr[g];
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  }

  for (int t0 = lo; t0 < hi; t0 += 2 * TP) {
    consume_tile<LPR, ROWS, G, PPT, MK, FUSED>(ta, qp, p.scale_log2, m, l, acc, t0 + r, hi, newpos, knew, vnew);
    if (t0 + TP >= hi) break;
    load_tile<ROWS, PPT, MK>(ta, sp, t0 + 2 * TP + r);
    consume_tile<LPR, ROWS, G, PPT, MK, FUSED>(tb, qp, p.scale_log2, m, l, acc, t0 + TP + r, hi, newpos, knew, vnew);
    load_tile<ROWS, PPT, MK>(tb, sp, t0 + 3 * TP + r);
  }

  // merge the RPW rows of each wave (lanes c, c + LPR, c + 2 LPR, ... hold the same dims): the G * 8 accumulators and
  // G sums, zero-padded to NQ groups of four, are summed across rows transposed, so row r of red[q] holds the wave's
  // total of value 4 q + r (for head_dim 64 the two 8-lane rows of each 16-lane row are added first)
  constexpr int NV = 9 * G, NQ = (NV + 3) / 4;
  float flat[4 * NQ];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int j = 0; j < 8; ++j) flat[8 * g + j] = acc[g][j];
    flat[8 * G + g] = l[g];
  }
#pragma unroll
  for (int v = NV; v < 4 * NQ; ++v) flat[v] = 0.f;
  if (LPR == 8) {
#pragma unroll
    for (int v = 0; v < NV; ++v) flat[v] += lane_xor8(flat[v]);
  }
  float red[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) red[q] = rows_sum4(flat[4 * q], flat[4 * q + 1], flat[4 * q + 2], flat[4 * q + 3]);

  // merge the NW waves through LDS
  __shared__ float s_acc[NW][G][D];
  __shared__ float s_m[NW][G], s_l[NW][G];
  const int w = tid / kWave, lane = tid % kWave, row16 = lane / 16;
  if (lane % 16 < LPR) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int f = 4 * q + row16;
      if (f < 8 * G) s_acc[w][f / 8][8 * c + f % 8] = red[q];
      else if (f < NV && c == 0) s_l[w][f - 8 * G] = red[q];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) s_m[w][g] = m[g];
  }
  __syncthreads();
  (void)RPW;

  for (int o = tid; o < G * D; o += NT) {
    const int g = o / D, d = o % D, hq = h * G + g;
    float M = s_m[0][g];
#pragma unroll
    for (int u = 1; u < NW; ++u) M = fmaxf(M, s_m[u][g]);
    const float mu = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float e = fast_exp2(s_m[u][g] - mu);
      L = fmaf(e, s_l[u][g], L);
      A = fmaf(e, s_acc[u][g][d], A);
    }
    if (nact == 1) {
      p.out[(int64_t)b * p.o_sb + (int64_t)tok * p.o_st + (int64_t)hq * p.o_sh + d] =
          f32_to_bf16(L > 0.f ? A / L : 0.f);
    } else {
      const int64_t ps = ((int64_t)z * p.NKV + h) * p.splits + split;  // this split of this (row, kv head)
      st_agent(p.part_acc + ps * (G * D) + o, A);
      if (d == 0) {
        st_agent(reinterpret_cast<float*>(p.part_ml + ps * G + g), M);
        st_agent(reinterpret_cast<float*>(p.part_ml + ps * G + g) + 1, L);
      }
    }
  }
  if (nact == 1 || !p.combine_last) return;

  // Last-arriving workgroup of this (b, kv head) merges the splits. Each wave waits until its agent-scope partial
  // stores have completed (s_waitcnt vmcnt(0); gfx9 encoding with expcnt/lgkmcnt left open), the barrier collects
  // the waves, and thread 0 counts the workgroup in with one agent-scope RMW. The workgroup that brings the
  // count to nact reads the partials with agent-scope loads; it resets the counter for the next call.
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0x0f70);
  __syncthreads();
  if (tid == 0) {
    int* cnt = p.counters + ((int64_t)z * p.NKV + h) * kCounterStride;
    const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == nact - 1);
    if (s_last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  merge_splits<D, G, NT>(p, z, h, nact, tpr);
}

// Second-launch merge: one workgroup per (kv head, row).
template <int D, int G>
__global__ void __launch_bounds__(kThreads) gqa_combine_kernel(const Params p) {
  const int h = blockIdx.x, z = blockIdx.y;  // z = row * T + token
  int start, end;
  unit_range<kThreads>(p, z / p.T, z % p.T, start, end);
  const int len = end - start;
  const int nact = split_count(len, split_chunk<D>(len, p.splits, p.inv_splits, p.min_chunk));
  if (nact == 1) return;  // the split kernel wrote the output
  merge_splits<D, G, kThreads>(p, z, h, nact, p.T);
}

// Interval of the additive mask row: first and last position with value > -1e30.
template <int MK>
__global__ void __launch_bounds__(kThreads) mask_range_kernel(const void* mask, int64_t m_sb, int cap,
                                                              int32_t* start, int32_t* end) {
  const int b = blockIdx.x, tid = threadIdx.x;
  int lo = cap, hi = -1;
  for (int pos = tid; pos < cap; pos += kThreads) {
    if (load_mask<MK>(mask, (int64_t)b * m_sb + pos) > kExcluded) {
      lo = min(lo, pos);
      hi = max(hi, pos);
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    lo = min(lo, __shfl_xor(lo, off));
    hi = max(hi, __shfl_xor(hi, off));
  }
  __shared__ int s_lo[kWaves], s_hi[kWaves];
  if (tid % kWave == 0) {
    s_lo[tid / kWave] = lo;
    s_hi[tid / kWave] = hi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int u = 1; u < kWaves; ++u) {
      lo = min(lo, s_lo[u]);
      hi = max(hi, s_hi[u]);
    }
    const bool any = hi >= 0;
    start[b] = any ? lo : 0;
    end[b] = any ? hi + 1 : 0;
  }
}

// Max (is_max) or sum of x over the kThreads threads of the workgroup; every thread gets the result.
__device__ __forceinline__ float block_reduce(float x, bool is_max) {
  __shared__ float s_red[kWaves];
  x = is_max ? wave_max(x) : wave_sum(x);
  __syncthreads();  // s_red may still be read by a previous reduction
  if (threadIdx.x % kWave == 0) s_red[threadIdx.x / kWave] = x;
  __syncthreads();
  float r = s_red[0];
#pragma unroll
  for (int u = 1; u < kWaves; ++u) r = is_max ? fmaxf(r, s_red[u]) : r + s_red[u];
  return r;
}

// The softmax probabilities of one decode step: the reference's optional dbg output (bb_attn.cu:74, :288-289,
// :323-325), for verification. One workgroup per (q head, row) writes probs[(b * NH + hq) * cap + pos] for every
// pos < cap: bf16(2^(s - M) / L) as fp32 inside the row's range, where s is the scaled score (plus the mask's value)
// and M, L the max and the sum over the range, and 0 at excluded positions and outside the range. Three passes
// through probs itself (scores, exponentials, normalised); each thread rereads only the positions it wrote.
// FUSED: the step of bz_gqa_decode_fused, after it ran: q is the head's raw projection in qkv, normed and rotated
// here as the fused kernel does it (norm_rope8, by the first D / 8 lanes, into LDS), and the cache already holds the
// step's new k at cache_pos.
template <int D, int MK, bool FUSED>
__global__ void __launch_bounds__(kThreads) gqa_probs_kernel(const Params p, float* probs) {
  static_assert(!FUSED || D == 128, "the fused prologue is built for head_dim 128");
  const int hq = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int h = hq / p.G;
  __shared__ __align__(16) uint16_t s_q[D];
  const uint16_t* qh = p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh;
  if constexpr (FUSED) {
    constexpr int LPR = D / 8;
    if (tid < LPR) {  // one 16-lane DPP row of wave 0: lane c holds dims 8c .. 8c + 7
      const uint4 x = *reinterpret_cast<const uint4*>(p.qkv + (int64_t)b * p.qkv_sb + (int64_t)hq * D + 8 * tid);
      const uint4 w = *reinterpret_cast<const uint4*>(p.qn_w + 8 * tid);
      const uint4 rc = *reinterpret_cast<const uint4*>(p.cos + (int64_t)b * p.cs_sb + 8 * tid);
      const uint4 rs = *reinterpret_cast<const uint4*>(p.sin + (int64_t)b * p.cs_sb + 8 * tid);
      *reinterpret_cast<uint4*>(s_q + 8 * tid) = norm_rope8<LPR>(x, w, rc, rs, p.eps, tid);
    }
    __syncthreads();
    qh = s_q;
  }
  int start, end;
  unit_range<kThreads, MK>(p, b, 0, start, end);
  float* const row = probs + ((int64_t)b * p.NH + hq) * p.cap;
  const uint16_t* const kb = p.k + (int64_t)b * p.kv_sb + (int64_t)h * p.kv_sh;
  float mx = -INFINITY;
  for (int pos = tid; pos < p.cap; pos += kThreads) {
    float s = -INFINITY;
    if (pos >= start && pos < end) {
      const uint16_t* const kr = kb + (int64_t)pos * p.kv_ss;
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < D; j += 8) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kr + j);
        const uint4 qv = *reinterpret_cast<const uint4*>(qh + j);
        d = dot2_bf16(qv.x, kv.x, d);
        d = dot2_bf16(qv.y, kv.y, d);
        d = dot2_bf16(qv.z, kv.z, d);
        d = dot2_bf16(qv.w, kv.w, d);
      }
      s = d * p.scale_log2;
      if (MK != BZ_MASK_NONE) {
        const float m = load_mask<MK>(p.mask, (int64_t)b * p.m_sb + pos);
        s = m > kExcluded ? fmaf(m, kLog2e, s) : -INFINITY;
      }
    }
    row[pos] = s;
    mx = fmaxf(mx, s);
  }
  const float M = block_reduce(mx, true);
  const float mu = (M == -INFINITY) ? 0.f : M;
  float sum = 0.f;
  for (int pos = tid; pos < p.cap; pos += kThreads) {
    const float e = fast_exp2(row[pos] - mu);  // 0 for -inf
    row[pos] = e;
    sum += e;
  }
  const float L = block_reduce(sum, false);
  for (int pos = tid; pos < p.cap; pos += kThreads) row[pos] = L > 0.f ? bf16_to_f32(f32_to_bf16(row[pos] / L)) : 0.f;
}

// ---------------------------------------------------------------------------------------------- kernel tables

template <int D, int G, int MK, int NT, bool FUSED>
SplitFn pick_ppt(int ppt) {
  switch (ppt) {
    case 1: return gqa_split_kernel<D, G, 1, MK, NT, FUSED>;
    default: return gqa_split_kernel<D, G, 2, MK, NT, FUSED>;
  }
}

template <int D, int G, int NT, bool FUSED>
SplitFn pick_mask(int mk, int ppt) {
  switch (mk) {
    case BZ_MASK_BF16: return pick_ppt<D, G, BZ_MASK_BF16, NT, FUSED>(ppt);
    case BZ_MASK_F32: return pick_ppt<D, G, BZ_MASK_F32, NT, FUSED>(ppt);
    default: return pick_ppt<D, G, BZ_MASK_NONE, NT, FUSED>(ppt);
  }
}

template <int D, int NT, bool FUSED>
SplitFn pick_group(int G, int mk, int ppt) {
  switch (G) {
    case 1: return pick_mask<D, 1, NT, FUSED>(mk, ppt);
    case 2: return pick_mask<D, 2, NT, FUSED>(mk, ppt);
    case 4: return pick_mask<D, 4, NT, FUSED>(mk, ppt);
    case 8: return pick_mask<D, 8, NT, FUSED>(mk, ppt);
    default: return nullptr;
  }
}

}  // namespace
