// Wave-level GQA decode attention: a device function for kernels that run a whole decode step in one launch (a
// persistent depth-transformer kernel of the reference's kind, flash/csrc/depth_frame.cu:193-272, whose attention
// stage gives each warp one (row, q head) pair over at most 17 cached positions). Here too one wave owns one (row,
// q head), and the K/V bytes go from the cache straight into VGPRs (no LDS staging, no barrier), so the caller may run
// it from any wave of any workgroup, with other waves busy elsewhere (tests/csrc/wave_stage.hip runs it so, beside
// waves streaming a scratch buffer through LDS). Any length works; it is built for short ones
// (two tiles of 4 * 64 / (D / 8) positions: 32 at head_dim 128).
//
// The q heads of a group read the same K/V bytes, each through its own wave (from the L2 after the first). A wave that
// owned a whole group instead, sharing each K/V load among its G heads, measured slower: its serial chain of dot
// products, row sums and softmax steps grows with G while the bytes are few (real depth shape, 8 q / 2 KV heads,
// lengths 2..17: 2.9 against 4.6 us per launch; config-5 frame: 2.64 against 3.21 us per launch).
//
// The arithmetic is the split kernel's (gqa_kernels.cuh: load_tile, consume_tile): bf16 dot2 products with fp32
// accumulation, online softmax in base 2 with one running max per wave, fp32 P.V; then the rows of the wave are summed
// (the max is wave-uniform, so plain sums merge them) and the first row writes bf16(acc * (1 / sum)), or 0 for an
// empty range.
#pragma once

#include "gqa_kernels.cuh"

namespace {

// Everything one wave needs: element pointers and strides, no batch or head indexing left to do.
struct WaveAttention {
  const uint16_t* q;   // the q head: D bf16 (16-byte aligned)
  const uint16_t* k;   // K and V of its kv head in this row: position p at k + p * kv_ss (16-byte aligned rows)
  const uint16_t* v;
  int64_t kv_ss;
  int cap;             // positions [0, cap) of k / v are readable; cap * kv_ss * 2 < 2^31
  float scale_log2;    // softmax scale * log2(e)
  uint16_t* out;       // D bf16 (16-byte aligned)
};

// Sum of x over the rows of the wave (LPR lanes per row): every lane ends with its column's total.
template <int LPR>
__device__ __forceinline__ float rows_total(float x) {
  if constexpr (LPR == 8) x += lane_xor8(x);
  float y = x;
  swap16(x, y);
  x += y;
  y = x;
  swap32(x, y);
  return x + y;
}

// Called by all 64 lanes of one wave (wave-uniform arguments). range(start, end) gives the attended positions
// [start, end), 0 <= start <= end <= cap; it is called once the first K / V loads are issued, so that whatever memory
// it reads is in flight together with them.
//
// The wave reads K / V in tiles of TP positions at absolute positions (tile k holds [k TP, (k + 1) TP)) and masks
// what lies outside [start, end). The first two tiles (positions [0, 2 TP): 32 at head_dim 128, 64 at head_dim 64,
// every length the automatic route sends here) are loaded together with q before the range is known: in a launch
// this short the range (a load of seq_lens that depends on the kernel arguments) and the K / V tiles were two
// dependent memory round trips, and now they overlap. A range past those tiles reloads them at its own start; longer
// ranges stream further tiles two at a time.
template <int D, class Range>
__device__ void attend_wave(const WaveAttention& a, Range range) {
  constexpr int G = 1;  // one q head per wave: the group size of the shared tile code (consume_tile)
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  constexpr int LPR = D / 8, RPW = kWave / LPR, PPT = 4, TP = RPW * PPT;
  const int lane = __lane_id(), r = lane / LPR, c = lane % LPR;
  // the arguments are wave-uniform; taking them through a scalar register keeps the buffer resources and the loop
  // bounds scalar whatever the caller derived them from
  const int64_t kv_ss = wave_uniform(a.kv_ss);
  const int cap = wave_uniform(a.cap);
  uint16_t* const outp = wave_uniform(a.out);

  Spans sp;
  sp.row_bytes = (uint32_t)kv_ss * 2;
  sp.lane_off = 16 * c;
  sp.k = span_rsrc(wave_uniform(a.k), cap * (int)sp.row_bytes);
  sp.v = span_rsrc(wave_uniform(a.v), cap * (int)sp.row_bytes);
  Tile<PPT> ta, tb;
  load_tile<RPW, PPT, BZ_MASK_NONE>(ta, sp, r);
  load_tile<RPW, PPT, BZ_MASK_NONE>(tb, sp, TP + r);
  const Rsrc rq = span_rsrc(wave_uniform(a.q), D * 2);
  const uint4 qp[G] = {__builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, (uint32_t)(16 * c), 0, 0))};
  __builtin_amdgcn_sched_barrier(0);

  int start = 0, end = 0;
  range(start, end);
  start = wave_uniform(start);
  end = max(start, wave_uniform(end));
  int t0 = 0;
  if (start >= 2 * TP) {  // only through bz_gqa_decode_wave, which takes any range
    t0 = start - start % TP;
    load_tile<RPW, PPT, BZ_MASK_NONE>(ta, sp, t0 + r);
    load_tile<RPW, PPT, BZ_MASK_NONE>(tb, sp, t0 + TP + r);
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  }
  const uint4 none = make_uint4(0, 0, 0, 0);
  for (;; t0 += 2 * TP) {
    consume_tile<LPR, RPW, G, PPT, BZ_MASK_NONE, false, true>(ta, qp, a.scale_log2, m, l, acc, t0 + r, end, -1, none,
                                                              none, start);
    if (t0 + TP >= end) break;
    if (t0 + 2 * TP < end) load_tile<RPW, PPT, BZ_MASK_NONE>(ta, sp, t0 + 2 * TP + r);
    consume_tile<LPR, RPW, G, PPT, BZ_MASK_NONE, false, true>(tb, qp, a.scale_log2, m, l, acc, t0 + TP + r, end, -1,
                                                              none, none, start);
    if (t0 + 2 * TP >= end) break;
    if (t0 + 3 * TP < end) load_tile<RPW, PPT, BZ_MASK_NONE>(tb, sp, t0 + 3 * TP + r);
  }

  // one reciprocal of the row total instead of a division per element (v_rcp_f32, within 1 ulp; exact for the powers
  // of two, so a single attended position still returns its V row unchanged)
  const float L = rows_total<LPR>(l[0]);
  const float inv = L > 0.f ? __builtin_amdgcn_rcpf(L) : 0.f;
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = rows_total<LPR>(acc[0][j]) * inv;
  if (r == 0) {
    uint4 w;
    w.x = pack_bf16x2(o[0], o[1]);
    w.y = pack_bf16x2(o[2], o[3]);
    w.z = pack_bf16x2(o[4], o[5]);
    w.w = pack_bf16x2(o[6], o[7]);
    *reinterpret_cast<uint4*>(outp + 8 * c) = w;
  }
}

// One wave per (row, token, q head) of a bz_gqa_decode call: range from seq_lens / kv_start (token t of T attends up
// to itself), then attend_wave. One wave per workgroup, so the waves spread over as many CUs as there are
// (config-5 frame with one wave per kv head: 102 us against 111 with four waves per workgroup, 108 with two).
// Grid (group size G, kv heads, rows * T): the launch covers exactly the waves, and the head indices need no division.
// What the first loads need (the range arrays, the K / V bases, strides and capacity) comes as leading scalar
// arguments, 56 bytes, which kernel-argument preloading puts in SGPRs when the wave starts: the K / V tiles and the
// range loads then go out at once rather than after a load of the argument buffer (they are p's fields again; kv_ss
// fits 32 bits, as the host bounds capacity * kv_stride_s).
template <int D>
__global__ void __launch_bounds__(kWave) gqa_wave_kernel(const int32_t* lens, const int32_t* starts, const uint16_t* k,
                                                         const uint16_t* v, int64_t kv_sb, int64_t kv_sh, int32_t kv_ss,
                                                         int32_t cap, const bz::Params p) {
  // every other kernel argument the wave reads is loaded before any of them is used, so that the loads go out
  // together: one round trip to the argument buffer instead of one per group of dependent uses
  const uint16_t* const q = p.q;
  const int64_t q_sb = p.q_sb, q_sh = p.q_sh, q_st = p.q_st;
  uint16_t* const out = p.out;
  const int64_t o_sb = p.o_sb, o_sh = p.o_sh, o_st = p.o_st;
  const int T = p.T, G = p.G;
  const float scale_log2 = p.scale_log2;
  __builtin_amdgcn_sched_barrier(0);

  const int h = blockIdx.y, hq = h * G + blockIdx.x, z = blockIdx.z;  // z = row * T + token
  const int b = T == 1 ? z : z / T, tok = z - b * T;
  WaveAttention a;
  a.q = q + (int64_t)b * q_sb + (int64_t)tok * q_st + (int64_t)hq * q_sh;
  a.k = k + (int64_t)b * kv_sb + (int64_t)h * kv_sh;
  a.v = v + (int64_t)b * kv_sb + (int64_t)h * kv_sh;
  a.kv_ss = kv_ss;
  a.cap = cap;
  a.scale_log2 = scale_log2;
  a.out = out + (int64_t)b * o_sb + (int64_t)tok * o_st + (int64_t)hq * o_sh;
  attend_wave<D>(a, [&](int& start, int& end) {
    // clamp_range and token_end on the values above; both loads are issued before either is waited for (without
    // kv_start the second reads seq_lens again and its value is dropped)
    int e = lens[b];
    int s = (starts ? starts : lens)[b];
    e = e < 0 ? 0 : (e > cap ? cap : e);
    s = starts == nullptr || s < 0 ? 0 : (s > e ? e : s);
    start = s;
    end = max(s, e - (T - 1 - tok));
  });
}

}  // namespace
