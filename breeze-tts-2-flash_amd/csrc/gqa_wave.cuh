// Wave-level GQA decode attention: a device function for kernels that run a whole decode step in one launch (a
// persistent depth-transformer kernel of the reference's kind, flash/csrc/depth_frame.cu:193-272, whose attention
// stage gives each warp one (row, q head) pair over at most 17 cached positions). Here too one wave owns one (row,
// q head), and the K/V bytes go from the cache straight into VGPRs (no LDS staging, no barrier), so the caller may run
// it from any wave of any workgroup, with other waves busy elsewhere. Any length works; it is built for short ones
// (one or two tiles of 2 * 64 / (D / 8) positions).
//
// The q heads of a group read the same K/V bytes, each through its own wave (from the L2 after the first). A wave that
// owned a whole group instead, sharing each K/V load among its G heads, measured slower: its serial chain of dot
// products, row sums and softmax steps grows with G while the bytes are few (real depth shape, 8 q / 2 KV heads,
// lengths 2..17: 2.9 against 4.6 us per launch; config-5 frame: 2.64 against 3.21 us per launch).
//
// The arithmetic is the split kernel's (gqa_kernels.cuh: load_tile, consume_tile): bf16 dot2 products with fp32
// accumulation, online softmax in base 2 with one running max per wave, fp32 P.V; then the rows of the wave are summed
// (the max is wave-uniform, so plain sums merge them) and the first row writes bf16(acc / sum), or 0 for an empty
// range.
#pragma once

#include "gqa_kernels.cuh"

namespace {

// Everything one wave needs: element pointers and strides, no batch or head indexing left to do.
struct WaveAttention {
  const uint16_t* q;   // the q head: D bf16 (16-byte aligned)
  const uint16_t* k;   // K and V of its kv head in this row: position p at k + p * kv_ss (16-byte aligned rows)
  const uint16_t* v;
  int64_t kv_ss;
  int start, end;      // attended positions [start, end), 0 <= start; end * kv_ss * 2 < 2^31
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

// Called by all 64 lanes of one wave (wave-uniform arguments).
template <int D>
__device__ void attend_wave(const WaveAttention& a) {
  constexpr int G = 1;  // one q head per wave: the group size of the shared tile code (consume_tile)
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  constexpr int LPR = D / 8, RPW = kWave / LPR, PPT = 2, TP = RPW * PPT;
  const int lane = __lane_id(), r = lane / LPR, c = lane % LPR;
  // the arguments are wave-uniform; taking them through a scalar register keeps the buffer resources and the loop
  // bounds scalar whatever the caller derived them from
  const int start = wave_uniform(a.start), end = max(start, wave_uniform(a.end));
  const int64_t kv_ss = wave_uniform(a.kv_ss);
  uint16_t* const outp = wave_uniform(a.out);

  // q first: loads complete in issue order, so the first tile's q.k waits for q and that tile alone
  const Rsrc rq = span_rsrc(wave_uniform(a.q), D * 2);
  const uint4 qp[G] = {__builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, (uint32_t)(16 * c), 0, 0))};
  Spans sp;
  sp.row_bytes = (uint32_t)kv_ss * 2;
  sp.lane_off = 16 * c;
  sp.k = span_rsrc(wave_uniform(a.k), end * (int)sp.row_bytes);
  sp.v = span_rsrc(wave_uniform(a.v), end * (int)sp.row_bytes);
  Tile<PPT> ta, tb;
  load_tile<RPW, PPT, BZ_MASK_NONE>(ta, sp, start + r);
  load_tile<RPW, PPT, BZ_MASK_NONE>(tb, sp, start + TP + r);
  __builtin_amdgcn_sched_barrier(0);

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.f;
  }
  const uint4 none = make_uint4(0, 0, 0, 0);
  for (int t0 = start; t0 < end; t0 += 2 * TP) {
    consume_tile<LPR, RPW, G, PPT, BZ_MASK_NONE, false>(ta, qp, a.scale_log2, m, l, acc, t0 + r, end, -1, none, none);
    if (t0 + TP >= end) break;
    load_tile<RPW, PPT, BZ_MASK_NONE>(ta, sp, t0 + 2 * TP + r);
    consume_tile<LPR, RPW, G, PPT, BZ_MASK_NONE, false>(tb, qp, a.scale_log2, m, l, acc, t0 + TP + r, end, -1, none,
                                                        none);
    load_tile<RPW, PPT, BZ_MASK_NONE>(tb, sp, t0 + 3 * TP + r);
  }

  const float L = rows_total<LPR>(l[0]);
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float A = rows_total<LPR>(acc[0][j]);
    o[j] = L > 0.f ? A / L : 0.f;
  }
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
template <int D>
__global__ void __launch_bounds__(kWave) gqa_wave_kernel(const bz::Params p, int waves) {
  const int gi = blockIdx.x;
  if (gi >= waves) return;
  const int hq = gi % p.NH, z = gi / p.NH;  // z = row * T + token
  const int h = hq / (p.NH / p.NKV);        // its kv head (repeat_kv)
  const int b = z / p.T, tok = z - b * p.T;
  WaveAttention a;
  a.q = p.q + (int64_t)b * p.q_sb + (int64_t)tok * p.q_st + (int64_t)hq * p.q_sh;
  a.k = p.k + (int64_t)b * p.kv_sb + (int64_t)h * p.kv_sh;
  a.v = p.v + (int64_t)b * p.kv_sb + (int64_t)h * p.kv_sh;
  a.kv_ss = p.kv_ss;
  token_range(p, b, tok, a.start, a.end);
  a.scale_log2 = p.scale_log2;
  a.out = p.out + (int64_t)b * p.o_sb + (int64_t)tok * p.o_st + (int64_t)hq * p.o_sh;
  attend_wave<D>(a);
}

}  // namespace
