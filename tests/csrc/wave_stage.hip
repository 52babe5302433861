// Test support (not part of the C ABI): the wave-level attention device function attend_wave
// (breeze-tts-2-flash_amd/csrc/gqa_wave.cuh) run as one stage of a multi-stage kernel, the way a kernel that runs a
// whole depth decode step would call it (flash/csrc/depth_frame.cu:193-272 gives each warp one (row, q head) pair of
// its attention stage while other warps work elsewhere). Every workgroup has kStageWaves waves; the waves whose bit is
// set in att_mask run attend_wave on consecutive (row, token, q head) items, and the others run an unrelated busy
// stage at the same time: streaming reads and read-modify-writes of their own slice of a scratch buffer, wave-local
// LDS traffic and VALU work, no barrier. The outputs must equal bz_gqa_decode_wave's (the same device function
// launched alone, one wave per workgroup) bit for bit.
//
//   int bz_test_wave_stage(const bz_gqa_decode_args* a, uint32_t att_mask, uint32_t* busy, int64_t busy_words,
//                          hipStream_t stream)
//       a: as for bz_gqa_decode_wave (seq_lens required, kv_start optional, no mask, head_dim 64 or 128, 16-byte
//       aligned q / out rows); att_mask: 1..15; busy: at least bz_test_wave_stage_busy_words() words, written.
//       0, or -1 for a bad argument or a launch error.
//   int64_t bz_test_wave_stage_busy_words(const bz_gqa_decode_args* a, uint32_t att_mask)
//   const char* bz_test_wave_stage_build_id(void)   the hash of the sources this library was built from
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "gqa_wave.cuh"

#ifndef BZ_TEST_BUILD_ID
#define BZ_TEST_BUILD_ID "unknown"
#endif

namespace {

constexpr int kStageWaves = 4;
constexpr int kBusyIters = 48;  // words per lane of the busy stage

struct StageArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh, q_st;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sb, kv_sh, kv_ss;
  int cap;
  const int32_t* lens;
  const int32_t* starts;
  uint16_t* out;
  int64_t o_sb, o_sh, o_st;
  int T, NH, G, items;
  float scale_log2;
};

template <int D>
__global__ void __launch_bounds__(kStageWaves * kWave) wave_stage_kernel(const StageArgs s, uint32_t att_mask,
                                                                          int att_per_wg, uint32_t* busy,
                                                                          int64_t busy_words) {
  __shared__ uint32_t lds[kStageWaves][kWave];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if ((att_mask >> wave) & 1u) {
    const int slot = __popc(att_mask & ((1u << wave) - 1u));
    const int item = blockIdx.x * att_per_wg + slot;
    if (item >= s.items) return;
    const int hq = item % s.NH, z = item / s.NH, h = hq / s.G;  // z = row * T + token
    const int b = z / s.T, tok = z - b * s.T;
    WaveAttention a;
    a.q = s.q + (int64_t)b * s.q_sb + (int64_t)tok * s.q_st + (int64_t)hq * s.q_sh;
    a.k = s.k + (int64_t)b * s.kv_sb + (int64_t)h * s.kv_sh;
    a.v = s.v + (int64_t)b * s.kv_sb + (int64_t)h * s.kv_sh;
    a.kv_ss = s.kv_ss;
    a.cap = s.cap;
    a.scale_log2 = s.scale_log2;
    a.out = s.out + (int64_t)b * s.o_sb + (int64_t)tok * s.o_st + (int64_t)hq * s.o_sh;
    const int32_t* lens = s.lens;
    const int32_t* starts = s.starts;
    const int cap = s.cap, T = s.T;
    attend_wave<D>(a, [&](int& start, int& end) {
      int e = lens[b];
      int st = (starts ? starts : lens)[b];
      e = e < 0 ? 0 : (e > cap ? cap : e);
      st = starts == nullptr || st < 0 ? 0 : (st > e ? e : st);
      start = st;
      end = max(st, e - (T - 1 - tok));
    });
    return;
  }
  // busy stage: this wave's own kBusyIters * 64 words of busy, its own row of LDS
  uint32_t x = (uint32_t)(blockIdx.x * kStageWaves + wave) * 2654435761u + (uint32_t)lane;
  const int64_t base = ((int64_t)blockIdx.x * kStageWaves + wave) * kBusyIters * kWave;
  for (int it = 0; it < kBusyIters; ++it) {
    const int64_t idx = base + (int64_t)it * kWave + lane;
    const uint32_t w = idx < busy_words ? busy[idx] : 0u;
    lds[wave][lane] = x ^ w;
    __builtin_amdgcn_wave_barrier();
    const uint32_t nb = lds[wave][(lane + 1) % kWave];
#pragma unroll
    for (int r = 0; r < 8; ++r) x = x * 1664525u + 1013904223u + (nb >> r);
    if (idx < busy_words) busy[idx] = x;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

bool valid(const bz_gqa_decode_args* a, uint32_t att_mask) {
  if (a == nullptr || a->q == nullptr || a->k_cache == nullptr || a->v_cache == nullptr || a->out == nullptr ||
      a->seq_lens == nullptr || a->mask != nullptr)
    return false;
  if (att_mask == 0 || att_mask >= (1u << kStageWaves)) return false;
  if (a->head_dim != 64 && a->head_dim != 128) return false;
  if (a->batch <= 0 || a->num_q_heads <= 0 || a->num_kv_heads <= 0 || a->num_q_heads % a->num_kv_heads != 0 ||
      a->capacity <= 0)
    return false;
  const int T = a->tokens_per_row > 1 ? a->tokens_per_row : 1;
  if ((int64_t)a->batch * T * a->num_q_heads > INT32_MAX / 2) return false;
  if (!aligned16(a->q) || !aligned16(a->out) || !aligned16(a->k_cache) || !aligned16(a->v_cache)) return false;
  if ((a->q_stride_b | a->q_stride_h | a->q_stride_t | a->out_stride_b | a->out_stride_h | a->out_stride_t |
       a->kv_stride_b | a->kv_stride_h | a->kv_stride_s) % 8 != 0)
    return false;
  if (a->kv_stride_s < a->head_dim || (int64_t)(a->capacity + 1024) * a->kv_stride_s * 2 >= ((int64_t)1 << 31))
    return false;
  return true;
}

int grid_of(const bz_gqa_decode_args* a, uint32_t att_mask, int* att_per_wg, int* items) {
  const int T = a->tokens_per_row > 1 ? a->tokens_per_row : 1;
  *items = a->batch * T * a->num_q_heads;
  *att_per_wg = __builtin_popcount(att_mask);
  return (*items + *att_per_wg - 1) / *att_per_wg;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) const char* bz_test_wave_stage_build_id(void) { return BZ_TEST_BUILD_ID; }

__attribute__((visibility("default"))) int64_t bz_test_wave_stage_busy_words(const bz_gqa_decode_args* a,
                                                                            uint32_t att_mask) {
  if (!valid(a, att_mask)) return -1;
  int per = 0, items = 0;
  return (int64_t)grid_of(a, att_mask, &per, &items) * kStageWaves * kBusyIters * kWave;
}

__attribute__((visibility("default"))) int bz_test_wave_stage(const bz_gqa_decode_args* a, uint32_t att_mask,
                                                             uint32_t* busy, int64_t busy_words, hipStream_t stream) {
  if (!valid(a, att_mask) || busy == nullptr) return -1;
  int per = 0, items = 0;
  const int grid = grid_of(a, att_mask, &per, &items);
  if (busy_words < (int64_t)grid * kStageWaves * kBusyIters * kWave) return -1;
  StageArgs s;
  s.q = static_cast<const uint16_t*>(a->q);
  s.q_sb = a->q_stride_b;
  s.q_sh = a->q_stride_h;
  s.q_st = a->q_stride_t;
  s.k = static_cast<const uint16_t*>(a->k_cache);
  s.v = static_cast<const uint16_t*>(a->v_cache);
  s.kv_sb = a->kv_stride_b;
  s.kv_sh = a->kv_stride_h;
  s.kv_ss = a->kv_stride_s;
  s.cap = a->capacity;
  s.lens = a->seq_lens;
  s.starts = a->kv_start;
  s.out = static_cast<uint16_t*>(a->out);
  s.o_sb = a->out_stride_b;
  s.o_sh = a->out_stride_h;
  s.o_st = a->out_stride_t;
  s.T = a->tokens_per_row > 1 ? a->tokens_per_row : 1;
  s.NH = a->num_q_heads;
  s.G = a->num_q_heads / a->num_kv_heads;
  s.items = items;
  s.scale_log2 = a->scale * kLog2e;  // as bz_gqa_decode derives it
  if (a->head_dim == 128)
    hipLaunchKernelGGL(wave_stage_kernel<128>, dim3(grid), dim3(kStageWaves * kWave), 0, stream, s, att_mask, per,
                       busy, busy_words);
  else
    hipLaunchKernelGGL(wave_stage_kernel<64>, dim3(grid), dim3(kStageWaves * kWave), 0, stream, s, att_mask, per,
                       busy, busy_words);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
