// Backbone decode GEMVs for gfx950 (include/bz_gemv.h): the reference's flash_bb_fused (flash/csrc/bb_fused.cu).
//
// y[m, n] = epilogue(sum_k xin[m, k] * W[n, k]) for the decode step's M <= 4 rows: weight-streaming and HBM-bound
// (each weight byte is used M times, 2 FLOPs each). The work is laid out for the weights:
//   - a wave owns R output rows (2 R weight rows for the SiLU * up epilogue: gate and up of the same outputs) and
//     streams them whole; lane l reads the 16 bytes at k = 8 l + 512 c of every chunk c, so one wave load instruction
//     covers 1 KiB of one weight row. Rows are raw buffer resources cut at k (and empty past the last output row), so
//     every load is unconditional, nothing past a row is read, and the compiler's vmcnt accounting stays exact.
//   - two tiles of R x U chunks are in flight (ping-pong); the first two are issued before the x prologue, after x's
//     own loads, so the prologue waits for x alone.
//   - x (RMSNorm'ed at the eager rounding points when asked) is held in registers when it fits (k <= 1024, or
//     k <= 2048 with M <= 2: every lane keeps its own 16 bytes of each chunk, and the norm's sum of squares is reduced
//     over the wave, so there is no LDS and no barrier); otherwise it is staged once per workgroup in LDS,
//     zero-padded to a multiple of the tile, and read with one ds_read_b128 per chunk and row of x.
//   - products: four v_dot2c_f32_bf16 per 16 bytes (bf16 x bf16 exact, fp32 accumulation); the R * M (2 R * M)
//     accumulators are summed over the wave with DPP inside 16-lane rows and transposed permlane swaps across rows,
//     so each lane of a row ends with one finished output, written with the epilogue by that row's first lane.
// The weight loads carry the non-temporal hint: 2.8 GB of weights stream through per decode step.
// Where it measured faster (4096 < k <= 6144 at any M, the backbone's down projection; 1024 < k <= 2048 at M >= 3)
// a block-ordered kernel runs instead: a workgroup streams its rows as one contiguous block, every thread holding one
// x vector for all of its rows, and the sums are reduced over the workgroup once, at the end (gemv_block_kernel).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "bz_gemv.h"
#include "device_common.cuh"

namespace bz {
int device_cu_count(int* cus);  // gqa_decode.hip: the current device's CU count, cached per device
}  // namespace bz

namespace {

constexpr int kGemvThreads = 256;              // 4 waves per workgroup (x in registers; rmsnorm)
constexpr int kGemvWaves = kGemvThreads / kWave;
// Threads of a workgroup that stages x in LDS: eight waves share one copy of x (down: 6.47 against 6.9 us with
// four); with x in registers every wave loads its own, and four waves per workgroup measured fastest.
constexpr int kGemvLdsThreads = 512;
template <int KC>
constexpr int gemv_threads() { return KC > 0 ? kGemvThreads : kGemvLdsThreads; }
constexpr int kChunk = 8 * kWave;              // k elements per wave load instruction
constexpr int kU = 2;                          // chunks per tile
constexpr int kTileK = kChunk * kU;            // k elements per tile
constexpr int kMaxLds = 64 * 1024;             // bytes of LDS for x
// With x in registers every wave issues all its weight loads at once; spacing them by s_sleep(kIssueGap) (about
// 64 * kIssueGap clocks) measured faster where the loads queue: q|k|v 5.06 against 5.19 us, gate/up 10.0 against
// 10.3-10.5. Gaps of 1, 3, 4 and 6 were tried; 2 was best or within noise of best. A small grid just waits longer for
// its last load (gate/up, M = 2, k = 2048: 12 workgroups 3.43 against 2.89 us, 32 workgroups 4.05 against 3.92, 128
// workgroups 4.25 against 4.43), and so does a grid of one workgroup per CU whose waves issue few loads (o_proj, 256
// workgroups of eight 1 KiB loads per wave: 3.31 us unpaced against 3.64 paced; q|k|v at two workgroups per CU 4.89
// either way; gate/up, 16 loads per wave, 9.68 paced against 9.96). So the host picks the paced variant (GAP =
// kIssueGap) for grids of at least kPaceMinGrid workgroups whose waves issue at least kPaceMinLoads weight loads each
// or that hold more workgroups than the device has CUs. The gap is a template parameter, not a runtime flag: a branch
// around each s_sleep split the loads over basic blocks, and the compiler's wait counts then went pessimistic (the
// prologue waited for three more weight loads than it needs).
constexpr int kIssueGap = 2;
constexpr int kPaceMinGrid = 64;
constexpr int kPaceMinLoads = 16;

struct GemvParams {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* nw;
  float eps;
  const uint16_t* w0;
  const uint16_t* w1;
  const uint16_t* w2;
  int n0, n1, ntot;  // rows of segments 0 and 1; output rows
  int k, kp;         // k, and k rounded up to kTileK (the LDS row pitch of x)
  uint16_t* y;
  int64_t ldy;
  const uint16_t* res;
  int64_t ldr;
};

// x is staged in two steps. x_issue loads the first kXr 16-byte vectors per thread into registers before the weight
// tiles are issued, so the prologue waits for x alone (loads complete in issue order). stage_x writes them to LDS,
// loads any rest directly, and with NORM rewrites LDS as bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), the mean over
// the k real elements (bb_fused.cu:95-140). One resource covers the x matrix; elements past k in a row (the row
// padding, or past the last row) read as 0, so LDS holds x zero-padded to kp.
constexpr int kXr = 4;

template <int M>
__device__ __forceinline__ uint4 x_vector(const GemvParams& p, const Rsrc& rx, int idx) {
  const int kv = p.kp / 8;
  const int m = idx / kv, j = idx - m * kv;
  const bool in = idx < M * kv && j * 8 < p.k;
  const uint32_t off = in ? (uint32_t)(m * p.ldx + j * 8) * 2 : 0xfffffff0u;  // out of range: reads 0
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
}

template <int M, int NT>
__device__ __forceinline__ void x_issue(const GemvParams& p, const Rsrc& rx, uint4 (&xr)[kXr]) {
#pragma unroll
  for (int i = 0; i < kXr; ++i) xr[i] = x_vector<M>(p, rx, threadIdx.x + i * NT);
}

template <int M, bool NORM, int NT>
__device__ __forceinline__ void stage_x(const GemvParams& p, const Rsrc& rx, const uint4 (&xr)[kXr], uint16_t* xs) {
  const int tid = threadIdx.x;
  const int kv = p.kp / 8, total = M * kv;
  float ss[M];
#pragma unroll
  for (int m = 0; m < M; ++m) ss[m] = 0.f;
  auto put = [&](int idx, const uint4& v) {
    reinterpret_cast<uint4*>(xs)[idx] = v;  // LDS row pitch kp: vector idx of the [M][kp] array
    if (NORM) {
      float f[8];
      unpack8(v, f);
      float s2 = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t) s2 = fmaf(f[t], f[t], s2);
      const int m = idx / kv;
#pragma unroll
      for (int mm = 0; mm < M; ++mm)
        if (mm == m) ss[mm] += s2;
    }
  };
#pragma unroll
  for (int i = 0; i < kXr; ++i) {
    const int idx = tid + i * NT;
    if (idx < total) put(idx, xr[i]);
  }
  for (int idx = tid + kXr * NT; idx < total; idx += NT) put(idx, x_vector<M>(p, rx, idx));
  if (!NORM) return;
  __shared__ float red[NT / kWave][M];
  const int lane = tid % kWave, wave = tid / kWave;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const float s2 = wave_sum(ss[m]);
    if (lane == 0) red[wave][m] = s2;
  }
  __syncthreads();
  const Rsrc rw = span_rsrc(p.nw, p.k * 2);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NT / kWave; ++w) tot += red[w][m];
    const float r = rsqrtf(tot * (1.f / (float)p.k) + p.eps);
    for (int j = tid; j < kv; j += NT) {
      float f[8], w[8];
      unpack8(reinterpret_cast<const uint4*>(xs + m * p.kp)[j], f);
      unpack8(__builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, j * 16, 0, 0)), w);
#pragma unroll
      for (int t = 0; t < 8; ++t) f[t] *= r;
      round8(f);
#pragma unroll
      for (int t = 0; t < 8; ++t) f[t] *= w[t];
      reinterpret_cast<uint4*>(xs + m * p.kp)[j] =
          make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
    }
  }
}

// x of one lane in registers: row m, chunk c (k = 512 c + 8 lane), zero past k.
__device__ __forceinline__ uint4 x_chunk(const GemvParams& p, const Rsrc& rx, int m, int c, int lane) {
  const int k0 = c * kChunk + lane * 8;
  const uint32_t off = k0 < p.k ? (uint32_t)(m * p.ldx + k0) * 2 : 0xfffffff0u;
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
}

// The residual values the writing lanes of a wave need (lane 16 q writes flat value 4 g + q of each group g, i.e.
// output row r = f / M of batch row m = f % M), loaded with the first weight tiles so that the epilogue waits for
// nothing: one 2-byte buffer load per group and lane. Values past the output rows are never used; loads past the
// residual matrix read 0 without a memory access.
template <int M, int R>
__device__ __forceinline__ void load_residual(const GemvParams& p, int row0, int lane, float (&res)[(R * M + 3) / 4]) {
  const Rsrc rr = span_rsrc(p.res, (int)(((int64_t)(M - 1) * p.ldr + p.ntot) * 2));
  const int q = lane / 16;
#pragma unroll
  for (int g = 0; g < (R * M + 3) / 4; ++g) {
    const int f = 4 * g + q, r = f / M, m = f % M;
    const uint32_t off = (uint32_t)(((int64_t)m * p.ldr + row0 + r) * 2);
    res[g] = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(rr, off, 0, 0));
  }
}

// KC > 0: x held in registers, KC chunks per lane (k <= 512 KC <= 2 tiles): no LDS, and the RMSNorm's sum of squares
// is reduced over the wave, so the prologue needs no barrier. KC == 0: x staged in LDS (any k).
// What the first loads need (the weight segments, their row counts, k, x and its stride) comes as leading scalar
// arguments, 56 bytes, which kernel-argument preloading (-mllvm -amdgpu-kernarg-preload-count) puts in SGPRs when the
// wave starts, so the weight and x loads go out at once rather than after a load of the argument buffer; they are
// the block's fields again, which the kernel then reads from these arguments.
template <int M, int R, bool NORM, int EPI, int KC, int GAP>
__global__ void __launch_bounds__(gemv_threads<KC>())
    gemv_kernel(const uint16_t* w0, const uint16_t* w1, const uint16_t* w2, int n0, int n1, int ntot, int k,
                const uint16_t* x, int64_t ldx, const GemvParams args) {
  GemvParams p = args;
  p.w0 = w0;
  p.w1 = w1;
  p.w2 = w2;
  p.n0 = n0;
  p.n1 = n1;
  p.ntot = ntot;
  p.k = k;
  p.x = x;
  p.ldx = ldx;
  static_assert(GAP == 0 || KC > 0, "issue pacing on the x-in-registers path only");
  constexpr int NT = gemv_threads<KC>(), NW = NT / kWave;
  constexpr int NR = EPI == BZ_GEMV_SILU_MUL ? 2 * R : R;  // weight rows per wave
  extern __shared__ __align__(16) uint16_t xs[];            // [M][kp] bf16
  // The paced variant takes the wave index through a scalar register, so the weight resources are scalar and each
  // load is one instruction, spaced by s_sleep. The unpaced variants (x in LDS; small grids) leave it in a VGPR, where
  // the compiler issues every load from a one-iteration loop over the wave's distinct resources. That measured faster
  // than scalar resources without pacing, for reasons not pinned down (down: 6.03 against 6.36 us, paced or not;
  // gate/up on 12 and 32 workgroups: 2.93 and 3.93 against 3.23 and 4.45 us).
  const int tid = threadIdx.x, lane = tid % kWave, wave = GAP > 0 ? wave_uniform(tid / kWave) : tid / kWave;
  const int row0 = (blockIdx.x * NW + wave) * R;

  // this wave's weight rows (a row past the last output: an empty resource, whose loads read 0)
  Rsrc wr[NR];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = row0 + r;
    const int bytes = n < p.ntot ? p.k * 2 : 0;
    if (EPI == BZ_GEMV_SILU_MUL) {
      wr[r] = span_rsrc(p.w0 + (int64_t)n * p.k, bytes);
      wr[R + r] = span_rsrc(p.w1 + (int64_t)n * p.k, bytes);
    } else {
      const uint16_t* base = n < p.n0 ? p.w0 + (int64_t)n * p.k
                           : n < p.n0 + p.n1 ? p.w1 + (int64_t)(n - p.n0) * p.k
                                             : p.w2 + (int64_t)(n - p.n0 - p.n1) * p.k;
      wr[r] = span_rsrc(base, bytes);
    }
  }

  uint4 ta[NR][kU], tb[NR][kU];
  const uint32_t lane_off = lane * 16;
  auto load = [&](uint4 (&t)[NR][kU], int it) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const uint32_t off = (uint32_t)(it * kTileK + u * kChunk) * 2 + lane_off;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        t[r][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr[r], off, 0, kStream));
        if constexpr (GAP > 0) __builtin_amdgcn_s_sleep(GAP);
      }
    }
  };
  const Rsrc rx = span_rsrc(p.x, (int)(((int64_t)(M - 1) * p.ldx + p.k) * 2));
  [[maybe_unused]] float resv[(R * M + 3) / 4];
  float acc[NR][M];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  auto dot16 = [](const uint4& w, const uint4& xv, float a) {
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, xv.x), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, xv.y), a, false);
    a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, xv.z), a, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, xv.w), a, false);
  };

  if constexpr (KC > 0) {
    static_assert(KC <= 2 * kU, "x in registers: the row fits the first two tiles");
    // x (and the norm weight) first, then both weight tiles; the prologue waits for x alone
    uint4 xv[M][KC], nwv[KC];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int c = 0; c < KC; ++c) xv[m][c] = x_chunk(p, rx, m, c, lane);
    if (NORM) {
      const Rsrc rw = span_rsrc(p.nw, p.k * 2);
#pragma unroll
      for (int c = 0; c < KC; ++c)
        nwv[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, (c * kChunk + lane * 8) * 2, 0, 0));
    }
    load(ta, 0);
    load(tb, 1);
    if (EPI == BZ_GEMV_RESIDUAL) load_residual<M, R>(p, row0, lane, resv);
    __builtin_amdgcn_sched_barrier(0);
    if (NORM) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          float f[8];
          unpack8(xv[m][c], f);
#pragma unroll
          for (int t = 0; t < 8; ++t) ss = fmaf(f[t], f[t], ss);
        }
        const float rs = rsqrtf(wave_sum(ss) * (1.f / (float)p.k) + p.eps);
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          float f[8], w[8];
          unpack8(xv[m][c], f);
          unpack8(nwv[c], w);
#pragma unroll
          for (int t = 0; t < 8; ++t) f[t] *= rs;
          round8(f);
#pragma unroll
          for (int t = 0; t < 8; ++t) f[t] *= w[t];
          xv[m][c] = make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                                pack_bf16x2(f[6], f[7]));
        }
      }
    }
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r)
          acc[r][m] = dot16(c < kU ? ta[r][c % kU] : tb[r][c % kU], xv[m][c], acc[r][m]);
  } else {
    // x first (the prologue then waits for x alone), then the first two weight tiles, all before the prologue
    uint4 xr[kXr];
    x_issue<M, NT>(p, rx, xr);
    load(ta, 0);
    load(tb, 1);
    if (EPI == BZ_GEMV_RESIDUAL) load_residual<M, R>(p, row0, lane, resv);
    __builtin_amdgcn_sched_barrier(0);

    stage_x<M, NORM, NT>(p, rx, xr, xs);
    __syncthreads();

    auto consume = [&](const uint4 (&t)[NR][kU], int it) {
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int kk = it * kTileK + u * kChunk + lane * 8;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xs + m * p.kp + kk);
#pragma unroll
          for (int r = 0; r < NR; ++r) acc[r][m] = dot16(t[r][u], xv, acc[r][m]);
        }
      }
    };
    const int nit = p.kp / kTileK;
    for (int it = 0; it < nit; it += 2) {
      consume(ta, it);
      load(ta, it + 2);  // past k: reads 0 without a memory access
      if (it + 1 < nit) consume(tb, it + 1);
      load(tb, it + 3);
    }
  }

  // sum the accumulators over the wave: DPP inside each 16-lane row, then transposed swaps across the 4 rows, so
  // row q of red[g] holds the total of flat value 4 g + q. Flat order: (r, m) -> r * M + m for the R output rows,
  // padded to a multiple of 4 (NG); the up rows of SILU_MUL follow at NG + r * M + m, in the same row as their gate.
  constexpr int NG = (R * M + 3) / 4 * 4;
  constexpr int NV = EPI == BZ_GEMV_SILU_MUL ? 2 * NG : NG;
  float flat[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) flat[v] = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      flat[r * M + m] = row_sum<16>(acc[r][m]);
      if (EPI == BZ_GEMV_SILU_MUL) flat[NG + r * M + m] = row_sum<16>(acc[R + r][m]);
    }
  float red[NV / 4];
#pragma unroll
  for (int g = 0; g < NV / 4; ++g) red[g] = rows_sum4(flat[4 * g], flat[4 * g + 1], flat[4 * g + 2], flat[4 * g + 3]);

  if (lane % 16 != 0) return;
  const int q = lane / 16;
#pragma unroll
  for (int g = 0; g < NG / 4; ++g) {
    const int f = 4 * g + q;
    if (f >= R * M) continue;
    const int r = f / M, m = f % M, n = row0 + r;
    if (n >= p.ntot) continue;
    float v;
    if (EPI == BZ_GEMV_PLAIN) {
      v = red[g];
    } else if (EPI == BZ_GEMV_RESIDUAL) {
      v = resv[g] + bf16_to_f32(f32_to_bf16(red[g]));
    } else {
      const float gt = bf16_to_f32(f32_to_bf16(red[g]));
      const float up = bf16_to_f32(f32_to_bf16(red[NG / 4 + g]));
      v = bf16_to_f32(f32_to_bf16(gt / (1.f + expf(-gt)))) * up;
    }
    p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(v);
  }
}

// Block-ordered GEMV: a workgroup of NT threads owns R = Q * NA output rows (2 R weight rows for the SiLU * up
// epilogue: the gate rows, then the up rows) and streams them as one contiguous block. A row holds KV = NT / Q vectors
// of 16 bytes (k <= 8 KV; the vectors past k read 0); load i of thread t reads vector t % KV of row Q i + t / KV, so
// each wave stays inside one row, every thread needs the same x vector (t % KV) for all of its rows, and all NS loads
// per thread go out at once. Against the wave-per-row kernel above this keeps the workgroup's bytes in flight
// contiguous (the wave-per-row kernel with x in LDS holds a third of each of eight rows 12 KB apart at k = 6144) and
// each workgroup reads x once (with x in registers there every wave reads its own: 32 MB of L2 traffic for q | k | v at
// M = 4). The sums of a row slot are reduced over the waves of its row group once, at the end: DPP and transposed
// swaps inside each wave, then the group's waves through LDS in wave order.
template <int M, int NT, int Q, int NA, bool NORM, int EPI>
__global__ void __launch_bounds__(NT)
    gemv_block_kernel(const uint16_t* w0, const uint16_t* w1, const uint16_t* w2, int n0, int n1, int ntot, int k,
                      const uint16_t* x, int64_t ldx, const GemvParams args) {
  GemvParams p = args;
  p.w0 = w0;
  p.w1 = w1;
  p.w2 = w2;
  p.n0 = n0;
  p.n1 = n1;
  p.ntot = ntot;
  p.k = k;
  p.x = x;
  p.ldx = ldx;
  constexpr int NW = NT / kWave, KV = NT / Q, WPG = NW / Q;  // waves per row group
  static_assert(KV % kWave == 0, "a wave reads within one row");
  constexpr bool SILU = EPI == BZ_GEMV_SILU_MUL;
  constexpr int NS = SILU ? 2 * NA : NA;  // weight-row slots per thread (SiLU: the gate slots, then the up slots)
  constexpr int R = Q * NA;               // output rows per workgroup
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int g = wave_uniform(wave / WPG);  // row group: the weight resources below stay scalar
  const int kv = tid % KV;
  const int row0 = blockIdx.x * R;

  // x (and the norm weight) first, then every weight load; the prologue waits for x alone
  const Rsrc rx = span_rsrc(p.x, (int)(((int64_t)(M - 1) * p.ldx + p.k) * 2));
  uint4 xv[M], nwv = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint32_t off = 8 * kv < p.k ? (uint32_t)(m * p.ldx + 8 * kv) * 2 : 0xfffffff0u;  // past k: reads 0
    xv[m] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
  }
  if (NORM)
    nwv = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(span_rsrc(p.nw, p.k * 2), 16 * kv, 0, 0));
  uint4 wt[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool up = SILU && s >= NA;
    const int n = row0 + Q * (up ? s - NA : s) + g;
    const int bytes = n < p.ntot ? p.k * 2 : 0;  // a row past the last output: an empty resource, its loads read 0
    const uint16_t* base;
    if (SILU) {
      base = (up ? p.w1 : p.w0) + (int64_t)n * p.k;
    } else {
      base = n < p.n0 ? p.w0 + (int64_t)n * p.k
           : n < p.n0 + p.n1 ? p.w1 + (int64_t)(n - p.n0) * p.k
                             : p.w2 + (int64_t)(n - p.n0 - p.n1) * p.k;
    }
    wt[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(span_rsrc(base, bytes), 16 * kv, 0, kStream));
  }
  // the residual value of the output this thread writes (thread f < R * M: row f / M, batch row f % M); loads past
  // the residual matrix read 0 without a memory access, and values past the output rows are never used
  float resv = 0.f;
  if (EPI == BZ_GEMV_RESIDUAL) {
    const Rsrc rr = span_rsrc(p.res, (int)(((int64_t)(M - 1) * p.ldr + p.ntot) * 2));
    const int f = tid % (R * M), n = row0 + f / M, m = f % M;
    resv = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(rr, (uint32_t)(((int64_t)m * p.ldr + n) * 2), 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);

  if (NORM) {
    // every row group holds all of x: the sum of squares over the waves of group 0
    __shared__ float s_ss[NW][M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float f[8], ss = 0.f;
      unpack8(xv[m], f);
#pragma unroll
      for (int t = 0; t < 8; ++t) ss = fmaf(f[t], f[t], ss);
      ss = wave_sum(ss);
      if (lane == 0) s_ss[wave][m] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) tot += s_ss[w][m];
      const float rs = rsqrtf(tot * (1.f / (float)p.k) + p.eps);
      float f[8], w[8];
      unpack8(xv[m], f);
      unpack8(nwv, w);
#pragma unroll
      for (int t = 0; t < 8; ++t) f[t] *= rs;
      round8(f);
#pragma unroll
      for (int t = 0; t < 8; ++t) f[t] *= w[t];
      xv[m] = make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                         pack_bf16x2(f[6], f[7]));
    }
  }

  // flat value s * M + m (zero-padded to a power of two), summed over the wave by the transposed sum: one total per
  // value, written to LDS by the first lane that holds it
  constexpr int NV = NS * M, NP = NV <= 4 ? 4 : NV <= 8 ? 8 : NV <= 16 ? 16 : NV <= 32 ? 32 : 64;
  float flat[NP];
#pragma unroll
  for (int v = 0; v < NP; ++v) flat[v] = 0.f;
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4& w = wt[s];
      float a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, xv[m].x),
                                                0.f, false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, xv[m].y), a,
                                          false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, xv[m].z), a,
                                          false);
      a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, xv[m].w), a,
                                          false);
      flat[s * M + m] = a;
    }
  const float tot = transposed_sum<NP>(flat, lane);
  __shared__ float s_red[NW][NP];
  if (transposed_writer<NP>(lane)) s_red[wave][transposed_index<NP>(lane)] = tot;
  __syncthreads();
  // thread f < R * M writes row row0 + f / M of batch row f % M: slot a = (f / M) / Q of row group (f / M) % Q
  if (tid >= R * M) return;
  const int rr = tid / M, m = tid % M, n = row0 + rr, a = rr / Q, gg = rr % Q;
  if (n >= p.ntot) return;
  float red = 0.f, upv = 0.f;
#pragma unroll
  for (int w = 0; w < WPG; ++w) {
    red += s_red[gg * WPG + w][a * M + m];
    if (SILU) upv += s_red[gg * WPG + w][(NA + a) * M + m];
  }
  float v;
  if (EPI == BZ_GEMV_PLAIN) {
    v = red;
  } else if (EPI == BZ_GEMV_RESIDUAL) {
    v = resv + bf16_to_f32(f32_to_bf16(red));
  } else {
    const float gt = bf16_to_f32(f32_to_bf16(red));
    const float u = bf16_to_f32(f32_to_bf16(upv));
    v = bf16_to_f32(f32_to_bf16(gt / (1.f + expf(-gt)))) * u;
  }
  p.y[(int64_t)m * p.ldy + n] = f32_to_bf16(v);
}

// Standalone row RMSNorm, one workgroup per row (bb_fused.cu:219-248).
__global__ void __launch_bounds__(kGemvThreads) rmsnorm_kernel(const uint16_t* x, int64_t ldx, const uint16_t* w,
                                                               float eps, uint16_t* y, int64_t ldy, int k) {
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const uint16_t* xr = x + (int64_t)m * ldx;
  float ss = 0.f;
  for (int j = tid * 8; j < k; j += kGemvThreads * 8) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(xr + j), f);
#pragma unroll
    for (int t = 0; t < 8; ++t) ss = fmaf(f[t], f[t], ss);
  }
  __shared__ float red[kGemvWaves];
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kGemvWaves; ++i) tot += red[i];
  const float r = rsqrtf(tot * (1.f / (float)k) + eps);
  for (int j = tid * 8; j < k; j += kGemvThreads * 8) {
    float f[8], ww[8];
    unpack8(*reinterpret_cast<const uint4*>(xr + j), f);
    unpack8(*reinterpret_cast<const uint4*>(w + j), ww);
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] *= r;
    round8(f);
#pragma unroll
    for (int t = 0; t < 8; ++t) f[t] *= ww[t];
    *reinterpret_cast<uint4*>(y + (int64_t)m * ldy + j) =
        make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
  }
}

// ---------------------------------------------------------------------------------------------- host side

using GemvFn = void (*)(const uint16_t*, const uint16_t*, const uint16_t*, int, int, int, int, const uint16_t*,
                        int64_t, const GemvParams);

template <int M, int R, int KC, int GAP>
GemvFn pick_epi(int epi, bool norm) {
  if (epi == BZ_GEMV_PLAIN)
    return norm ? gemv_kernel<M, R, true, BZ_GEMV_PLAIN, KC, GAP> : gemv_kernel<M, R, false, BZ_GEMV_PLAIN, KC, GAP>;
  if (epi == BZ_GEMV_RESIDUAL) return norm ? nullptr : gemv_kernel<M, R, false, BZ_GEMV_RESIDUAL, KC, GAP>;
  if (epi == BZ_GEMV_SILU_MUL)
    return norm ? gemv_kernel<M, R, true, BZ_GEMV_SILU_MUL, KC, GAP>
                : gemv_kernel<M, R, false, BZ_GEMV_SILU_MUL, KC, GAP>;
  return nullptr;
}

// With x in LDS: R = 1, 2 or 4 rows per wave, no pacing. With x in registers: R = 2, paced or not.
template <int M, int KC>
GemvFn pick_r(int r, int epi, bool norm, bool pace) {
  if constexpr (KC > 0) {
    if (r != 2) return nullptr;
    return pace ? pick_epi<M, 2, KC, kIssueGap>(epi, norm) : pick_epi<M, 2, KC, 0>(epi, norm);
  } else {
    switch (r) {
      case 1: return pick_epi<M, 1, KC, 0>(epi, norm);
      case 2: return pick_epi<M, 2, KC, 0>(epi, norm);
      default: return pick_epi<M, 4, KC, 0>(epi, norm);
    }
  }
}

// x in registers for k <= 2048 (KC = 2: k <= 1024, KC = 4: k <= 2048); LDS otherwise.
template <int M>
GemvFn pick_kc(int kc, int r, int epi, bool norm, bool pace) {
  if (kc == 4) return pick_r<M, 4>(r, epi, norm, pace);
  if (kc == 2) return pick_r<M, 2>(r, epi, norm, pace);
  return pick_r<M, 0>(r, epi, norm, pace);
}

// Chunks of x per lane held in registers (0: x in LDS).
int kc_for(int m, int k) {
  (void)m;
  const int chunks = (k + kChunk - 1) / kChunk;
  return chunks <= 2 ? 2 : (chunks <= 4 ? 4 : 0);
}

GemvFn pick_gemv(int m, int kc, int r, int epi, bool norm, bool pace) {
  switch (m) {
    case 1: return pick_kc<1>(kc, r, epi, norm, pace);
    case 2: return pick_kc<2>(kc, r, epi, norm, pace);
    case 3: return pick_kc<3>(kc, r, epi, norm, pace);
    case 4: return pick_kc<4>(kc, r, epi, norm, pace);
    default: return nullptr;
  }
}

// The block-ordered kernel where it measured faster than the wave-per-row kernel (cold, graph replay, us per call,
// wave-per-row -> block):
//   4096 < k <= 6144, any M: 768 threads, one row per load instruction (down at k = 6144, M = 1 / 2 / 4: 6.71 / 6.77 /
//     7.50 -> 5.93 / 6.01 / 6.30);
//   1024 < k <= 2048 and M >= 3: 512 threads, two rows per load instruction (M = 4: q | k | v 7.04 -> 5.41, gate / up
//     12.75 -> 12.0, o_proj 3.85 -> 3.58). At M <= 2 the wave-per-row kernel with x in registers stays faster there
//     (the backbone step at M = 2 on one box: gate / up 9.70 against 9.92 us, the step 852 against 861 us).
// Eight row slots per thread (256 workgroups at the backbone's down and q | k | v), four where eight leave fewer than
// 256 workgroups (o_proj), and four gate plus four up slots for the SiLU * up epilogue (eight of each: gate / up 11.7
// against 10.4 us at M = 2).
constexpr int kBlockMinGrid = 256;

template <int M, int NT, int Q, int NA>
GemvFn pick_block_epi(int epi, bool norm) {
  if (epi == BZ_GEMV_PLAIN)
    return norm ? gemv_block_kernel<M, NT, Q, NA, true, BZ_GEMV_PLAIN>
                : gemv_block_kernel<M, NT, Q, NA, false, BZ_GEMV_PLAIN>;
  if (epi == BZ_GEMV_RESIDUAL) return norm ? nullptr : gemv_block_kernel<M, NT, Q, NA, false, BZ_GEMV_RESIDUAL>;
  return nullptr;
}
template <int M, int NT, int Q>
GemvFn pick_block_na(int na, int epi, bool norm) {
  if (epi == BZ_GEMV_SILU_MUL)
    return norm ? gemv_block_kernel<M, NT, Q, 4, true, BZ_GEMV_SILU_MUL>
                : gemv_block_kernel<M, NT, Q, 4, false, BZ_GEMV_SILU_MUL>;
  if constexpr (Q == 1) {
    (void)na;
    return pick_block_epi<M, NT, Q, 8>(epi, norm);  // one row per instruction: eight slots
  } else {
    return na == 8 ? pick_block_epi<M, NT, Q, 8>(epi, norm) : pick_block_epi<M, NT, Q, 4>(epi, norm);
  }
}
// The block kernel for this call, its workgroup size and grid; nullptr where the wave-per-row kernel is taken.
GemvFn pick_block(int m, int k, int ntot, int epi, bool norm, int* threads, int* grid) {
  int q;
  if (k > 4096 && k <= 6144) {
    q = 1;
    *threads = 768;
  } else if (k > 1024 && k <= 2048 && m >= 3) {
    q = 2;
    *threads = 512;
  } else {
    return nullptr;
  }
  int na = 8;
  if (epi == BZ_GEMV_SILU_MUL || (q == 2 && (ntot + 8 * q - 1) / (8 * q) < kBlockMinGrid)) na = 4;
  *grid = (ntot + q * na - 1) / (q * na);
  if (q == 1) {
    switch (m) {
      case 1: return pick_block_na<1, 768, 1>(na, epi, norm);
      case 2: return pick_block_na<2, 768, 1>(na, epi, norm);
      case 3: return pick_block_na<3, 768, 1>(na, epi, norm);
      case 4: return pick_block_na<4, 768, 1>(na, epi, norm);
      default: return nullptr;
    }
  }
  return m == 3 ? pick_block_na<3, 512, 2>(na, epi, norm) : pick_block_na<4, 512, 2>(na, epi, norm);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Output rows per wave. With x in registers every wave loads its own x, so two rows per wave halve that L2 traffic
// (measured at the backbone shapes: q|k|v 6.6 -> 5.3 us, o_proj 3.7 -> 3.55 us); with x in LDS, one row per wave
// keeps more waves streaming until the rows are many (down: 7.2 us with two rows, 6.9 with one).
int rows_per_wave(int ntot, int epi, int kc) {
  const int rows = epi == BZ_GEMV_SILU_MUL ? 2 * ntot : ntot;
  if (kc > 0) return 2;
  if (rows >= 16384) return 4;
  if (rows >= 8192) return 2;
  return 1;
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) int bz_gemv(const bz_gemv_args* a, hipStream_t stream) {
  if (a == nullptr || a->x == nullptr || a->y == nullptr || a->w[0] == nullptr) return BZ_ERR_NULL;
  if (a->m < 1 || a->m > 4 || a->k <= 0 || (a->k & 7)) return BZ_ERR_SHAPE;
  if (a->epilogue < BZ_GEMV_PLAIN || a->epilogue > BZ_GEMV_SILU_MUL) return BZ_ERR_UNSUPPORTED;
  for (int i = 0; i < 3; ++i)
    if (a->n[i] < 0) return BZ_ERR_SHAPE;
  int ntot;
  if (a->epilogue == BZ_GEMV_SILU_MUL) {
    if (a->w[1] == nullptr) return BZ_ERR_NULL;
    if (a->n[0] != a->n[1] || a->n[2] != 0) return BZ_ERR_SHAPE;
    ntot = a->n[0];
  } else {
    if ((a->n[1] > 0 && a->w[1] == nullptr) || (a->n[2] > 0 && a->w[2] == nullptr)) return BZ_ERR_NULL;
    if ((int64_t)a->n[0] + a->n[1] + a->n[2] > INT32_MAX) return BZ_ERR_SHAPE;
    ntot = a->n[0] + a->n[1] + a->n[2];
  }
  if (ntot <= 0) return BZ_ERR_SHAPE;
  if (a->epilogue == BZ_GEMV_RESIDUAL) {
    if (a->res == nullptr) return BZ_ERR_NULL;
    if (a->norm_weight != nullptr) return BZ_ERR_UNSUPPORTED;  // the reference's gemv_resid takes no norm
  }
  if (a->x_stride < a->k || a->y_stride < ntot || (a->epilogue == BZ_GEMV_RESIDUAL && a->res_stride < ntot))
    return BZ_ERR_SHAPE;
  if (!aligned16(a->x) || (a->x_stride & 7) || (a->norm_weight && !aligned16(a->norm_weight))) return BZ_ERR_ALIGNMENT;
  for (int i = 0; i < 3; ++i)
    if (a->w[i] && !aligned16(a->w[i])) return BZ_ERR_ALIGNMENT;
  const int kp = (a->k + kTileK - 1) / kTileK * kTileK;
  const size_t lds = (size_t)a->m * kp * 2;
  if (lds > (size_t)kMaxLds || (int64_t)a->k * 2 > INT32_MAX) return BZ_ERR_UNSUPPORTED;
  if (((int64_t)(a->m - 1) * a->x_stride + a->k) * 2 > INT32_MAX) return BZ_ERR_SHAPE;  // x: 32-bit byte offsets
  if (a->epilogue == BZ_GEMV_RESIDUAL && ((int64_t)(a->m - 1) * a->res_stride + ntot) * 2 > INT32_MAX)
    return BZ_ERR_SHAPE;  // the residual: 32-bit byte offsets

  GemvParams p;
  p.x = static_cast<const uint16_t*>(a->x);
  p.ldx = a->x_stride;
  p.nw = static_cast<const uint16_t*>(a->norm_weight);
  p.eps = a->eps;
  p.w0 = static_cast<const uint16_t*>(a->w[0]);
  p.w1 = static_cast<const uint16_t*>(a->w[1] ? a->w[1] : a->w[0]);
  p.w2 = static_cast<const uint16_t*>(a->w[2] ? a->w[2] : a->w[0]);
  p.n0 = a->n[0];
  p.n1 = a->epilogue == BZ_GEMV_SILU_MUL ? 0 : a->n[1];
  p.ntot = ntot;
  p.k = a->k;
  p.kp = kp;
  p.y = static_cast<uint16_t*>(a->y);
  p.ldy = a->y_stride;
  p.res = static_cast<const uint16_t*>(a->res);
  p.ldr = a->res_stride;
  int bthreads = 0, bgrid = 0;
  if (GemvFn bf = pick_block(a->m, a->k, ntot, a->epilogue, a->norm_weight != nullptr, &bthreads, &bgrid)) {
    hipLaunchKernelGGL(bf, dim3(bgrid), dim3(bthreads), 0, stream, p.w0, p.w1, p.w2, p.n0, p.n1, p.ntot, p.k, p.x,
                       p.ldx, p);
    return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
  }
  const int kc = kc_for(a->m, a->k);
  const int r = rows_per_wave(ntot, a->epilogue, kc);
  const int threads = kc > 0 ? kGemvThreads : kGemvLdsThreads;
  const int rows_per_block = threads / kWave * r;
  const int grid = (ntot + rows_per_block - 1) / rows_per_block;
  bool pace = kc > 0 && grid >= kPaceMinGrid;
  if (pace && (a->epilogue == BZ_GEMV_SILU_MUL ? 2 * r : r) * kc < kPaceMinLoads) {
    int cus = 0;
    const int rc = bz::device_cu_count(&cus);
    if (rc != BZ_OK) return rc;
    pace = grid > cus;
  }
  GemvFn fn = pick_gemv(a->m, kc, r, a->epilogue, a->norm_weight != nullptr, pace);
  if (fn == nullptr) return BZ_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(threads), kc > 0 ? 0 : lds, stream, p.w0, p.w1, p.w2, p.n0, p.n1, p.ntot,
                     p.k, p.x, p.ldx, p);
  return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

__attribute__((visibility("default"))) int bz_rmsnorm(const void* x, int64_t x_stride, const void* w, float eps,
                                                       void* y, int64_t y_stride, int32_t m, int32_t k,
                                                       hipStream_t stream) {
  if (x == nullptr || w == nullptr || y == nullptr) return BZ_ERR_NULL;
  if (m <= 0 || m > 65535 || k <= 0 || (k & 7) || x_stride < k || y_stride < k) return BZ_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || (x_stride & 7) || (y_stride & 7)) return BZ_ERR_ALIGNMENT;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(m), dim3(kGemvThreads), 0, stream, static_cast<const uint16_t*>(x), x_stride,
                     static_cast<const uint16_t*>(w), eps, static_cast<uint16_t*>(y), y_stride, k);
  return hipGetLastError() == hipSuccess ? BZ_OK : BZ_ERR_LAUNCH;
}

}  // extern "C"
