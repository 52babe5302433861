// Device helpers shared by the kernels of libbz_gqa_decode.so (gfx950): bf16 conversion and packing, DPP and
// permlane-swap reductions over a wave64, raw buffer resources and their cache-policy bits.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace {

constexpr int kWave = 64;

// Cache-policy operand bits of buffer loads on gfx940 and later: nt (non-temporal, streamed once) and sc1 (the cache
// behaviour of an agent-scope relaxed atomic access: coherent across the XCDs' separate L2s).
constexpr int kStream = 2;
constexpr int kSc1 = 16;

// The first active lane's value, in a scalar register. For values that are wave-uniform but that the compiler cannot
// prove so (anything derived from threadIdx.x / kWave): a buffer resource built from a value the compiler takes for
// divergent is held in VGPRs, and every load through it becomes a loop over the distinct resources of the wave
// (v_readfirstlane, compare, exec mask, branch per load instruction).
__device__ __forceinline__ int wave_uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t wave_uniform(int64_t x) {
  const uint64_t u = (uint64_t)x;
  return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(u >> 32)) << 32) |
                   (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u));
}
template <class T>
__device__ __forceinline__ T* wave_uniform(T* ptr) {
  return reinterpret_cast<T*>(wave_uniform(reinterpret_cast<int64_t>(ptr)));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16, round to nearest even, NaN stays NaN (quiet): gfx950's v_cvt_pk_bf16_f32, one instruction for a pair,
// no branch.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ void unpack8(const uint4& w, float f[8]) {
  f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// c + a.lo * b.lo + a.hi * b.hi for two packed bf16 pairs, accumulated in fp32 (v_dot2c_f32_bf16)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}

// Sum over the LPR (8 or 16) consecutive lanes that hold one KV row; every lane of the row gets the same value
// (each step adds a lane-permuted copy, and fp32 addition is commutative, so all lanes agree bit for bit).
template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
  static_assert(LPR == 8 || LPR == 16, "row_sum covers 8 or 16 lanes");
  x += dpp<0xb1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4e>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror: lane i <-> 7 - i within each 8 lanes
  if (LPR == 16) x += dpp<0x140>(x);  // row_mirror: lane i <-> 15 - i within each 16 lanes
  return x;
}

// Value of lane (lane ^ 8) inside each 16-lane row: DPP row_ror:8, on the VALU.
__device__ __forceinline__ float lane_xor8(float x) { return dpp<0x128>(x); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// Round 8 floats to bf16 precision in place (RNE), two per conversion.
__device__ __forceinline__ void round8(float (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const uint32_t w = pack_bf16x2(v[j], v[j + 1]);
    v[j] = bf16_lo(w);
    v[j + 1] = bf16_hi(w);
  }
}

// v_permlane16_swap / v_permlane32_swap on two registers: rows 1 and 3 (16 lanes each) of a trade places with rows
// 0 and 2 of b (swap16); lanes 32..63 of a trade places with lanes 0..31 of b (swap32). With rows written
// [r0 r1 r2 r3]: swap16 turns a, b into [a0 b0 a2 b2], [a1 b1 a3 b3]; swap32 into [a0 a1 b0 b1], [a2 a3 b2 b3].
__device__ __forceinline__ void swap16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// Transposed sum over the four 16-lane rows of a wave: returns x with row r of x holding v_r summed over all four rows
// (three swaps and three adds for four values, against two swaps and two adds per value for a broadcast sum).
__device__ __forceinline__ float rows_sum4(float v0, float v1, float v2, float v3) {
  swap16(v0, v1);
  swap16(v2, v3);
  float s = v0 + v1;  // [v0(01) v1(01) v0(23) v1(23)]
  float t = v2 + v3;  // [v2(01) v3(01) v2(23) v3(23)]
  swap32(s, t);
  return s + t;       // [v0 v1 v2 v3], each summed over the four rows
}

// Sum over the 64 lanes of a wave of NV values v[0..NV) (NV a power of two up to 64), transposed: each level pairs
// the lanes across one lane bit (bit 5 and bit 4 by the permlane swaps; bits 3, 2, 1, 0 by DPP row_ror:8,
// row_half_mirror, quad_perm [2,3,0,1] and [1,0,3,2]), and while more than one value is left every lane keeps half of
// them (the upper half where its bit is set) and adds its partner's share of that half, so the values halve at every
// level (NV - 1 swaps or DPP moves in all, against four DPP adds per value for row sums). The lanes each pairing
// joins are always disjoint (the pairings differ on each level), so after the six levels lane L holds, in its v[0],
// the total of value transposed_index<NV>(L), bit for bit the same in every lane that holds that value.
template <int H, int CTRL>
__device__ __forceinline__ void dpp_level(float* v, bool hi) {
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float keep = hi ? v[i + H] : v[i], send = hi ? v[i] : v[i + H];
    v[i] = keep + dpp<CTRL>(send);
  }
}
template <int H>
__device__ __forceinline__ void swap_level(float* v, bool upper32) {
#pragma unroll
  for (int i = 0; i < H; ++i) {
    if (upper32) swap32(v[i], v[i + H]);
    else swap16(v[i], v[i + H]);
    v[i] += v[i + H];
  }
}
template <int NV>
__device__ __forceinline__ float transposed_sum(float (&v)[NV], int lane) {
  static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "a power of two up to 64 values");
  // values left before the levels on bits 5, 4, 3, 2, 1, 0
  constexpr int N5 = NV, N4 = N5 > 1 ? N5 / 2 : 1, N3 = N4 > 1 ? N4 / 2 : 1, N2 = N3 > 1 ? N3 / 2 : 1,
                N1 = N2 > 1 ? N2 / 2 : 1, N0 = N1 > 1 ? N1 / 2 : 1;
  float t;
  if constexpr (N5 > 1) {
    swap_level<N5 / 2>(v, true);  // bit 5: lanes 0..31 against 32..63
  } else {
    t = v[0];
    swap32(v[0], t);
    v[0] += t;
  }
  if constexpr (N4 > 1) {
    swap_level<N4 / 2>(v, false);  // bit 4: rows 0 / 2 against rows 1 / 3
  } else {
    t = v[0];
    swap16(v[0], t);
    v[0] += t;
  }
  if constexpr (N3 > 1) dpp_level<N3 / 2, 0x128>(v, lane & 8);  // bit 3: row_ror:8
  else v[0] += dpp<0x128>(v[0]);
  if constexpr (N2 > 1) dpp_level<N2 / 2, 0x141>(v, lane & 4);  // bit 2: row_half_mirror (lane i <-> 7 - i)
  else v[0] += dpp<0x141>(v[0]);
  if constexpr (N1 > 1) dpp_level<N1 / 2, 0x4e>(v, lane & 2);  // bit 1: quad_perm [2,3,0,1]
  else v[0] += dpp<0x4e>(v[0]);
  if constexpr (N0 > 1) dpp_level<N0 / 2, 0xb1>(v, lane & 1);  // bit 0: quad_perm [1,0,3,2]
  else v[0] += dpp<0xb1>(v[0]);
  return v[0];
}
// The value whose total lane L holds after transposed_sum<NV>: bit 5 of L selects the upper half of the values, bit 4
// the upper half of that half, and so on for as many levels as halve NV.
template <int NV>
__device__ __forceinline__ int transposed_index(int lane) {
  int idx = 0, h = NV / 2;
  const int bits[6] = {32, 16, 8, 4, 2, 1};
#pragma unroll
  for (int b = 0; b < 6; ++b) {
    if (h >= 1 && (lane & bits[b])) idx += h;
    h /= 2;
  }
  return idx;
}
// Whether lane L is the first of the lanes holding its value (its bits below the transposed levels are zero).
template <int NV>
__device__ __forceinline__ bool transposed_writer(int lane) {
  int levels = 0;
  for (int n = NV; n > 1; n /= 2) ++levels;
  return (lane & ((1 << (6 - levels)) - 1)) == 0;
}

// Max over the four 16-lane rows of a wave of each of the N values x[i]; every lane ends with all N maxima.
template <int N>
__device__ __forceinline__ void rows_max(float (&x)[N]) {
  if constexpr (N == 1) {
    float y = x[0];
    swap16(x[0], y);
    x[0] = fmaxf(x[0], y);
    y = x[0];
    swap32(x[0], y);
    x[0] = fmaxf(x[0], y);
  } else if constexpr (N == 2) {
    swap16(x[0], x[1]);
    float s = fmaxf(x[0], x[1]);  // [A(01) B(01) A(23) B(23)]
    float t = s;
    swap32(s, t);
    s = fmaxf(s, t);              // [A B A B]
    t = s;
    swap16(s, t);                 // [A A A A], [B B B B]
    x[0] = s;
    x[1] = t;
  } else {
    static_assert(N % 4 == 0, "rows_max: 1, 2 or a multiple of 4 values");
#pragma unroll
    for (int q = 0; q < N; q += 4) {
      swap16(x[q], x[q + 1]);
      swap16(x[q + 2], x[q + 3]);
      float s = fmaxf(x[q], x[q + 1]), t = fmaxf(x[q + 2], x[q + 3]);
      swap32(s, t);
      float a = fmaxf(s, t);      // [A B C D]
      float c = a;
      swap16(a, c);               // [A A C C], [B B D D]
      float a2 = a, c2 = c;
      swap32(a, a2);              // [A A A A], [C C C C]
      swap32(c, c2);              // [B B B B], [D D D D]
      x[q] = a;
      x[q + 1] = c;
      x[q + 2] = a2;
      x[q + 3] = c2;
    }
  }
}

// Raw buffer resource (gfx9 V#: base, stride 0, num_records bytes, word 3 = DATA_FORMAT 32) over the bytes [0, bytes)
// of one (row, kv head) span. A buffer load at an offset >= bytes returns zero and makes no memory access.
using Rsrc = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ Rsrc span_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, kRsrcWord3);
}

// Reductions over the wave: inside 16-lane rows with DPP (quad_perm x2, half mirror, mirror), then across rows with
// the permlane swaps. Every lane ends with the same value.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<0xb1>(x));
  x = fmaxf(x, dpp<0x4e>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  float y = x;
  swap16(x, y);  // [x0 x0 x2 x2], [x1 x1 x3 x3]
  x = fmaxf(x, y);
  y = x;
  swap32(x, y);
  return fmaxf(x, y);
}
// The same order of additions in every lane, so all lanes hold the same bits.
__device__ __forceinline__ float wave_sum(float x) {
  x = row_sum<16>(x);
  float y = x;
  swap16(x, y);
  x += y;
  y = x;
  swap32(x, y);
  return x + y;
}

}  // namespace
