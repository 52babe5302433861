/* C ABI of the MI355X (gfx950) backbone decode GEMVs in libbz_gqa_decode.so.
 *
 * Replaces the reference's extension flash_bb_fused (flash/csrc/bb_fused.cu): skinny bf16 GEMVs over the decode
 * step's M = 1..4 rows (the CFG pair is M = 2), y[m, n] = sum_k xin[m, k] * W[n, k] with W in nn.Linear layout
 * ([N, K] row-major) and fp32 accumulation, with an optional Qwen3 RMSNorm prologue and a residual or SiLU * up
 * epilogue at the eager rounding points (bb_fused.cu:1-7), and the standalone row RMSNorm (bb_fused.cu:219-248).
 *
 * Conventions as in bz_gqa_decode.h: device pointers, element strides, status codes (bz_status), nothing allocated,
 * nothing launched when a check fails, the caller's stream. Thread-safe and reentrant.
 */
#ifndef BZ_GEMV_H
#define BZ_GEMV_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "bz_gqa_decode.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum bz_gemv_epilogue {
  BZ_GEMV_PLAIN = 0,     /* y = bf16(acc)                                         (bb_fused.cu:198-199) */
  BZ_GEMV_RESIDUAL = 1,  /* y = bf16(res + bf16(acc))                              (:200-201) */
  BZ_GEMV_SILU_MUL = 2   /* y = bf16(bf16(silu(bf16(acc_gate))) * bf16(acc_up))    (:202-205) */
} bz_gemv_epilogue;

/* Arguments of bz_gemv. */
typedef struct bz_gemv_args {
  /* x [m, k] bf16, element (i, j) at x[i * x_stride + j]; x and x_stride 16-byte aligned (multiple of 8 elements) */
  const void* x;
  int64_t x_stride;
  /* optional Qwen3 RMSNorm prologue: xin = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), w [k] bf16 16-byte aligned;
     NULL: xin = x */
  const void* norm_weight;
  float eps;
  /* weight segments W_i [n_i, k] bf16 row-major, 16-byte aligned. PLAIN / RESIDUAL: the output rows are the rows of
     W_0, then W_1, then W_2 (the q | k | v projections without concatenating them; n_1, n_2 may be 0).
     SILU_MUL: w[0] = gate, w[1] = up, n[0] == n[1] output rows, n[2] == 0. */
  const void* w[3];
  int32_t n[3];
  /* residual [m, N] bf16 (RESIDUAL only), element (i, j) at res[i * res_stride + j] */
  const void* res;
  int64_t res_stride;
  /* y [m, N] bf16, element (i, j) at y[i * y_stride + j] (N = n[0] + n[1] + n[2], or n[0] for SILU_MUL) */
  void* y;
  int64_t y_stride;
  int32_t m;         /* rows of x: 1..4 */
  int32_t k;         /* multiple of 8; m * round_up(k, 1024) * 2 bytes of x must fit 64 KiB of LDS */
  int32_t epilogue;  /* bz_gemv_epilogue */
} bz_gemv_args;

/* y = epilogue(norm?(x) @ W^T). Replaces gemv_seg (bb_fused.cu:293-317; PLAIN, optional norm, up to three segments),
   gemv_resid (:319-335; RESIDUAL) and gemv_gateup (:337-356; SILU_MUL with the norm), pybind :370-377. */
int bz_gemv(const bz_gemv_args* args, hipStream_t stream);

/* Row RMSNorm y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))) over m rows of k elements (x, y, w bf16, 16-byte
   aligned rows, k multiple of 8). Replaces rmsnorm (bb_fused.cu:358-368, kernel :219-248). */
int bz_rmsnorm(const void* x, int64_t x_stride, const void* w, float eps, void* y, int64_t y_stride, int32_t m,
               int32_t k, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BZ_GEMV_H */
