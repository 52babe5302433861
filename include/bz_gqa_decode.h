/*
 * bz_gqa_decode.h - C ABI of the MI355X (gfx950) GQA flash-decoding attention library
 * (libbz_gqa_decode.so).
 *
 * One query token per sequence (decode step, q_len == 1) attends over a bf16 KV cache:
 *
 *   out[b, h, :] = sum_p softmax_p(scale * q[b, h, :] . K[b, h / G, p, :] + mask[b, p]) * V[b, h / G, p, :]
 *
 * over the positions p in [kv_start[b], seq_lens[b]) of row b (G = num_q_heads / num_kv_heads; q head h reads
 * KV head h / G, the head map of repeat_kv). Positions outside that range are never read: NaN or Inf stored there
 * cannot reach the output. Arithmetic is fp32 (online softmax in base 2, split-K partials merged by their
 * log-sum-exp); the output is rounded to bf16 (round-to-nearest-even).
 *
 * Conventions shared by every entry point:
 *   - All pointers in an argument struct are DEVICE pointers on the current HIP device, except the struct itself.
 *   - Strides are in ELEMENTS. The last dimension (head_dim) of every tensor is contiguous.
 *   - The library allocates nothing and makes no host-side decision from device data, so a call can be recorded
 *     into a HIP graph. The grid depends only on host arguments; lengths are read on the device.
 *   - Return value: BZ_OK (0) or a negative bz_status. Nothing is launched when a check fails. No call throws.
 *   - Calls are reentrant. Two calls that share one workspace must be ordered on one stream.
 *   - A workspace starts with the split kernel's arrival counters, one per (row, kv head), which every call leaves
 *     at zero; the rest is written before it is read. One zero-filled workspace therefore serves any sequence of
 *     calls with the same batch * tokens_per_row * num_kv_heads (any split count, length, mask or entry point) that
 *     it is large enough for. A call with another batch * tokens_per_row * num_kv_heads needs a workspace of its own
 *     (or a fresh zero fill): its counters would lie on the previous layout's partials.
 */
#ifndef BZ_GQA_DECODE_H
#define BZ_GQA_DECODE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BZ_GQA_DECODE_ABI_VERSION 9

typedef enum bz_status {
  BZ_OK = 0,
  BZ_ERR_NULL = -1,           /* a required pointer is NULL */
  BZ_ERR_SHAPE = -2,          /* a size is out of range or num_q_heads % num_kv_heads != 0 */
  BZ_ERR_UNSUPPORTED = -3,    /* head_dim or GQA group size without a compiled kernel */
  BZ_ERR_ALIGNMENT = -4,      /* K/V base pointers or strides not 16-byte aligned */
  BZ_ERR_WORKSPACE = -5,      /* workspace NULL or smaller than bz_gqa_decode_workspace_size() */
  BZ_ERR_MASK_DTYPE = -6,     /* mask_dtype is not one of bz_mask_dtype */
  BZ_ERR_LAUNCH = -7,         /* hipLaunchKernelGGL / hipGetLastError reported an error */
  BZ_ERR_DEVICE = -8,         /* hipGetDevice / hipDeviceGetAttribute failed */
  BZ_ERR_COMBINE_MODE = -9,   /* combine is not one of bz_combine_mode */
  BZ_ERR_SCRATCH = -10        /* bz_gqa_decode_noalloc: the sizes exceed its static scratch */
} bz_status;

typedef enum bz_mask_dtype {
  BZ_MASK_NONE = 0,           /* no additive mask */
  BZ_MASK_BF16 = 1,           /* bf16 additive mask (the reference's serving dtype) */
  BZ_MASK_F32 = 2             /* fp32 additive mask */
} bz_mask_dtype;

typedef enum bz_combine_mode {
  BZ_COMBINE_AUTO = 0,        /* library default */
  BZ_COMBINE_LAST_BLOCK = 1,  /* the last workgroup of each (batch, kv head) merges the splits: one launch */
  BZ_COMBINE_KERNEL = 2       /* a second kernel merges the splits: two launches */
} bz_combine_mode;

/* Arguments of bz_gqa_decode (the reference op's (q, k_cache, v_cache, seq_lens, scale) -> out). */
typedef struct bz_gqa_decode_args {
  /* query [batch, num_q_heads, head_dim] bf16: element (b, h, d) at q[b*q_stride_b + h*q_stride_h + d]; q and its
     strides 16-byte aligned (multiples of 8 elements) */
  const void* q;
  int64_t q_stride_b, q_stride_h;
  /* KV cache [batch, num_kv_heads, capacity, head_dim] bf16 (transformers StaticCache layer layout). K and V
     share strides; k_cache, v_cache and all three strides must be 16-byte aligned (multiples of 8 elements).
     One (batch, kv head) span must be addressable with 31-bit byte offsets: (capacity + 1024) * kv_stride_s * 2
     < 2^31, else BZ_ERR_SHAPE. */
  const void* k_cache;
  const void* v_cache;
  int64_t kv_stride_b, kv_stride_h, kv_stride_s;
  /* [batch] int32: row b attends [kv_start[b], seq_lens[b]). kv_start may be NULL (all zeros). Values are
     clamped on the device to 0 <= kv_start <= seq_lens <= capacity, so no access leaves the cache. */
  const int32_t* seq_lens;
  const int32_t* kv_start;
  /* optional additive mask, row b at mask + b*mask_stride_b (mask_stride_b = 0 broadcasts one row), position p
     at element p, p < capacity. A position whose mask value is <= -1e30 is excluded (the reference's threshold
     for finfo.min); other values are added to the scaled score. */
  const void* mask;
  int32_t mask_dtype;         /* bz_mask_dtype */
  int64_t mask_stride_b;
  float scale;                /* softmax scale (head_dim ** -0.5 for the reference's layers) */
  /* out [batch, num_q_heads, head_dim] bf16 */
  void* out;
  int64_t out_stride_b, out_stride_h;
  int32_t batch, num_q_heads, num_kv_heads, head_dim, capacity;
  /* workgroups per (batch, kv head); 0 picks bz_gqa_decode_default_splits(.., max_seq_len or capacity, ..) */
  int32_t num_splits;
  /* expected upper bound of seq_lens - kv_start (0 = capacity); only steers the default tiling */
  int32_t max_seq_len;
  int32_t combine;            /* bz_combine_mode */
  /* caller-owned scratch of at least bz_gqa_decode_workspace_size() bytes, 256-byte aligned. It must be
     zero-filled once before first use; the library leaves it ready for the next call with the same
     batch * tokens_per_row * num_kv_heads (see the conventions above). */
  void* workspace;
  size_t workspace_bytes;
  /* Query tokens per row, T (0 or 1: one). With T > 1 each row carries its last T positions as queries, causal
     among themselves (the depth transformer's first step, flash/csrc/depth_frame.cu:221-227): token t of row b
     attends [kv_start[b], seq_lens[b] - (T - 1 - t)). q element (b, t, h, d) is at q[b*q_stride_b + t*q_stride_t +
     h*q_stride_h + d], out element (b, t, h, d) at out[b*out_stride_b + t*out_stride_t + h*out_stride_h + d]. The
     workspace and the default split count are those of batch * T rows. bz_gqa_decode_fused takes T = 1 only. */
  int32_t tokens_per_row;
  int64_t q_stride_t, out_stride_t;
} bz_gqa_decode_args;

/* GQA decode attention. Replaces the reference op attn_decode (flash/csrc/bb_attn.cu:416-429, pybind :463-465)
   with the north-star signature (q, k_cache, v_cache, seq_lens, scale) -> out; kv_start carries the left-padding
   start the reference encodes in its interval mask (backbone_graph.py:239-252). With num_splits 0, combine AUTO and
   no mask, on short rows (max_seq_len, else capacity: at most 4096 / head_dim positions for 2 q heads per kv head,
   8192 / head_dim for 4 or more) it runs the kernel of bz_gqa_decode_wave (the depth transformer's shape); otherwise
   the split kernel. */
int bz_gqa_decode(const bz_gqa_decode_args* args, hipStream_t stream);

/* bz_gqa_decode without a workspace and without any allocation: args->workspace and args->workspace_bytes are ignored
   and the split partials and arrival counters live in a static scratch of the library (8 MiB per device, held until
   the process ends). No counterpart in the reference (which takes caller-owned workspaces); it is for callers that
   cannot allocate: code under HIP graph capture (such as torch.compile's CUDA-graph trees) or serving loops that
   forbid allocation. With args->seq_lens NULL the range of each row comes from args->mask, as in
   bz_gqa_decode_masked. Limits: at most 1024 (row, kv head) groups (batch * tokens_per_row * num_kv_heads) and
   8 MiB of split partials (batch * tokens_per_row * num_q_heads * splits * (head_dim + 2) * 4 bytes), else
   BZ_ERR_SCRATCH. Every call on a device shares that device's scratch: calls that overlap in time on one device
   (several streams, several host threads) race and must be ordered by the caller. */
int bz_gqa_decode_noalloc(const bz_gqa_decode_args* args, hipStream_t stream);

/* Bytes of workspace bz_gqa_decode needs for these sizes (num_splits as passed, 0 = default; with tokens_per_row
   T > 1 pass batch * T). Replaces the caller-side sizing of the reference's scores/cmax/part/counters buffers
   (flash/backbone.py:27-37). */
int bz_gqa_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t capacity, int32_t num_splits, int32_t max_seq_len, size_t* bytes);

/* The split count bz_gqa_decode uses when num_splits == 0 (device CU count, sizes; with tokens_per_row T > 1 pass
   batch * T). No counterpart in the
   reference, which fixes 64-position chunks at compile time (bb_attn.cu:28, :382). */
int bz_gqa_decode_default_splits(int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t capacity,
                                 int32_t max_seq_len, int32_t* num_splits);

/* Interval-mask form used by the reference's BackboneGraph: derives [kv_start, seq_end) for each row on the
   device from an additive mask [batch or 1, capacity] (first and last position with mask > -1e30), then runs
   bz_gqa_decode with that mask applied inside the interval. args->seq_lens / args->kv_start are ignored; args->mask
   is required. Replaces attn_decode's mask argument (bb_attn.cu:416-418, mask scan :111-117). */
int bz_gqa_decode_masked(const bz_gqa_decode_args* args, hipStream_t stream);

/* Arguments of bz_gqa_decode_fused: the raw q | k | v projections of the decode token, the q / k RMSNorm weights and
   the RoPE tables, and the cache slot the new k and v go to. base.q is ignored (q comes from qkv); base.k_cache and
   base.v_cache must be writable; head_dim must be 128. All pointers and strides 16-byte aligned. */
typedef struct bz_gqa_decode_fused_args {
  bz_gqa_decode_args base;
  /* [batch, (num_q_heads + 2 * num_kv_heads) * head_dim] bf16: q heads, then k heads, then v heads (Qwen3 q/k/v_proj) */
  const void* qkv;
  int64_t qkv_stride_b;
  const void* q_norm_weight;  /* [head_dim] bf16 */
  const void* k_norm_weight;  /* [head_dim] bf16 */
  float eps;                  /* RMSNorm epsilon */
  const void* cos;            /* [batch, head_dim] bf16 RoPE tables of this token's position */
  const void* sin;
  int64_t rope_stride_b;
  const int64_t* cache_pos;   /* device scalar: the cache slot written with the new k and v (all rows) */
} bz_gqa_decode_fused_args;

/* Fused decode step: q_norm / k_norm (Qwen3 RMSNorm) and RoPE on the raw projections at the eager bf16 rounding points,
   the new k (normed, roped) and v written into slot *cache_pos of every row's cache (skipped when the slot lies
   outside [0, capacity)), then bz_gqa_decode over the updated cache. With base.seq_lens set, rows attend
   [kv_start, seq_lens); with base.seq_lens NULL, the range comes from base.mask as in bz_gqa_decode_masked.
   Replaces attn_decode_fused (flash/csrc/bb_attn.cu:433-460, prologue :78-149, pybind :466-469), the entry the
   reference's decode step calls (flash/backbone.py:123-124). */
int bz_gqa_decode_fused(const bz_gqa_decode_fused_args* args, hipStream_t stream);

/* The same attention as bz_gqa_decode (seq_lens / kv_start ranges, tokens_per_row causal tokens), computed by one
   wave per (row, token, q head) with no split, no workspace and no barrier. The wave's work is the device function
   attend_wave (breeze-tts-2-flash_amd/csrc/gqa_wave.cuh), the attention stage for a kernel that runs a whole depth
   decode step in one launch, as the reference's depth megakernel does (flash/csrc/depth_frame.cu:208-272, at most 17
   positions per step); this entry launches it alone, so that it is tested and timed through the C ABI. Each q head
   reads its K/V itself, so it is faster than bz_gqa_decode only on short rows already in the cache hierarchy (the
   real depth shape); on cold or long rows it is slower. No mask (BZ_ERR_UNSUPPORTED); out and its strides 16-byte
   aligned; workspace, num_splits, max_seq_len and combine are ignored; any row length works. */
int bz_gqa_decode_wave(const bz_gqa_decode_args* args, hipStream_t stream);

/* The softmax probabilities of the bz_gqa_decode call with these arguments: probs[(b * num_q_heads + h) * capacity + p]
   = bf16(exp(s - max) / sum) as fp32 for position p inside row b's range (s the scaled score of q head h plus the
   mask's value, max and sum over the range), 0 at excluded positions and outside the range; every p < capacity is
   written. The range comes from seq_lens / kv_start, or with seq_lens NULL from the mask (as bz_gqa_decode_masked);
   a mask, when given, is added inside the range. tokens_per_row must be 1; out and v_cache are not read or written;
   probs is a float [batch, num_q_heads, capacity] device array, 4-byte aligned. Replaces the optional dbg output of
   attn_decode / attn_decode_fused (flash/csrc/bb_attn.cu:74, :288-289, :323-325, :401-405): a verification path,
   three passes over the row, not a fast one. */
int bz_gqa_decode_probs(const bz_gqa_decode_args* args, float* probs, hipStream_t stream);

/* bz_gqa_decode_probs for the fused step: the probabilities of the bz_gqa_decode_fused call with these arguments,
   made after it (the cache then holds the step's new k at cache_pos; q is the raw projection in qkv, normed and
   rotated as the fused kernel does it). The dbg output of attn_decode_fused (bb_attn.cu:288-289, :401-405). */
int bz_gqa_decode_fused_probs(const bz_gqa_decode_fused_args* args, float* probs, hipStream_t stream);

/* Per row b, the interval [kv_start[b], seq_lens[b]) of positions p < capacity whose additive mask value is > -1e30
   ([0, 0) for a row with none): the range bz_gqa_decode_masked and the mask form of bz_gqa_decode_fused derive on the
   device, written to caller buffers so that one launch serves every layer of a decode step, whose layers share one
   mask, and the per-layer calls pass seq_lens / kv_start. Inverts the reference's mask construction from pad_lens
   and the position (third_party/breeze-tts/models/cudagraph/backbone_graph.py:239-252), which its attention
   re-reads per layer to skip masked chunks (flash/csrc/bb_attn.cu:111-117). mask: bz_mask_dtype BF16 or F32, row b
   at mask + b*mask_stride_b (0 broadcasts one row); seq_lens, kv_start: int32 [batch] device arrays. */
int bz_mask_interval(const void* mask, int32_t mask_dtype, int64_t mask_stride_b, int32_t batch, int32_t capacity,
                     int32_t* seq_lens, int32_t* kv_start, hipStream_t stream);

/* Human-readable text of a bz_status. */
const char* bz_status_string(int status);

/* BZ_GQA_DECODE_ABI_VERSION of the loaded library. */
int bz_gqa_decode_abi_version(void);

/* Identity of the sources and compiler flags the library was built from (a hex string; "unknown" when built without
   one). The Python loader compares it with the sources next to the library and refuses a stale build, as the
   reference's loader rebuilds its extension when a source or a flag changes (flash/kernels.py:1-4, :64-79). */
const char* bz_gqa_decode_build_id(void);

#ifdef __cplusplus
}
#endif

#endif /* BZ_GQA_DECODE_H */
