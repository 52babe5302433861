// Kernel table of the fused-prologue variants (q_norm / k_norm + RoPE + KV-cache write, then attention; the
// reference's attn_decode_fused, flash/csrc/bb_attn.cu:433-460), in a translation unit of its own so that it
// compiles in parallel with gqa_decode.hip. head_dim 128 only, as in the reference (bb_attn.cu:27).
#include "gqa_kernels.cuh"

namespace bz {

SplitFn pick_split_fused(int D, int G, int mk, int ppt, int nt) {
  if (D != 128 || nt != kSplitThreads) return nullptr;
  return pick_group<128, kSplitThreads, true>(G, mk, ppt);
}

}  // namespace bz
