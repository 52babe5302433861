// Kernel table of the fused-prologue variants (q_norm / k_norm + RoPE + KV-cache write, then attention; the
// reference's attn_decode_fused, flash/csrc/bb_attn.cu:433-460), in a translation unit of its own so that it
// compiles in parallel with gqa_decode.hip. head_dim 128 only, as in the reference (bb_attn.cu:27).
#include "gqa_kernels.cuh"

namespace bz {

SplitFn pick_split_fused(int D, int G, int mk, int ppt, int nt) {
  if (D != 128) return nullptr;
  return nt == 512 ? pick_group<128, 512, true>(G, mk, ppt) : pick_group<128, 256, true>(G, mk, ppt);
}

}  // namespace bz
