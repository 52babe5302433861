"""MI355X (gfx950) GQA flash-decoding attention for Breeze-TTS-2-flash's decode steps.

Public API:
  gqa_decode(q, k_cache, v_cache, seq_lens, scale, out=None, *, kv_start=None, mask=None, num_splits=0, ...)
  gqa_decode_masked(q, k_cache, v_cache, mask, scale, out=None, ...)
  attn_decode(query, kc, vc, mask, scaling, scores, cmax, part, counters, out, dbg=None)   (reference order)
  build() / load()   compile / open libbz_gqa_decode.so (C ABI: include/bz_gqa_decode.h)
"""
from .attention import default_splits, get_workspace, gqa_decode, gqa_decode_masked, workspace_bytes
from .compat import attn_decode
from .kernels import build, load

__all__ = ["gqa_decode", "gqa_decode_masked", "attn_decode", "workspace_bytes", "default_splits", "get_workspace",
           "build", "load"]
