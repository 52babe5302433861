"""MI355X (gfx950) GQA flash-decoding attention for Breeze-TTS-2-flash's decode steps.

Public API:
  gqa_decode(q, k_cache, v_cache, seq_lens, scale, out=None, *, kv_start=None, mask=None, num_splits=0, ...)
  gqa_decode_masked(q, k_cache, v_cache, mask, scale, out=None, ...)
  gqa_decode_wave(q, k_cache, v_cache, seq_lens, scale, out=None, *, kv_start=None)   one wave per q head, short rows
  gqa_decode_fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale, ...)
  gqa_decode_probs(q, k_cache, seq_lens, scale, probs=None, *, kv_start=None, mask=None)   softmax probabilities (dbg)
  attn_decode(query, kc, vc, mask, scaling, scores, cmax, part, counters, out, dbg=None)   (reference order)
  attn_decode_fused(qkv, qn_w, kn_w, eps, cos, sin, kc, vc, mask, cache_pos, scaling, ..., out, dbg=None)
  gemv_seg / gemv_resid / gemv_gateup / rmsnorm   backbone decode GEMVs (reference order; C ABI include/bz_gemv.h)
  mask_interval(mask, capacity, ...)   the [kv_start, seq_lens) rows of an interval mask, once per decode step
  backbone.fused_decode_step(graph) / backbone.install(BackboneGraph)   the whole backbone decode step
  build() / load()   compile / open libbz_gqa_decode.so (C ABI: include/bz_gqa_decode.h, include/bz_gemv.h)
  torch.ops.bz.*     the same entry points as torch operators (torch_ops.py), used while torch.compile traces
"""
from .attention import (default_splits, get_workspace, gqa_decode, gqa_decode_fused, gqa_decode_masked,
                        gqa_decode_probs, gqa_decode_wave, mask_interval, workspace_bytes)
from .compat import attn_decode, attn_decode_fused
from .gemv import gemv_gateup, gemv_resid, gemv_seg, rmsnorm
from .kernels import build, load
from . import backbone, hf_attention, torch_ops

__all__ = ["gqa_decode", "gqa_decode_masked", "gqa_decode_wave", "gqa_decode_fused", "gqa_decode_probs", "attn_decode",
           "attn_decode_fused", "gemv_seg", "gemv_resid", "gemv_gateup", "rmsnorm", "mask_interval", "backbone",
           "workspace_bytes", "default_splits", "get_workspace", "build", "load"]
