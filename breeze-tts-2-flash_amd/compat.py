"""The reference's ops under their own names and argument order, for its call sites.

attn_decode(query, kc, vc, mask, scaling, scores, cmax, part, counters, out, dbg=None) is the pybind signature of
flash/csrc/bb_attn.cu:463-465 (host function :416-429). The reference takes the KV range from an additive interval
mask (valid = [pad_lens[b], position], everything else finfo.min; backbone_graph.py:239-252) and needs four
caller-owned workspaces. Here the range is derived from the mask on the device (bz_gqa_decode_masked) and the
library's own cached workspace is used; scores / cmax / part / counters are accepted for signature compatibility and
left untouched. The reference's optional dbg output (bf16-rounded probabilities, bb_attn.cu:288) has no caller
(flash/backbone.py:123-124 passes none) and is not produced: passing one raises.
"""
from __future__ import annotations

import torch

from .attention import gqa_decode_fused, gqa_decode_masked


def attn_decode(query: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, mask: torch.Tensor, scaling: float,
                scores=None, cmax=None, part=None, counters=None, out: torch.Tensor | None = None,
                dbg: torch.Tensor | None = None) -> torch.Tensor:
    """query [B, NH, 1, D] bf16; kc/vc [B, NKV, S, D] bf16 (stride(3) == 1); mask [B or 1, 1, 1, >= S] bf16/fp32;
    out [B, 1, NH, D] bf16 contiguous (the eager attn_output.transpose(1, 2) layout). Returns out."""
    if dbg is not None:
        raise RuntimeError("attn_decode: the dbg probabilities output is not supported")
    if query.dim() != 4 or query.size(2) != 1:
        raise RuntimeError(f"attn_decode: query must be [B, NH, 1, D], got {tuple(query.shape)}")
    if out is None:
        out = torch.empty(query.size(0), 1, query.size(1), query.size(3), dtype=torch.bfloat16, device=query.device)
    if mask.dim() != 4 or mask.size(2) != 1:
        raise RuntimeError(f"attn_decode: mask must be [B or 1, 1, 1, S], got {tuple(mask.shape)}")
    return gqa_decode_masked(query, kc, vc, mask, scaling, out)


def attn_decode_fused(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float, cos: torch.Tensor,
                      sin: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, mask: torch.Tensor,
                      cache_pos: torch.Tensor, scaling: float, scores=None, cmax=None, part=None, counters=None,
                      out: torch.Tensor | None = None, dbg: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's fused decode step, pybind signature flash/csrc/bb_attn.cu:466-469 (host function :433-460),
    as called by flash/backbone.py:123-124: qkv [B, (NH + 2 NKV) * 128] raw projections, qn_w/kn_w [128],
    cos/sin [B, 1, 128], kc/vc the layer's StaticCache tensors (written at slot cache_pos[0]), mask the interval
    mask, out [B, 1, NH, 128]. The four workspaces are accepted and left untouched; dbg is not supported."""
    if dbg is not None:
        raise RuntimeError("attn_decode_fused: the dbg probabilities output is not supported")
    if out is None:
        NKV, D = kc.size(1), kc.size(3)
        NH = qkv.size(1) // D - 2 * NKV
        out = torch.empty(qkv.size(0), 1, NH, D, dtype=torch.bfloat16, device=qkv.device)
    if mask.dim() != 4 or mask.size(2) != 1:
        raise RuntimeError(f"attn_decode_fused: mask must be [B or 1, 1, 1, S], got {tuple(mask.shape)}")
    return gqa_decode_fused(qkv, qn_w, kn_w, eps, cos, sin, kc, vc, cache_pos, scaling, out, mask=mask)
