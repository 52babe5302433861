"""The reference's ops under their own names and argument order, for its call sites.

attn_decode(query, kc, vc, mask, scaling, scores, cmax, part, counters, out, dbg=None) is the pybind signature of
flash/csrc/bb_attn.cu:463-465 (host function :416-429). The reference takes the KV range from an additive interval
mask (valid = [pad_lens[b], position], everything else finfo.min; backbone_graph.py:239-252) and needs four
caller-owned workspaces. Here the range is derived from the mask on the device (bz_gqa_decode_masked); scores / cmax /
part / counters are accepted for signature compatibility and left untouched. attn_decode takes the library's
workspace handling (a captured call runs on its static scratch). attn_decode_fused keeps one library workspace per
reference workspace it is called with (keyed by the `counters` tensor, which the reference allocates once per
device and shape, flash/backbone.py:27-37), made at the first call: the reference's BackboneGraph.capture() runs the
step eagerly before it captures (backbone_graph.py:288-315), so the captured call finds it and allocates nothing. The
reference's optional dbg output (float32 [B, NH, S], the bf16-rounded softmax probabilities,
bb_attn.cu:288-289, checked at :401-405) is produced when given, by a second launch after the attention
(bz_gqa_decode_probs / bz_gqa_decode_fused_probs); the reference's decode step passes none (flash/backbone.py:123-124).
"""
from __future__ import annotations

import torch

from . import attention
from .attention import gqa_decode_fused, gqa_decode_masked, gqa_decode_probs, workspace_bytes

_WS: dict = {}  # (device index, counters data_ptr or 0) -> the library workspace of attn_decode_fused calls


def _fused_workspace(qkv: torch.Tensor, kc: torch.Tensor, NH: int, counters) -> torch.Tensor:
    """The library workspace for attn_decode_fused calls made with this reference `counters` buffer (zero-filled,
    replaced by a larger one when a call needs more). Raises instead of allocating while the stream is being
    captured."""
    B, NKV, cap, D = kc.shape
    idx = qkv.device.index if qkv.device.index is not None else torch.cuda.current_device()
    key = (idx, counters.data_ptr() if isinstance(counters, torch.Tensor) else 0)
    with torch.cuda.device(idx):
        need = workspace_bytes(B, NH, NKV, D, cap)
    ws = _WS.get(key)
    if ws is not None and ws.numel() >= need:
        return ws
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("attn_decode_fused: no workspace exists yet for these sizes, and nothing is allocated during "
                           "a capture: run the decode step once eagerly before capturing it (as BackboneGraph.capture "
                           "does)")
    ws = attention._zeroed_outside_pools((need + 255) // 256 * 256, idx)
    if ws.data_ptr() % 256:
        raise RuntimeError("workspace allocation is not 256-byte aligned")
    _WS[key] = ws
    return ws


def _check_dbg(dbg: torch.Tensor, B: int, NH: int, S: int, device, what: str) -> None:
    """The reference's dbg check (bb_attn.cu:401-405), made before anything is launched."""
    if not (dbg.dtype == torch.float32 and dbg.is_contiguous() and dbg.device == device and dbg.numel() >= B * NH * S):
        raise RuntimeError(f"{what}: dbg must be a contiguous float32 tensor on the query's device with at least "
                           f"B * NH * S = {B * NH * S} elements")


def attn_decode(query: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, mask: torch.Tensor, scaling: float,
                scores=None, cmax=None, part=None, counters=None, out: torch.Tensor | None = None,
                dbg: torch.Tensor | None = None) -> torch.Tensor:
    """query [B, NH, 1, D] bf16; kc/vc [B, NKV, S, D] bf16 (stride(3) == 1); mask [B or 1, 1, 1, >= S] bf16/fp32;
    out [B, 1, NH, D] bf16 contiguous (the eager attn_output.transpose(1, 2) layout); dbg, when given, float32
    contiguous with at least B * NH * S elements, receives the probabilities. Returns out."""
    if query.dim() != 4 or query.size(2) != 1:
        raise RuntimeError(f"attn_decode: query must be [B, NH, 1, D], got {tuple(query.shape)}")
    if out is None:
        out = torch.empty(query.size(0), 1, query.size(1), query.size(3), dtype=torch.bfloat16, device=query.device)
    if mask.dim() != 4 or mask.size(2) != 1:
        raise RuntimeError(f"attn_decode: mask must be [B or 1, 1, 1, S], got {tuple(mask.shape)}")
    if dbg is not None:
        _check_dbg(dbg, query.size(0), query.size(1), kc.size(2), query.device, "attn_decode")
    gqa_decode_masked(query, kc, vc, mask, scaling, out)
    if dbg is not None:
        gqa_decode_probs(query, kc, None, scaling, dbg, mask=mask)
    return out


def attn_decode_fused(qkv: torch.Tensor, qn_w: torch.Tensor, kn_w: torch.Tensor, eps: float, cos: torch.Tensor,
                      sin: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, mask: torch.Tensor,
                      cache_pos: torch.Tensor, scaling: float, scores=None, cmax=None, part=None, counters=None,
                      out: torch.Tensor | None = None, dbg: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's fused decode step, pybind signature flash/csrc/bb_attn.cu:466-469 (host function :433-460),
    as called by flash/backbone.py:123-124: qkv [B, (NH + 2 NKV) * 128] raw projections, qn_w/kn_w [128],
    cos/sin [B, 1, 128], kc/vc the layer's StaticCache tensors (written at slot cache_pos[0]), mask the interval
    mask, out [B, 1, NH, 128]. The four workspaces are accepted and left untouched (`counters` keys the library
    workspace the call uses); dbg, when given (float32, contiguous, at least B * NH * S elements), receives the step's
    probabilities, its own new position included."""
    NKV, D = kc.size(1), kc.size(3)
    NH = qkv.size(1) // D - 2 * NKV
    if out is None:
        out = torch.empty(qkv.size(0), 1, NH, D, dtype=torch.bfloat16, device=qkv.device)
    if mask.dim() != 4 or mask.size(2) != 1:
        raise RuntimeError(f"attn_decode_fused: mask must be [B or 1, 1, 1, S], got {tuple(mask.shape)}")
    ws = _fused_workspace(qkv, kc, NH, counters)
    if dbg is None:
        return gqa_decode_fused(qkv, qn_w, kn_w, eps, cos, sin, kc, vc, cache_pos, scaling, out, mask=mask,
                                workspace=ws)
    _check_dbg(dbg, qkv.size(0), out.size(2), kc.size(2), qkv.device, "attn_decode_fused")
    return attention._gqa_decode_fused(qkv, qn_w, kn_w, eps, cos, sin, kc, vc, cache_pos, scaling, out, None, None,
                                       mask, 0, 0, "auto", ws, probs=dbg)
