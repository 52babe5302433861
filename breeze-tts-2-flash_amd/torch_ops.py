"""The library's entry points as torch operators (namespace "bz", torch.library.custom_op), so that torch.compile
treats each call as one opaque graph node instead of breaking the graph at the ctypes call. The reference's ops are
torch operators through its pybind extension (flash/csrc/bb_attn.cu:462-469, bb_fused.cu:370-377); here the C ABI
stays the boundary and each operator's implementation is the package function's own call through it.

Each operator writes its outputs in place (declared in mutates_args) and returns nothing; the fake implementations
(shapes only) do nothing, as the outputs are the caller's tensors. bz::gqa_decode and bz::gqa_decode_masked without a
workspace run on the library's static scratch (bz_gqa_decode_noalloc), so that a compiled graph allocates nothing
inside torch.compile's CUDA-graph trees; bz::gqa_decode_fused has no such form and takes the stream's cached
workspace, so under CUDA-graph trees pass it a workspace allocated beforehand. The package functions (attention.gqa_decode and
the rest) call these operators while torch.compile traces them and call the C ABI directly otherwise, which keeps the
eager per-call host cost of a plain function call.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import attention, gemv

_M = ("out",)


@torch.library.custom_op("bz::gqa_decode", mutates_args=("out", "workspace"))
def gqa_decode(q: Tensor, k_cache: Tensor, v_cache: Tensor, seq_lens: Tensor, scale: float, out: Tensor,
               kv_start: Optional[Tensor], mask: Optional[Tensor], num_splits: int, max_seq_len: int, combine: int,
               workspace: Optional[Tensor]) -> None:
    attention._gqa_decode(q, k_cache, v_cache, seq_lens, scale, out, kv_start, mask, num_splits, max_seq_len, combine,
                          workspace, static_scratch=True)


@gqa_decode.register_fake
def _(q, k_cache, v_cache, seq_lens, scale, out, kv_start, mask, num_splits, max_seq_len, combine, workspace):
    return None


@torch.library.custom_op("bz::gqa_decode_wave", mutates_args=_M)
def gqa_decode_wave(q: Tensor, k_cache: Tensor, v_cache: Tensor, seq_lens: Tensor, scale: float, out: Tensor,
                    kv_start: Optional[Tensor]) -> None:
    attention._gqa_decode_wave(q, k_cache, v_cache, seq_lens, scale, out, kv_start)


@gqa_decode_wave.register_fake
def _(q, k_cache, v_cache, seq_lens, scale, out, kv_start):
    return None


@torch.library.custom_op("bz::gqa_decode_masked", mutates_args=("out", "workspace"))
def gqa_decode_masked(q: Tensor, k_cache: Tensor, v_cache: Tensor, mask: Tensor, scale: float, out: Tensor,
                      num_splits: int, max_seq_len: int, combine: int, workspace: Optional[Tensor]) -> None:
    attention._gqa_decode_masked(q, k_cache, v_cache, mask, scale, out, num_splits, max_seq_len, combine, workspace,
                                 static_scratch=True)


@gqa_decode_masked.register_fake
def _(q, k_cache, v_cache, mask, scale, out, num_splits, max_seq_len, combine, workspace):
    return None


@torch.library.custom_op("bz::gqa_decode_fused", mutates_args=("k_cache", "v_cache", "out", "workspace"))
def gqa_decode_fused(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, eps: float, cos: Tensor, sin: Tensor,
                     k_cache: Tensor, v_cache: Tensor, cache_pos: Tensor, scale: float, out: Tensor,
                     seq_lens: Optional[Tensor], kv_start: Optional[Tensor], mask: Optional[Tensor], num_splits: int,
                     max_seq_len: int, combine: int, workspace: Optional[Tensor]) -> None:
    attention._gqa_decode_fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale,
                                out, seq_lens, kv_start, mask, num_splits, max_seq_len, combine, workspace)


@gqa_decode_fused.register_fake
def _(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale, out, seq_lens, kv_start,
      mask, num_splits, max_seq_len, combine, workspace):
    return None


@torch.library.custom_op("bz::gemv_seg", mutates_args=("y",))
def gemv_seg(x: Tensor, nw: Optional[Tensor], eps: float, W0: Tensor, W1: Optional[Tensor], W2: Optional[Tensor],
             y: Tensor) -> None:
    gemv._gemv_seg(x, nw, eps, W0, W1, W2, y)


@gemv_seg.register_fake
def _(x, nw, eps, W0, W1, W2, y):
    return None


@torch.library.custom_op("bz::gemv_resid", mutates_args=("y",))
def gemv_resid(x: Tensor, W: Tensor, res: Tensor, y: Tensor) -> None:
    gemv._gemv_resid(x, W, res, y)


@gemv_resid.register_fake
def _(x, W, res, y):
    return None


@torch.library.custom_op("bz::gemv_gateup", mutates_args=("y",))
def gemv_gateup(x: Tensor, nw: Tensor, eps: float, Wg: Tensor, Wu: Tensor, y: Tensor) -> None:
    gemv._gemv_gateup(x, nw, eps, Wg, Wu, y)


@gemv_gateup.register_fake
def _(x, nw, eps, Wg, Wu, y):
    return None


@torch.library.custom_op("bz::rmsnorm", mutates_args=("y",))
def rmsnorm(x: Tensor, w: Tensor, eps: float, y: Tensor) -> None:
    gemv._rmsnorm(x, w, eps, y)


@rmsnorm.register_fake
def _(x, w, eps, y):
    return None
