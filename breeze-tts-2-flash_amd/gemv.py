"""The backbone decode GEMVs under the reference's names and argument order (flash/csrc/bb_fused.cu:370-377, called by
flash/backbone.py:122-129): gemv_seg, gemv_resid, gemv_gateup and rmsnorm, on bz_gemv / bz_rmsnorm
(include/bz_gemv.h). The reference's tuning arguments R, U and warps (rows per warp, unroll, warps per block, tuned
per batch size for its GPU in flash/backbone.py:18-22) are accepted and ignored: the library picks its own tiling.
Argument errors raise RuntimeError, as the reference's TORCH_CHECKs do.
"""
from __future__ import annotations

import torch

from . import kernels


def gemv_seg(x: torch.Tensor, nw: torch.Tensor | None, eps: float, W0: torch.Tensor, W1: torch.Tensor,
             W2: torch.Tensor, y: torch.Tensor, R: int = 2, U: int = 1, warps: int = 8) -> torch.Tensor:
    """y[:, 0:N0+N1+N2] = norm?(x) @ [W0; W1; W2]^T (bb_fused.cu:293-317). W1 / W2 may be empty tensors; nw None
    skips the RMSNorm. Returns y. Under torch.compile the call is the registered operator torch.ops.bz.gemv_seg."""
    if torch.compiler.is_compiling():
        torch.ops.bz.gemv_seg(x, nw, float(eps), W0, W1, W2, y)
        return y
    return _gemv_seg(x, nw, eps, W0, W1, W2, y)


def _gemv_seg(x, nw, eps, W0, W1, W2, y) -> torch.Tensor:
    """gemv_seg's call through the C ABI (the body of the eager path and of torch.ops.bz.gemv_seg): the argument
    checks, the device and stream, and bz_gemv in one native call (csrc/eager_ext.cpp)."""
    return kernels.eager().gemv(0, x, nw, float(eps), W0, W1, W2, None, y)


def gemv_resid(x: torch.Tensor, W: torch.Tensor, res: torch.Tensor, y: torch.Tensor, R: int = 2, U: int = 1,
               warps: int = 8) -> torch.Tensor:
    """y = res + x @ W^T with the GEMV rounded to bf16 before the add, as eager (bb_fused.cu:319-335). Returns y.
    Under torch.compile the call is the registered operator torch.ops.bz.gemv_resid."""
    if torch.compiler.is_compiling():
        torch.ops.bz.gemv_resid(x, W, res, y)
        return y
    return _gemv_resid(x, W, res, y)


def _gemv_resid(x, W, res, y) -> torch.Tensor:
    """gemv_resid's call through the C ABI (native, as _gemv_seg)."""
    return kernels.eager().gemv(1, x, None, 0.0, W, None, None, res, y)


def gemv_gateup(x: torch.Tensor, nw: torch.Tensor, eps: float, Wg: torch.Tensor, Wu: torch.Tensor, y: torch.Tensor,
                R: int = 1, U: int = 1, warps: int = 8) -> torch.Tensor:
    """y = silu(norm(x) @ Wg^T) * (norm(x) @ Wu^T) at the eager rounding points (bb_fused.cu:337-356). Returns y.
    Under torch.compile the call is the registered operator torch.ops.bz.gemv_gateup."""
    if torch.compiler.is_compiling():
        torch.ops.bz.gemv_gateup(x, nw, float(eps), Wg, Wu, y)
        return y
    return _gemv_gateup(x, nw, eps, Wg, Wu, y)


def _gemv_gateup(x, nw, eps, Wg, Wu, y) -> torch.Tensor:
    """gemv_gateup's call through the C ABI (native, as _gemv_seg)."""
    return kernels.eager().gemv(2, x, nw, float(eps), Wg, Wu, None, None, y)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, y: torch.Tensor) -> torch.Tensor:
    """y = Qwen3RMSNorm(x) row by row (bb_fused.cu:358-368). Returns y. Under torch.compile the call is the registered
    operator torch.ops.bz.rmsnorm."""
    if torch.compiler.is_compiling():
        torch.ops.bz.rmsnorm(x, w, float(eps), y)
        return y
    return _rmsnorm(x, w, eps, y)


def _rmsnorm(x, w, eps, y) -> torch.Tensor:
    """rmsnorm's call through the C ABI (native, as _gemv_seg)."""
    return kernels.eager().rmsnorm(x, w, float(eps), y)
