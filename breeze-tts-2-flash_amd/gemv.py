"""The backbone decode GEMVs under the reference's names and argument order (flash/csrc/bb_fused.cu:370-377, called by
flash/backbone.py:122-129): gemv_seg, gemv_resid, gemv_gateup and rmsnorm, on bz_gemv / bz_rmsnorm
(include/bz_gemv.h). The reference's tuning arguments R, U and warps (rows per warp, unroll, warps per block, tuned
per batch size for its GPU in flash/backbone.py:18-22) are accepted and ignored: the library picks its own tiling.
Argument errors raise RuntimeError, as the reference's TORCH_CHECKs do.
"""
from __future__ import annotations

import ctypes

import torch

from . import kernels


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _x2d(x: torch.Tensor, name: str = "x") -> tuple[int, int]:
    _check(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1,
           f"{name} must be a bf16 [M, K] device tensor with a contiguous last dim")
    M, K = x.shape
    _check(1 <= M <= 4, f"{name}: M must be 1..4, got {M}")
    _check(K % 8 == 0 and x.stride(0) % 8 == 0, f"{name}: K and the row stride must be multiples of 8")
    return M, K


def _w(W: torch.Tensor, K: int, name: str) -> int:
    _check(W.is_cuda and W.dtype == torch.bfloat16 and W.is_contiguous() and W.dim() == 2 and W.size(1) == K,
           f"{name} must be a contiguous bf16 [N, {K}] device tensor")
    return W.size(0)


def _y(y: torch.Tensor, M: int, N: int, name: str = "y") -> None:
    _check(y.is_cuda and y.dtype == torch.bfloat16 and y.dim() == 2 and tuple(y.shape) == (M, N) and y.stride(1) == 1,
           f"{name} must be a bf16 [{M}, {N}] device tensor with a contiguous last dim")


def _norm_w(nw: torch.Tensor, K: int) -> None:
    _check(nw.is_cuda and nw.dtype == torch.bfloat16 and nw.is_contiguous() and nw.numel() == K,
           f"the norm weight must be a contiguous bf16 [{K}] device tensor")


def _launch(a: kernels.GemvArgs, dev: torch.device, what: str) -> None:
    kernels.run_on(dev, lambda stream: kernels.check(kernels.load().bz_gemv(ctypes.byref(a), ctypes.c_void_p(stream)),
                                                     what))


def _args(x, y, epilogue) -> kernels.GemvArgs:
    a = kernels.GemvArgs()
    a.x, a.x_stride = x.data_ptr(), x.stride(0)
    a.y, a.y_stride = y.data_ptr(), y.stride(0)
    a.m, a.k = x.size(0), x.size(1)
    a.epilogue = epilogue
    return a


def gemv_seg(x: torch.Tensor, nw: torch.Tensor | None, eps: float, W0: torch.Tensor, W1: torch.Tensor,
             W2: torch.Tensor, y: torch.Tensor, R: int = 2, U: int = 1, warps: int = 8) -> torch.Tensor:
    """y[:, 0:N0+N1+N2] = norm?(x) @ [W0; W1; W2]^T (bb_fused.cu:293-317). W1 / W2 may be empty tensors; nw None
    skips the RMSNorm. Returns y. Under torch.compile the call is the registered operator torch.ops.bz.gemv_seg."""
    if torch.compiler.is_compiling():
        torch.ops.bz.gemv_seg(x, nw, float(eps), W0, W1, W2, y)
        return y
    return _gemv_seg(x, nw, eps, W0, W1, W2, y)


def _gemv_seg(x, nw, eps, W0, W1, W2, y) -> torch.Tensor:
    """gemv_seg's call through the C ABI (the body of the eager path and of torch.ops.bz.gemv_seg)."""
    M, K = _x2d(x)
    N0 = _w(W0, K, "W0")
    N1 = _w(W1, K, "W1") if W1 is not None and W1.numel() else 0
    N2 = _w(W2, K, "W2") if W2 is not None and W2.numel() else 0
    _y(y, M, N0 + N1 + N2)
    a = _args(x, y, kernels.GEMV_PLAIN)
    if nw is not None:
        _norm_w(nw, K)
        a.norm_weight, a.eps = nw.data_ptr(), float(eps)
    a.w[0], a.n[0] = W0.data_ptr(), N0
    if N1:
        a.w[1], a.n[1] = W1.data_ptr(), N1
    if N2:
        a.w[2], a.n[2] = W2.data_ptr(), N2
    _launch(a, x.device, "gemv_seg")
    return y


def gemv_resid(x: torch.Tensor, W: torch.Tensor, res: torch.Tensor, y: torch.Tensor, R: int = 2, U: int = 1,
               warps: int = 8) -> torch.Tensor:
    """y = res + x @ W^T with the GEMV rounded to bf16 before the add, as eager (bb_fused.cu:319-335). Returns y.
    Under torch.compile the call is the registered operator torch.ops.bz.gemv_resid."""
    if torch.compiler.is_compiling():
        torch.ops.bz.gemv_resid(x, W, res, y)
        return y
    return _gemv_resid(x, W, res, y)


def _gemv_resid(x, W, res, y) -> torch.Tensor:
    """gemv_resid's call through the C ABI."""
    M, K = _x2d(x)
    N = _w(W, K, "W")
    _y(res, M, N, "res")
    _y(y, M, N)
    a = _args(x, y, kernels.GEMV_RESIDUAL)
    a.w[0], a.n[0] = W.data_ptr(), N
    a.res, a.res_stride = res.data_ptr(), res.stride(0)
    _launch(a, x.device, "gemv_resid")
    return y


def gemv_gateup(x: torch.Tensor, nw: torch.Tensor, eps: float, Wg: torch.Tensor, Wu: torch.Tensor, y: torch.Tensor,
                R: int = 1, U: int = 1, warps: int = 8) -> torch.Tensor:
    """y = silu(norm(x) @ Wg^T) * (norm(x) @ Wu^T) at the eager rounding points (bb_fused.cu:337-356). Returns y.
    Under torch.compile the call is the registered operator torch.ops.bz.gemv_gateup."""
    if torch.compiler.is_compiling():
        torch.ops.bz.gemv_gateup(x, nw, float(eps), Wg, Wu, y)
        return y
    return _gemv_gateup(x, nw, eps, Wg, Wu, y)


def _gemv_gateup(x, nw, eps, Wg, Wu, y) -> torch.Tensor:
    """gemv_gateup's call through the C ABI."""
    M, K = _x2d(x)
    N = _w(Wg, K, "Wg")
    _check(_w(Wu, K, "Wu") == N, "Wg and Wu must have the same number of rows")
    _y(y, M, N)
    _norm_w(nw, K)
    a = _args(x, y, kernels.GEMV_SILU_MUL)
    a.norm_weight, a.eps = nw.data_ptr(), float(eps)
    a.w[0], a.w[1] = Wg.data_ptr(), Wu.data_ptr()
    a.n[0], a.n[1] = N, N
    _launch(a, x.device, "gemv_gateup")
    return y


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, y: torch.Tensor) -> torch.Tensor:
    """y = Qwen3RMSNorm(x) row by row (bb_fused.cu:358-368). Returns y. Under torch.compile the call is the registered
    operator torch.ops.bz.rmsnorm."""
    if torch.compiler.is_compiling():
        torch.ops.bz.rmsnorm(x, w, float(eps), y)
        return y
    return _rmsnorm(x, w, eps, y)


def _rmsnorm(x, w, eps, y) -> torch.Tensor:
    """rmsnorm's call through the C ABI."""
    _check(x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1,
           "x must be a bf16 [M, K] device tensor with a contiguous last dim")
    M, K = x.shape
    _norm_w(w, K)
    _y(y, M, K)
    kernels.run_on(x.device, lambda stream: kernels.check(kernels.load().bz_rmsnorm(
        x.data_ptr(), x.stride(0), w.data_ptr(), float(eps), y.data_ptr(), y.stride(0), M, K, ctypes.c_void_p(stream)),
        "rmsnorm"))
    return y
