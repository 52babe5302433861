"""The library's entry points as torch operators (namespace "bz"), so that torch.compile treats each call as one
opaque graph node instead of breaking the graph at the ctypes call. The reference's ops are torch operators through its
pybind extension (flash/csrc/bb_attn.cu:462-469, bb_fused.cu:370-377); here the C ABI stays the boundary and each
operator's implementation is the package function's own call through it.

Each operator writes its outputs in place (declared as mutable arguments in its schema) and returns nothing; the fake
implementations (shapes only) do nothing, as the outputs are the caller's tensors. Workspaces follow the package
functions: without one, a call takes its stream's cached workspace (allocated, when first needed, outside any graph
memory pool), except while the stream is being captured, as when torch.compile's CUDA-graph trees record a graph:
bz::gqa_decode and bz::gqa_decode_masked then run on the library's static scratch (bz_gqa_decode_noalloc) and
bz::gqa_decode_fused raises unless it is given a workspace made beforehand. So compiled calls on different streams
never share a workspace. The package functions (attention.gqa_decode and the rest) call these operators while
torch.compile traces them and call the C ABI directly otherwise, which keeps the eager per-call host cost of a plain
function call.

The operators are defined with torch.library.Library (a schema, a CUDA kernel and a fake kernel each) rather than the
torch.library.custom_op decorator: an eager call then goes through the dispatcher straight to the kernel, without the
decorator's Python wrapper layers (a do-nothing operator measured 3.8 µs per call against 19.3 through custom_op on
the build host).
"""
from __future__ import annotations

import torch

from . import attention, gemv

_LIB = torch.library.Library("bz", "DEF")  # kept alive for the process: dropping it would unregister the ops

_SCHEMAS = {
    "gqa_decode": "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor seq_lens, float scale, Tensor(a!) out, "
                  "Tensor? kv_start, Tensor? mask, SymInt num_splits, SymInt max_seq_len, SymInt combine, "
                  "Tensor(b!)? workspace) -> ()",
    "gqa_decode_wave": "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor seq_lens, float scale, Tensor(a!) out, "
                       "Tensor? kv_start) -> ()",
    "gqa_decode_masked": "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor mask, float scale, Tensor(a!) out, "
                         "SymInt num_splits, SymInt max_seq_len, SymInt combine, Tensor(b!)? workspace) -> ()",
    "gqa_decode_fused": "(Tensor qkv, Tensor q_norm_weight, Tensor k_norm_weight, float eps, Tensor cos, Tensor sin, "
                        "Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor cache_pos, float scale, Tensor(c!) out, "
                        "Tensor? seq_lens, Tensor? kv_start, Tensor? mask, SymInt num_splits, SymInt max_seq_len, "
                        "SymInt combine, Tensor(d!)? workspace) -> ()",
    "gqa_decode_probs": "(Tensor q, Tensor k_cache, Tensor? seq_lens, float scale, Tensor(a!) probs, Tensor? kv_start, "
                        "Tensor? mask) -> ()",
    "gemv_seg": "(Tensor x, Tensor? nw, float eps, Tensor W0, Tensor? W1, Tensor? W2, Tensor(a!) y) -> ()",
    "gemv_resid": "(Tensor x, Tensor W, Tensor res, Tensor(a!) y) -> ()",
    "gemv_gateup": "(Tensor x, Tensor nw, float eps, Tensor Wg, Tensor Wu, Tensor(a!) y) -> ()",
    "rmsnorm": "(Tensor x, Tensor w, float eps, Tensor(a!) y) -> ()",
}


def _gqa_decode(q, k_cache, v_cache, seq_lens, scale, out, kv_start, mask, num_splits, max_seq_len, combine,
                workspace):
    attention._gqa_decode(q, k_cache, v_cache, seq_lens, scale, out, kv_start, mask, num_splits, max_seq_len, combine,
                          workspace)


def _gqa_decode_wave(q, k_cache, v_cache, seq_lens, scale, out, kv_start):
    attention._gqa_decode_wave(q, k_cache, v_cache, seq_lens, scale, out, kv_start)


def _gqa_decode_masked(q, k_cache, v_cache, mask, scale, out, num_splits, max_seq_len, combine, workspace):
    attention._gqa_decode_masked(q, k_cache, v_cache, mask, scale, out, num_splits, max_seq_len, combine, workspace)


def _gqa_decode_fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale, out,
                      seq_lens, kv_start, mask, num_splits, max_seq_len, combine, workspace):
    attention._gqa_decode_fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale,
                                out, seq_lens, kv_start, mask, num_splits, max_seq_len, combine, workspace)


def _gqa_decode_probs(q, k_cache, seq_lens, scale, probs, kv_start, mask):
    attention._gqa_decode_probs(q, k_cache, seq_lens, scale, probs, kv_start, mask)


# the GEMV bodies return their output tensor; an operator whose schema returns () must return None
def _gemv_seg(x, nw, eps, W0, W1, W2, y):
    gemv._gemv_seg(x, nw, eps, W0, W1, W2, y)


def _gemv_resid(x, W, res, y):
    gemv._gemv_resid(x, W, res, y)


def _gemv_gateup(x, nw, eps, Wg, Wu, y):
    gemv._gemv_gateup(x, nw, eps, Wg, Wu, y)


def _rmsnorm(x, w, eps, y):
    gemv._rmsnorm(x, w, eps, y)


_KERNELS = {
    "gqa_decode": _gqa_decode,
    "gqa_decode_wave": _gqa_decode_wave,
    "gqa_decode_masked": _gqa_decode_masked,
    "gqa_decode_fused": _gqa_decode_fused,
    "gqa_decode_probs": _gqa_decode_probs,
    "gemv_seg": _gemv_seg,
    "gemv_resid": _gemv_resid,
    "gemv_gateup": _gemv_gateup,
    "rmsnorm": _rmsnorm,
}


def _fake(*args, **kwargs):
    """Fake (meta) kernel of every operator: the outputs are caller tensors written in place, so there is nothing to
    allocate or return."""
    return None


for _name, _schema in _SCHEMAS.items():
    _LIB.define(_name + _schema)
    _LIB.impl(_name, _KERNELS[_name], "CUDA")
    torch.library.register_fake("bz::" + _name, _fake, lib=_LIB)
