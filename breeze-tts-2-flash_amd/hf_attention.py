"""The MI355X decode attention as a transformers attention implementation, for q_len == 1 steps.

Follows the reference's own pattern for swapping the attention of its Qwen3 layers (flash/prefill_attn.py:27-46:
AttentionInterface.register of a function with the eager signature, selected through config._attn_implementation).
The function receives what transformers' eager attention receives (modeling_qwen3.Qwen3Attention.forward): query
[B, NH, q_len, D] after q_norm and RoPE, key / value [B, NKV, kv_len, D] (the whole StaticCache layer, or the
DynamicCache so far) with the new token already written, the 4D additive mask, and module.scaling. It returns
(attn_output [B, q_len, NH, D], None), as eager_attention_forward does (models/breeze.py:259-286).

Routing:
  - q_len == 1, bf16 CUDA tensors, head_dim 64 / 128, group size 1 / 2 / 4 / 8, no dropout: bz_gqa_decode_masked (the
    range of each row comes from the mask on the device, left padding included) or, with no mask, bz_gqa_decode over
    the whole key length. A missing or broken library raises; there is no silent fallback for these calls.
  - anything else (prefill, other dtypes or shapes, CPU tensors): eager attention. CPU tensors get the model's own
    eager function, exactly as without this module; GPU tensors get eager_attention below, the same rounding points
    with every operand of the batched products made contiguous (a bf16 batched product whose right operand is a
    transposed view, as in the eager function's q @ k^T, is kept off the GPU). calls["hip"] / calls["eager"] count
    the two routes.

The mask: transformers builds no mask for attention implementations it does not know, so install() also registers
transformers' eager mask builder under the same name; the function then gets the eager [B, 1, q_len, kv_len] mask
(0 on attended positions, finfo(dtype).min elsewhere), whose excluded value the kernel's threshold (<= -1e30,
flash/csrc/bb_attn.cu:9-11) recognises in bf16 and fp32.
"""
from __future__ import annotations

import sys

import torch

from . import kernels
from .attention import gqa_decode, gqa_decode_masked

NAME = "mi355_decode"
EAGER_NAME = "mi355_eager"   # eager_attention alone, for reference runs of a model on the GPU
calls = {"hip": 0, "eager": 0}

_SUPPORTED_D = (64, 128)
_SUPPORTED_G = (1, 2, 4, 8)


def eager_attention(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                    attention_mask: torch.Tensor | None, scaling: float | None = None, dropout: float = 0.0,
                    **kwargs):
    """Eager attention at the rounding points of transformers' eager_attention_forward (modeling_qwen3): KV heads
    repeated for their group (q head h reads KV head h // G), scores = (q @ k^T in the input dtype) * scaling, plus the
    additive mask, softmax in fp32 rounded back to the input dtype, then @ v. Both products take contiguous operands.
    Returns (attn_output [B, q_len, NH, D], weights)."""
    G = query.size(1) // key.size(1)
    k = key.repeat_interleave(G, dim=1) if G > 1 else key
    v = value.repeat_interleave(G, dim=1) if G > 1 else value
    if scaling is None:
        scaling = query.size(-1) ** -0.5
    w = torch.matmul(query.contiguous(), k.transpose(2, 3).contiguous()) * scaling
    if attention_mask is not None:
        w = w + attention_mask[:, :, :, :k.size(2)]
    w = torch.softmax(w, dim=-1, dtype=torch.float32).to(query.dtype)
    w = torch.nn.functional.dropout(w, p=dropout, training=module.training)
    out = torch.matmul(w, v.contiguous())
    return out.transpose(1, 2).contiguous(), w


def _eager(module, query):
    """GPU tensors: eager_attention. CPU tensors: the eager attention of the module's own model file (Qwen3:
    modeling_qwen3.eager_attention_forward), else transformers' SDPA forward, which takes the same additive mask."""
    if query.is_cuda:
        return eager_attention
    fn = getattr(sys.modules.get(type(module).__module__), "eager_attention_forward", None)
    if fn is None:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward as fn
    return fn


def _hip_route(module, query, key, value, attention_mask, dropout) -> bool:
    if query.dim() != 4 or query.size(2) != 1 or key.dim() != 4:
        return False
    if not (query.is_cuda and key.is_cuda and value.is_cuda):
        return False
    if kernels.device_unsupported(query.device.index) is not None:
        return False
    if query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        return False
    if dropout and module.training:
        return False
    B, NH, _, D = query.shape
    NKV = key.size(1)
    if D not in _SUPPORTED_D or NH % NKV or NH // NKV not in _SUPPORTED_G:
        return False
    if key.stride(3) != 1 or key.stride() != value.stride() or key.shape != value.shape:
        return False
    if attention_mask is not None:
        if attention_mask.dim() != 4 or attention_mask.dtype not in (torch.bfloat16, torch.float32):
            return False
        if attention_mask.size(-1) < key.size(2) or attention_mask.stride(-1) != 1:
            return False
    return True


def mi355_decode_attention(module, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                           attention_mask: torch.Tensor | None, scaling: float | None = None, dropout: float = 0.0,
                           **kwargs):
    """Attention with the eager signature; q_len == 1 runs the gfx950 split-K kernel (see the module docstring)."""
    if not _hip_route(module, query, key, value, attention_mask, dropout):
        calls["eager"] += 1
        return _eager(module, query)(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout,
                                     **kwargs)
    calls["hip"] += 1
    B, NH, _, D = query.shape
    if scaling is None:
        scaling = D ** -0.5
    out = torch.empty(B, 1, NH, D, dtype=torch.bfloat16, device=query.device)
    if attention_mask is None:
        lens = torch.full((B,), key.size(2), dtype=torch.int32, device=query.device)
        gqa_decode(query, key, value, lens, scaling, out)
    else:
        # the query row's mask ([B, 1, 1, S] at decode already: no slicing view to build)
        mask = attention_mask if attention_mask.size(2) == 1 else attention_mask[:, :, -1:, :]
        gqa_decode_masked(query, key, value, mask, scaling, out)
    return out, None


def install() -> str:
    """Register the attention function and the eager mask builder under NAME, and eager_attention under EAGER_NAME
    (idempotent). Returns NAME: pass it as attn_implementation (from_pretrained / from_config) or set it on a config,
    as the reference does with its own implementation (flash/prefill_attn.py:41-46). A visible GPU other than gfx950
    declines: nothing is registered, the reason is printed and "eager" (transformers' own attention) is returned, as
    the reference's pre-flight keeps the official path (flash/support.py:67-84). Calls on such a device that reach
    mi355_decode_attention anyway go to eager attention."""
    import torch
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, eager_mask

    if torch.cuda.is_available():
        reason = kernels.device_unsupported()
        if reason is not None:
            print(f"[breeze_tts_2_flash_amd] {NAME} attention not installed: {reason}", flush=True)
            return "eager"

    AttentionInterface.register(NAME, mi355_decode_attention)
    ALL_MASK_ATTENTION_FUNCTIONS.register(NAME, eager_mask)
    AttentionInterface.register(EAGER_NAME, eager_attention)
    ALL_MASK_ATTENTION_FUNCTIONS.register(EAGER_NAME, eager_mask)
    return NAME
