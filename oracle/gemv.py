"""CPU restatement of the reference's backbone decode GEMVs (test infrastructure: only tests/, smoke() and bench.py's
cpu_baseline may use it; the product path never does).

flash/csrc/bb_fused.cu:1-7 states the semantics: y[m, n] = sum_k xin[m, k] * W[n, k] (nn.Linear layout, W [N, K],
fp32 accumulation in the reference, float64 here), with
  prologue: xin = x, or Qwen3RMSNorm(x) at the eager rounding points, bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))
            (bb_fused.cu:95-140, the same as transformers' Qwen3RMSNorm)
  epilogue: plain      y = bf16(acc)                                          (bb_fused.cu:198-199)
            residual   y = bf16(res + bf16(acc))                              (:200-201)
            silu_mul   y = bf16(bf16(silu(bf16(acc_gate))) * bf16(acc_up))    (:202-205, Qwen3MLP's act(gate) * up)
and the standalone row RMSNorm of the final norm (bb_fused.cu:219-248). All tensors are bf16 bit patterns (uint16).
"""
from __future__ import annotations

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16


def rmsnorm(x_bits, w_bits, eps: float):
    """Qwen3RMSNorm over the last dim at the eager rounding points: mean of squares and rsqrt in fp32 (as the eager
    chain computes them), h = bf16(x * rsqrt), y = bf16(w * h). Returns uint16 bits."""
    x = bf16_to_f32(x_bits).astype(np.float32)
    w = bf16_to_f32(w_bits).astype(np.float32)
    var = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    inv = (1.0 / np.sqrt(var.astype(np.float64) + np.float64(np.float32(eps)))).astype(np.float32)
    h = bf16_to_f32(f32_to_bf16(x * inv))
    return f32_to_bf16(w * h)


def gemv(x_bits, weights, norm_weight_bits=None, eps: float = 1e-6, epilogue: str = "plain", res_bits=None):
    """The fused GEMV of bb_fused.cu:55-216 for M rows of x [M, K].

    weights: a list of [N_i, K] bf16 bit arrays. plain / residual: the outputs are the rows of the concatenation
    (the q | k | v segments of gemv_seg, bb_fused.cu:293-317). silu_mul: exactly two matrices, gate and up.
    Returns y [M, N] as uint16 bits."""
    xin = x_bits if norm_weight_bits is None else rmsnorm(x_bits, norm_weight_bits, eps)
    xf = bf16_to_f32(xin).astype(np.float64)
    ws = [bf16_to_f32(w).astype(np.float64) for w in weights]
    if epilogue == "silu_mul":
        if len(ws) != 2:
            raise ValueError("silu_mul takes the gate and up matrices")
        g = bf16_to_f32(f32_to_bf16((xf @ ws[0].T).astype(np.float32))).astype(np.float32)
        u = bf16_to_f32(f32_to_bf16((xf @ ws[1].T).astype(np.float32))).astype(np.float32)
        act = bf16_to_f32(f32_to_bf16((g / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32)))
        return f32_to_bf16(act * u)
    acc = (xf @ np.concatenate(ws, axis=0).T).astype(np.float32)
    if epilogue == "plain":
        return f32_to_bf16(acc)
    if epilogue == "residual":
        r = bf16_to_f32(res_bits)
        return f32_to_bf16(r + bf16_to_f32(f32_to_bf16(acc)))
    raise ValueError(f"unknown epilogue {epilogue!r}")


def decoder_layer(x_bits, p: dict, cos_bits, sin_bits, k_cache_bits, v_cache_bits, cache_pos: int, seq_lens,
                  kv_start=None):
    """One Qwen3 decoder layer of the reference's fused decode step (flash/backbone.py:122-128):
    qkv = gemv(rmsnorm(x)) -> attn = fused_decode(qkv) -> h1 = x + o_proj(attn) -> act = silu(gate) * up of
    rmsnorm(h1) -> out = h1 + down(act). p holds bf16 bits: ln1, wq, wk, wv, qn, kn, wo, ln2, wg, wu, wd, plus
    eps (RMSNorm) and qk_eps, scale. Returns (out bits [M, H], updated K / V caches)."""
    from .attention import fused_decode

    M = x_bits.shape[0]
    qkv = gemv(x_bits, [p["wq"], p["wk"], p["wv"]], p["ln1"], p["eps"])
    attn, k2, v2 = fused_decode(qkv, p["qn"], p["kn"], p["qk_eps"], cos_bits, sin_bits, k_cache_bits, v_cache_bits,
                                cache_pos, seq_lens, p["scale"], kv_start=kv_start)
    ao = f32_to_bf16(attn.astype(np.float32)).reshape(M, -1)
    h1 = gemv(ao, [p["wo"]], epilogue="residual", res_bits=x_bits)
    act = gemv(h1, [p["wg"], p["wu"]], p["ln2"], p["eps"], epilogue="silu_mul")
    out = gemv(act, [p["wd"]], epilogue="residual", res_bits=h1)
    return out, k2, v2
