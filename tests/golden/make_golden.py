"""Write the golden fixtures of the decode-attention path (tests/golden/decode_attention.npz).

The reference ships no test vectors for this path (its repository has no tests or fixtures), so these fixtures are
the CPU oracle's outputs (oracle.attention.decode_attention, float64) on small seeded inputs, pinned independently by
tests/test_oracle.py. They freeze the oracle's results so that a later change to it is caught, and they give the GPU
tests inputs whose expected outputs need no recomputation.

Cases (q [B, NH, D], K/V [B, NKV, cap, D] stored as bf16 bit patterns in uint16; outputs float32):
  backbone   B2, 16 q / 8 KV heads (G 2), D128, cap 24, lens [24, 17], starts [0, 5]
  depth      B2, 8 q / 2 KV heads (G 4), D128, cap 16, lens [2, 16]  (the reference's depth shape)
  d64        B2, 16 q / 8 KV heads, D64, cap 32, lens [1, 32]
  masked     B2, 16 q / 8 KV heads, D128, cap 24, bf16 interval mask (pad_lens [0, 5], position 18) plus a finite
             bias and one excluded hole; K/V NaN outside [pad, position]
A second file, tests/golden/fused_and_tokens.npz, holds the fused decode step (oracle.attention.fused_decode: raw
q | k | v projections, Qwen3 q/k RMSNorm + RoPE at the eager bf16 rounding points, new k / v written at cache_pos,
attention over the updated cache) and several query tokens per row (oracle.attention.decode_attention_tokens):
  fused_backbone  B2, 16 q / 8 KV heads, D128, cap 24, slot 17, lens [18, 18], starts [0, 4]
  fused_depth     B2, 8 q / 2 KV heads, D128, cap 16, slot 7, lens [8, 8]
  tokens_depth    B2, 8 q / 2 KV heads, D128, cap 16, two tokens at positions 0 and 1 (the depth first step)
  tokens_backbone B2, 16 q / 8 KV heads, D128, cap 24, three tokens, lens [24, 17], starts [0, 6]
Usage: python tests/golden/make_golden.py   (from the repository root)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.attention import (decode_attention, decode_attention_tokens, fused_decode, interval_mask,  # noqa: E402
                              rope_cos_sin)
from oracle.bf16 import bf16_to_f32, f32_to_bf16  # noqa: E402

OUT = HERE / "decode_attention.npz"
OUT2 = HERE / "fused_and_tokens.npz"


def _bf16(rng, *shape):
    return f32_to_bf16(rng.standard_normal(shape).astype(np.float32))


def case(rng, B, NH, NKV, D, cap, lens, starts):
    q, k, v = _bf16(rng, B, NH, D), _bf16(rng, B, NKV, cap, D), _bf16(rng, B, NKV, cap, D)
    lens = np.asarray(lens, np.int32)
    starts = np.asarray(starts, np.int32)
    out = decode_attention(bf16_to_f32(q), bf16_to_f32(k), bf16_to_f32(v), lens, D ** -0.5, kv_start=starts)
    return dict(q=q, k=k, v=v, lens=lens, starts=starts, scale=np.float32(D ** -0.5), out=out.astype(np.float32))


def main():
    rng = np.random.default_rng(20261201)
    cases = {
        "backbone": case(rng, 2, 16, 8, 128, 24, [24, 17], [0, 5]),
        "depth": case(rng, 2, 8, 2, 128, 16, [2, 16], [0, 0]),
        "d64": case(rng, 2, 16, 8, 64, 32, [1, 32], [0, 0]),
    }
    # masked: the reference's interval mask, plus a finite bias and one hole, with NaN K/V outside the interval
    B, NH, NKV, D, cap = 2, 16, 8, 128, 24
    q, k, v = _bf16(rng, B, NH, D), _bf16(rng, B, NKV, cap, D), _bf16(rng, B, NKV, cap, D)
    pad, position = [0, 5], 18
    mask = interval_mask(pad, position, cap).float().numpy().reshape(B, cap)
    bias = (rng.standard_normal((B, cap)) * 0.5).astype(np.float32)
    mask = np.where(mask > -1e30, mask + bias, mask)
    mask[1, 9] = np.float32(-3.3895314e38)  # a hole inside row 1's interval
    mask_bits = f32_to_bf16(mask)
    nan = f32_to_bf16(np.array([np.nan], np.float32))[0]
    for b in range(B):
        for pos in range(cap):
            if not (pad[b] <= pos <= position) or (b == 1 and pos == 9):
                k[b, :, pos] = nan
                v[b, :, pos] = nan
    out = decode_attention(bf16_to_f32(q), bf16_to_f32(k), bf16_to_f32(v), np.full(B, cap, np.int32), D ** -0.5,
                           mask=bf16_to_f32(mask_bits))
    cases["masked"] = dict(q=q, k=k, v=v, lens=np.full(B, cap, np.int32), starts=np.zeros(B, np.int32),
                           scale=np.float32(D ** -0.5), mask=mask_bits, out=out.astype(np.float32))
    flat = {f"{name}/{key}": val for name, c in cases.items() for key, val in c.items()}
    np.savez_compressed(OUT, **flat)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, cases: {', '.join(cases)})")

    rng2 = np.random.default_rng(20261202)
    cases2 = {
        "fused_backbone": fused_case(rng2, 2, 16, 8, 24, 17, [18, 18], [0, 4]),
        "fused_depth": fused_case(rng2, 2, 8, 2, 16, 7, [8, 8], [0, 0]),
        "tokens_depth": tokens_case(rng2, 2, 8, 2, 128, 16, 2, [2, 2], [0, 0]),
        "tokens_backbone": tokens_case(rng2, 2, 16, 8, 128, 24, 3, [24, 17], [0, 6]),
    }
    flat = {f"{name}/{key}": val for name, c in cases2.items() for key, val in c.items()}
    np.savez_compressed(OUT2, **flat)
    print(f"wrote {OUT2} ({OUT2.stat().st_size} bytes, cases: {', '.join(cases2)})")


def fused_case(rng, B, NH, NKV, cap, pos, lens, starts, D=128):
    qkv = f32_to_bf16((rng.standard_normal((B, (NH + 2 * NKV) * D)) * 2).astype(np.float32))
    qn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    kn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    cos, sin = (f32_to_bf16(t) for t in rope_cos_sin([pos] * B, D))
    k, v = _bf16(rng, B, NKV, cap, D), _bf16(rng, B, NKV, cap, D)
    lens, starts = np.asarray(lens, np.int32), np.asarray(starts, np.int32)
    out, k2, v2 = fused_decode(qkv, qn, kn, 1e-6, cos, sin, k, v, pos, lens, D ** -0.5, kv_start=starts)
    return dict(qkv=qkv, qn=qn, kn=kn, eps=np.float32(1e-6), cos=cos, sin=sin, k=k, v=v, pos=np.int64(pos), lens=lens,
                starts=starts, scale=np.float32(D ** -0.5), out=out.astype(np.float32), k_slot=k2[:, :, pos],
                v_slot=v2[:, :, pos])


def tokens_case(rng, B, NH, NKV, D, cap, T, lens, starts):
    q, k, v = _bf16(rng, B, NH, T, D), _bf16(rng, B, NKV, cap, D), _bf16(rng, B, NKV, cap, D)
    lens, starts = np.asarray(lens, np.int32), np.asarray(starts, np.int32)
    out = decode_attention_tokens(bf16_to_f32(q), bf16_to_f32(k), bf16_to_f32(v), lens, D ** -0.5, kv_start=starts)
    return dict(q=q, k=k, v=v, lens=lens, starts=starts, scale=np.float32(D ** -0.5), out=out.astype(np.float32))


def load(path: Path = OUT) -> dict:
    """{case: {field: array}} from a committed fixture file (default: the decode-attention cases)."""
    data = np.load(path, allow_pickle=False)
    cases: dict = {}
    for key in data.files:
        name, field = key.split("/", 1)
        cases.setdefault(name, {})[field] = data[key]
    return cases


if __name__ == "__main__":
    main()
