"""Pins of the fused-prologue oracle (oracle.attention.qk_norm_rope / fused_decode): transformers' own Qwen3RMSNorm
and apply_rotary_pos_emb in bf16 on the CPU (the library code the reference's backbone layers run), closed forms,
and planted mistakes."""
import numpy as np
import pytest
import torch

from oracle.attention import decode_attention, fused_decode, qk_norm_rope, rope_cos_sin
from oracle.bf16 import bf16_to_f32, f32_to_bf16

qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _t(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _inputs(seed, n=24, D=128):
    rng = np.random.default_rng(seed)
    x = f32_to_bf16((rng.standard_normal((n, D)) * rng.uniform(0.2, 30)).astype(np.float32))
    w = f32_to_bf16((1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32))
    cos, sin = rope_cos_sin(rng.integers(0, 4096, n), D)
    return x, w, f32_to_bf16(cos), f32_to_bf16(sin)


def _transformers(x, w, eps, cos, sin):
    D = x.shape[-1]
    norm = qwen3.Qwen3RMSNorm(D, eps=eps)
    with torch.no_grad():
        norm.weight.copy_(_t(w).float())
    norm = norm.to(torch.bfloat16)
    xt = _t(x)[:, None, None, :]                       # [n, heads=1, seq=1, D]
    with torch.no_grad():
        y = norm(xt)
        q_embed, _ = qwen3.apply_rotary_pos_emb(y, y, _t(cos)[:, None, :], _t(sin)[:, None, :])
    return _bits(q_embed.reshape(-1, D))


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
@pytest.mark.parametrize("D", [64, 128])
def test_matches_transformers_qwen3(seed, D):
    x, w, cos, sin = _inputs(seed, D=D)
    ours = qk_norm_rope(x, w, 1e-6, cos, sin)
    theirs = _transformers(x, w, 1e-6, cos, sin)
    diff = np.abs(bf16_to_f32(ours).astype(np.float64) - bf16_to_f32(theirs))
    ulp = np.abs(bf16_to_f32(theirs)) * 2.0 ** -7 + 1e-30
    # identical except where the fp32 mean's summation order moves a value across a bf16 rounding boundary
    assert (diff <= ulp).all()
    assert (ours == theirs).mean() > 0.995


def test_closed_forms():
    x, w, cos, sin = _inputs(7)
    one = f32_to_bf16(np.ones(128, np.float32))
    zero = f32_to_bf16(np.zeros(128, np.float32))
    xf = bf16_to_f32(x).astype(np.float64)
    rms = np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6)
    # w = 1, cos = 1, sin = 0: plain RMSNorm
    y = bf16_to_f32(qk_norm_rope(x, one, 1e-6, one, zero))
    assert np.allclose(y, xf / rms, rtol=2 ** -7, atol=0)
    # cos = 0, sin = 1: rotate_half of the normed vector
    r = bf16_to_f32(qk_norm_rope(x, one, 1e-6, zero, one))
    assert np.array_equal(r, np.concatenate([-y[:, 64:], y[:, :64]], axis=-1))
    # scale invariance of RMSNorm (up to eps): x * 4 gives the same output
    x4 = f32_to_bf16(bf16_to_f32(x) * 4)
    assert np.array_equal(qk_norm_rope(x4, w, 0.0, cos, sin), qk_norm_rope(x, w, 0.0, cos, sin))


def test_planted_mistakes_caught():
    x, w, cos, sin = _inputs(9)
    ref = _transformers(x, w, 1e-6, cos, sin)
    close = lambda a: (np.abs(bf16_to_f32(a) - bf16_to_f32(ref)) <= np.abs(bf16_to_f32(ref)) * 2 ** -7 + 1e-30).all()  # noqa: E731
    assert close(qk_norm_rope(x, w, 1e-6, cos, sin))
    neg_sin = f32_to_bf16(-bf16_to_f32(sin))
    assert not close(qk_norm_rope(x, w, 1e-6, cos, neg_sin))              # rotate_half with the sign flipped
    assert not close(qk_norm_rope(x, f32_to_bf16(np.ones(128, np.float32)), 1e-6, cos, sin))   # weight dropped
    assert not close(qk_norm_rope(x, w, 1e-6, sin, cos))                  # cos / sin swapped


def test_fused_decode_writes_slot_and_attends():
    rng = np.random.default_rng(11)
    B, NH, NKV, D, cap = 2, 16, 8, 128, 40
    qkv = f32_to_bf16(rng.standard_normal((B, (NH + 2 * NKV) * D)).astype(np.float32))
    qn, kn = (f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32)) for _ in range(2))
    cos, sin = (f32_to_bf16(a) for a in rope_cos_sin([29, 29], D))
    kc = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))
    vc = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))
    pos = 29
    out, k2, v2 = fused_decode(qkv, qn, kn, 1e-6, cos, sin, kc, vc, pos, np.full(B, pos + 1), D ** -0.5)
    heads = qkv.reshape(B, NH + 2 * NKV, D)
    assert np.array_equal(v2[:, :, pos], heads[:, NH + NKV:])
    assert np.array_equal(k2[:, :, pos], qk_norm_rope(heads[:, NH:NH + NKV], kn, 1e-6, cos[:, None], sin[:, None]))
    untouched = np.ones(cap, bool)
    untouched[pos] = False
    assert np.array_equal(k2[:, :, untouched], kc[:, :, untouched]) and np.array_equal(v2[:, :, untouched], vc[:, :, untouched])
    q = qk_norm_rope(heads[:, :NH], qn, 1e-6, cos[:, None], sin[:, None])
    ref = decode_attention(bf16_to_f32(q), bf16_to_f32(k2), bf16_to_f32(v2), np.full(B, pos + 1), D ** -0.5)
    assert np.array_equal(out, ref)
    # a slot outside the cache writes nothing
    _, k3, v3 = fused_decode(qkv, qn, kn, 1e-6, cos, sin, kc, vc, cap, np.full(B, cap), D ** -0.5)
    assert np.array_equal(k3, kc) and np.array_equal(v3, vc)
