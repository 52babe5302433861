"""Pins of the GEMV oracle (oracle.gemv): library routines (transformers' Qwen3RMSNorm, torch's bf16 F.linear and
F.silu on the CPU, which the eager chain of the reference's backbone runs), closed forms, invariants and planted
mistakes. bf16 results may differ from the library by one ulp where a different fp32 summation order moves a value
across a rounding boundary."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.gemv import gemv, rmsnorm

qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


def _t(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _bf16(rng, *shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def within_ulp(a, b, frac_exact=0.99):
    fa, fb = bf16_to_f32(a).astype(np.float64), bf16_to_f32(b).astype(np.float64)
    ok = np.abs(fa - fb) <= np.abs(fb) * 2.0 ** -7 + 1e-30
    return bool(ok.all() and (a == b).mean() >= frac_exact)


@pytest.mark.parametrize("K", [64, 2048])
def test_rmsnorm_matches_transformers(K):
    rng = np.random.default_rng(K)
    x, w = _bf16(rng, 4, K, scale=3.0), f32_to_bf16((1 + 0.3 * rng.standard_normal(K)).astype(np.float32))
    norm = qwen3.Qwen3RMSNorm(K, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(_t(w).float())
        ref = _bits(norm.to(torch.bfloat16)(_t(x)))
    assert within_ulp(rmsnorm(x, w, 1e-6), ref)


def test_plain_and_segments_match_torch_linear():
    rng = np.random.default_rng(1)
    x = _bf16(rng, 2, 512)
    W = [_bf16(rng, n, 512, scale=0.05) for n in (96, 32, 32)]
    ref = _bits(F.linear(_t(x), _t(np.concatenate(W))))
    assert within_ulp(gemv(x, W), ref)
    # segments are the rows of the concatenation
    parts = np.concatenate([gemv(x, [w]) for w in W], axis=1)
    assert np.array_equal(gemv(x, W), parts)


def test_prologue_residual_and_silu_match_torch():
    rng = np.random.default_rng(2)
    K, N = 256, 128
    x, nw = _bf16(rng, 2, K, scale=2.0), f32_to_bf16((1 + 0.2 * rng.standard_normal(K)).astype(np.float32))
    Wg, Wu, Wo = _bf16(rng, N, K, scale=0.06), _bf16(rng, N, K, scale=0.06), _bf16(rng, N, K, scale=0.06)
    res = _bf16(rng, 2, N)
    norm = qwen3.Qwen3RMSNorm(K, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(_t(nw).float())
        xn = norm.to(torch.bfloat16)(_t(x))
        act = F.silu(F.linear(xn, _t(Wg))) * F.linear(xn, _t(Wu))     # Qwen3MLP: act_fn(gate_proj(x)) * up_proj(x)
        resid = _t(res) + F.linear(_t(x), _t(Wo))                     # residual add after the bf16 linear
    assert within_ulp(gemv(x, [Wg, Wu], nw, 1e-5, epilogue="silu_mul"), _bits(act), 0.98)
    assert within_ulp(gemv(x, [Wo], epilogue="residual", res_bits=res), _bits(resid))


def test_closed_forms():
    rng = np.random.default_rng(3)
    x = _bf16(rng, 2, 64)
    eye = f32_to_bf16(np.eye(64, dtype=np.float32))
    zero = f32_to_bf16(np.zeros((64, 64), np.float32))
    res = _bf16(rng, 2, 64)
    assert np.array_equal(gemv(x, [eye]), x)                                      # identity weights
    assert np.array_equal(gemv(x, [zero], epilogue="residual", res_bits=res), res)  # zero weights: y = res
    assert (bf16_to_f32(gemv(x, [zero, eye], epilogue="silu_mul")) == 0).all()   # silu(0) * up = 0
    big = f32_to_bf16(np.full((2, 64), 40.0, np.float32))                        # silu(g) = g for large g
    assert np.array_equal(gemv(big, [eye, eye], epilogue="silu_mul"),
                          f32_to_bf16(np.full((2, 64), 1600.0, np.float32)))
    # RMSNorm is scale invariant at eps = 0 (a power of two scales every rounding point exactly)
    nw = f32_to_bf16((1 + 0.3 * rng.standard_normal(64)).astype(np.float32))
    assert np.array_equal(rmsnorm(f32_to_bf16(bf16_to_f32(x) * 8), nw, 0.0), rmsnorm(x, nw, 0.0))


def test_planted_mistakes_caught():
    rng = np.random.default_rng(4)
    K, N = 256, 128
    x = _bf16(rng, 2, K)
    W = _bf16(rng, N, K, scale=0.06)
    res = _bf16(rng, 2, N, scale=50.0)
    ref_resid = _bits(_t(res) + F.linear(_t(x), _t(W)))
    good = gemv(x, [W], epilogue="residual", res_bits=res)
    assert within_ulp(good, ref_resid)
    # the residual added to the unrounded fp32 product (no bf16 rounding of the GEMV first)
    acc = bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(W).astype(np.float64).T
    unrounded = f32_to_bf16((bf16_to_f32(res) + acc.astype(np.float32)).astype(np.float32))
    assert not np.array_equal(unrounded, ref_resid)
    # transposed weights
    Ws = _bf16(rng, K, K, scale=0.06)
    assert not within_ulp(gemv(x, [f32_to_bf16(bf16_to_f32(Ws).T.copy())]), _bits(F.linear(_t(x), _t(Ws))), 0.5)
    # silu applied after the product with up
    Wg, Wu = _bf16(rng, N, K, scale=0.06), _bf16(rng, N, K, scale=0.06)
    ref_act = _bits(F.silu(F.linear(_t(x), _t(Wg))) * F.linear(_t(x), _t(Wu)))
    wrong = _bits(F.silu(F.linear(_t(x), _t(Wg)) * F.linear(_t(x), _t(Wu))))
    assert within_ulp(gemv(x, [Wg, Wu], epilogue="silu_mul"), ref_act, 0.98)
    assert not within_ulp(wrong, ref_act, 0.5)
    # eps outside the square root of the RMSNorm
    nw = f32_to_bf16(np.ones(K, np.float32))
    xs = _bf16(rng, 2, K, scale=0.01)
    xf = bf16_to_f32(xs)
    bad = f32_to_bf16(bf16_to_f32(f32_to_bf16(xf / (np.sqrt((xf ** 2).mean(-1, keepdims=True)) + 0.5))))
    assert not within_ulp(bad, rmsnorm(xs, nw, 0.5), 0.5)
