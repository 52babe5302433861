"""Pins of the CPU oracle (oracle/): library routines, brute force, closed forms, invariants, planted mistakes.

Every check below is written as a function of an attention implementation so that it can also be run against
deliberately broken variants of the oracle (planted mistakes, on the CPU): each variant must fail at least one check.
"""
import math

import numpy as np
import pytest
import torch

from oracle.attention import decode_attention, eager_bf16, interval_mask, mask_interval, sdpa_fp32
from oracle.bf16 import bf16_to_f32, f32_to_bf16, round_to_bf16


def _bf16_vals(rng, *shape, scale=1.0):
    return round_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


# ---------------------------------------------------------------------------------------------- bf16

def test_bf16_round_trip_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.4e38, -3.4e38, 1e-40, -1e-40,
                  2 ** -133, 1.00390625, 1.01171875], dtype=np.float32),  # ties to even both ways, denormals
    ]).astype(np.float32)
    ours = f32_to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    back = bf16_to_f32(ours)
    assert np.array_equal(back, torch.from_numpy(ours.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_bf16_nan_stays_nan():
    x = np.array([np.nan, -np.nan], dtype=np.float32)
    assert np.isnan(bf16_to_f32(f32_to_bf16(x))).all()


# ---------------------------------------------------------------------------------------------- checks

def _case(seed, B=3, NH=8, NKV=2, D=64, cap=40, lens=None, starts=None):
    rng = np.random.default_rng(seed)
    q = _bf16_vals(rng, B, NH, D)
    k = _bf16_vals(rng, B, NKV, cap, D)
    v = _bf16_vals(rng, B, NKV, cap, D)
    lens = np.array(lens if lens is not None else rng.integers(1, cap + 1, B), dtype=np.int32)
    starts = None if starts is None else np.array(starts, dtype=np.int32)
    return q, k, v, lens, starts, D ** -0.5


def check_vs_sdpa(impl):
    for seed, NKV, D, starts in ((1, 2, 64, None), (2, 8, 128, None), (3, 4, 64, [0, 3, 7]), (4, 1, 128, [5, 0, 0])):
        q, k, v, lens, st, scale = _case(seed, NKV=NKV, D=D, starts=starts)
        ref = sdpa_fp32(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), lens, scale, st).numpy()
        got = impl(q, k, v, lens, scale, st)
        if not np.allclose(got, ref, atol=2e-6, rtol=2e-5):
            return False
    return True


def _brute(q, k, v, lens, scale, starts=None, mask=None):
    """Pure-Python float64 loops, written independently of the oracle's vectorised form."""
    B, NH, D = q.shape
    NKV = k.shape[1]
    G = NH // NKV
    out = np.zeros((B, NH, D))
    for b in range(B):
        lo = 0 if starts is None else int(starts[b])
        hi = int(lens[b])
        for h in range(NH):
            kvh = h // G
            scores = []
            for p in range(lo, hi):
                mv = 0.0 if mask is None else float(mask[b if mask.shape[0] > 1 else 0][p])
                if mv <= -1e30:
                    continue
                dot = sum(float(q[b, h, d]) * float(k[b, kvh, p, d]) for d in range(D))
                scores.append((p, dot * scale + mv))
            if not scores:
                continue
            mx = max(s for _, s in scores)
            den = sum(math.exp(s - mx) for _, s in scores)
            for d in range(D):
                out[b, h, d] = sum(math.exp(s - mx) / den * float(v[b, kvh, p, d]) for p, s in scores)
    return out


def check_vs_brute(impl):
    rng = np.random.default_rng(7)
    B, NH, NKV, D, cap = 2, 4, 2, 3, 7
    q, k, v = _bf16_vals(rng, B, NH, D), _bf16_vals(rng, B, NKV, cap, D), _bf16_vals(rng, B, NKV, cap, D)
    lens, starts = np.array([5, 7], np.int32), np.array([1, 0], np.int32)
    ok = np.allclose(impl(q, k, v, lens, 0.7, starts), _brute(q, k, v, lens, 0.7, starts), atol=1e-12)
    mask = rng.standard_normal((B, cap)) * 0.5
    mask[0, 2] = -3.0e38
    mask[1, 6] = -1e31
    got = impl(q, k, v, lens, 0.7, starts, mask=mask)
    return ok and np.allclose(got, _brute(q, k, v, lens, 0.7, starts, mask=mask), atol=1e-12)


def check_closed_forms(impl):
    rng = np.random.default_rng(11)
    B, NH, NKV, D, cap = 2, 8, 4, 64, 50
    q, k, v = _bf16_vals(rng, B, NH, D), _bf16_vals(rng, B, NKV, cap, D), _bf16_vals(rng, B, NKV, cap, D)
    G = NH // NKV
    heads = np.arange(NH) // G
    # one position -> that position's V row, exactly
    starts, lens = np.array([3, 17], np.int32), np.array([4, 18], np.int32)
    out = impl(q, k, v, lens, 0.125, starts)
    for b in range(B):
        if not np.array_equal(out[b], v[b, heads, starts[b]]):
            return False
    # q = 0 (and, separately, scale = 0) -> uniform weights -> mean of V over [start, end)
    starts, lens = np.array([5, 0], np.int32), np.array([37, 50], np.int32)
    for qq, sc in ((np.zeros_like(q), 0.125), (q, 0.0)):
        out = impl(qq, k, v, lens, sc, starts)
        for b in range(B):
            mean = v[b, :, starts[b]:lens[b]].astype(np.float64).mean(axis=1)[heads]
            if not np.allclose(out[b], mean, atol=1e-12):
                return False
    # one dominant key (score gap >= 30 nats) -> its V row
    kd = k.copy()
    p_star = 21
    for kvh in range(NKV):
        for b in range(B):
            qdir = q[b, kvh * G:(kvh + 1) * G].sum(axis=0)
            kd[b, kvh, p_star] = 200.0 * qdir / np.linalg.norm(qdir)
    out = impl(q, kd, v, np.array([50, 50], np.int32), 1.0, None)
    return np.allclose(out, v[:, heads, p_star], atol=1e-6)


def check_invariants(impl):
    q, k, v, lens, _, scale = _case(21, B=3, NH=8, NKV=2, D=64, cap=40, lens=[13, 40, 1])
    base = impl(q, k, v, lens, scale, None)
    # GQA == MHA on repeat_kv-expanded K/V
    G = q.shape[1] // k.shape[1]
    ke, ve = np.repeat(k, G, axis=1), np.repeat(v, G, axis=1)
    if not np.allclose(impl(q, ke, ve, lens, scale, None), base, atol=1e-12):
        return False
    # NaN / Inf outside [start, end) never reaches the output
    kn, vn = k.copy(), v.copy()
    for b, L in enumerate(lens):
        kn[b, :, L:] = np.nan
        vn[b, :, L:] = np.inf
    if not np.array_equal(impl(q, kn, vn, lens, scale, None), base):
        return False
    # rows are independent
    q2 = q.copy()
    q2[1] = -q2[1]
    o2 = impl(q2, k, v, lens, scale, None)
    return np.array_equal(o2[0], base[0]) and np.array_equal(o2[2], base[2]) and not np.allclose(o2[1], base[1])


CHECKS = [check_vs_sdpa, check_vs_brute, check_closed_forms, check_invariants]


def _oracle(q, k, v, lens, scale, starts, mask=None):
    return decode_attention(q, k, v, lens, scale, kv_start=starts, mask=mask)


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes(check):
    assert check(_oracle)


# ---------------------------------------------------------------------------------------------- planted mistakes

def _mutant_head_map(q, k, v, lens, scale, starts, mask=None):
    # q head h reads KV head h % NKV instead of h // G
    NH, NKV = q.shape[1], k.shape[1]
    idx = np.arange(NH) % NKV
    return decode_attention(q, k[:, idx], v[:, idx], lens, scale, kv_start=starts, mask=mask)


def _mutant_off_by_one(q, k, v, lens, scale, starts, mask=None):
    # range end treated as inclusive
    cap = k.shape[2]
    return decode_attention(q, k, v, np.minimum(np.asarray(lens) + 1, cap), scale, kv_start=starts, mask=mask)


def _mutant_no_scale(q, k, v, lens, scale, starts, mask=None):
    return decode_attention(q, k, v, lens, 1.0, kv_start=starts, mask=mask)


def _mutant_zero_weight_tail(q, k, v, lens, scale, starts, mask=None):
    # masks the tail by multiplying V by a zero weight instead of slicing it away (0 * NaN = NaN)
    cap = k.shape[2]
    out = decode_attention(q, k, v, lens, scale, kv_start=starts, mask=mask)
    tail_nan = np.array([np.isnan(v[b, :, int(lens[b]):]).any() or np.isinf(v[b, :, int(lens[b]):]).any()
                         for b in range(q.shape[0])]) if cap else np.zeros(q.shape[0], bool)
    out[tail_nan] = np.nan
    return out


def _mutant_transposed(q, k, v, lens, scale, starts, mask=None):
    # keys and values swapped
    return decode_attention(q, v, k, lens, scale, kv_start=starts, mask=mask)


@pytest.mark.parametrize("mutant", [_mutant_head_map, _mutant_off_by_one, _mutant_no_scale, _mutant_zero_weight_tail,
                                    _mutant_transposed], ids=lambda m: m.__name__)
def test_planted_mistakes_are_caught(mutant):
    assert not all(check(mutant) for check in CHECKS)


# ---------------------------------------------------------------------------------------------- mask + eager chain

def test_interval_mask_round_trip():
    m = interval_mask([0, 7, 3], 20, 64)
    assert m.dtype == torch.bfloat16 and tuple(m.shape) == (3, 1, 1, 64)
    start, end = mask_interval(m.float().numpy())
    assert start.tolist() == [0, 7, 3] and end.tolist() == [21, 21, 21]
    assert float(m[0, 0, 0, 21]) == torch.finfo(torch.bfloat16).min
    empty = torch.full((1, 1, 1, 8), torch.finfo(torch.float32).min)
    assert [a.tolist() for a in mask_interval(empty.numpy())] == [[0], [0]]


def test_masked_oracle_equals_range_oracle():
    q, k, v, lens, _, scale = _case(31, B=3, NH=8, NKV=2, D=64, cap=40, lens=[40, 40, 40])
    pad = np.array([0, 9, 4])
    pos = 30
    mask = interval_mask(pad, pos, 40).float().numpy().reshape(3, 40)
    a = decode_attention(q, k, v, np.full(3, 40), scale, mask=mask)
    b = decode_attention(q, k, v, np.full(3, pos + 1), scale, kv_start=pad)
    assert np.allclose(a, b, atol=1e-12)


def test_eager_chain_close_to_oracle():
    # the bf16 eager chain (CPU baseline code) agrees with the fp32 oracle to bf16 accuracy
    q, k, v, lens, _, scale = _case(41, B=2, NH=16, NKV=8, D=128, cap=96, lens=[96, 96])
    mask = interval_mask([0, 0], 95, 96)
    out = eager_bf16(torch.from_numpy(q).bfloat16()[:, :, None], torch.from_numpy(k).bfloat16(),
                     torch.from_numpy(v).bfloat16(), mask, scale)
    ref = decode_attention(q, k, v, lens, scale)
    assert out.shape == (2, 1, 16, 128)
    assert np.allclose(out[:, 0].float().numpy(), ref, atol=2e-2, rtol=5e-2)
