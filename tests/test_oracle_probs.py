"""Pins of oracle.attention.decode_probabilities (the softmax probabilities behind decode_attention; the reference's
optional dbg output of attn_decode, flash/csrc/bb_attn.cu:288-289):

- library routine: torch.softmax in float64 over q.k * scale + mask with the KV heads expanded (repeat_kv), inside each
  row's range, zeros outside;
- consistency: probabilities @ V equals decode_attention, itself pinned against torch SDPA (test_oracle.py);
- closed forms: one position has probability 1; q = 0 spreads 1 / n over the n kept positions; excluded holes, the
  tail and empty rows are 0;
- planted mistakes (head map h % NKV, inclusive range end, no scale, no normalisation, K taken from the wrong row)
  each fail at least one of these.
"""
import numpy as np
import pytest
import torch

from oracle.attention import decode_attention, decode_probabilities, EXCLUDED


def _case(seed, B=3, NH=8, NKV=2, D=32, cap=40):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, NH, D))
    k = rng.standard_normal((B, NKV, cap, D))
    v = rng.standard_normal((B, NKV, cap, D))
    lens = rng.integers(cap // 2, cap + 1, B)
    starts = np.array([min(int(rng.integers(0, 6)), int(lens[b])) for b in range(B)])
    mask = rng.standard_normal((B, cap)) * 0.5
    mask[:, 3] = -1e38  # an excluded hole
    return q, k, v, lens, starts, mask, D ** -0.5


def check_vs_torch(impl):
    for seed in range(3):
        q, k, v, lens, starts, mask, scale = _case(seed)
        B, NH, D = q.shape
        G = NH // k.shape[1]
        got = impl(q, k, lens, scale, starts, mask)
        ref = np.zeros_like(got)
        for b in range(B):
            s0, e0 = int(starts[b]), int(lens[b])
            kk = torch.from_numpy(k[b]).repeat_interleave(G, dim=0)[:, s0:e0]       # [NH, L, D]
            sc = torch.einsum("hd,hld->hl", torch.from_numpy(q[b]), kk) * scale
            m = torch.from_numpy(mask[b, s0:e0])
            sc = torch.where(m > EXCLUDED, sc + m, torch.tensor(-np.inf, dtype=torch.float64))
            ref[b, :, s0:e0] = torch.softmax(sc, dim=-1).numpy()
        if not np.allclose(got, ref, atol=1e-12):
            return False
    return True


def check_consistency(impl):
    for seed in range(3, 6):
        q, k, v, lens, starts, mask, scale = _case(seed)
        p = impl(q, k, lens, scale, starts, mask)
        NH, NKV = q.shape[1], k.shape[1]
        vh = np.repeat(v, NH // NKV, axis=1)                                      # [B, NH, cap, D]
        out = np.einsum("bhl,bhld->bhd", p, vh)
        if not np.allclose(out, decode_attention(q, k, v, lens, scale, kv_start=starts, mask=mask), atol=1e-12):
            return False
    return True


def check_closed_forms(impl):
    q, k, v, lens, starts, mask, scale = _case(7, B=2)
    cap = k.shape[2]
    one = impl(q, k, np.array([6, 0]), scale, np.array([5, 0]), None)
    if not (one[0, :, 5] == 1.0).all() or np.count_nonzero(one[0]) != q.shape[1] or np.count_nonzero(one[1]):
        return False
    m = np.zeros((2, cap))
    m[:, 10] = -1e38
    flat = impl(np.zeros_like(q), k, np.array([20, 20]), scale, np.array([0, 4]), m)
    for b, n in ((0, 19), (1, 15)):
        kept = np.ones(cap, bool)
        kept[10] = False
        kept[:(0, 4)[b]] = False
        kept[20:] = False
        if not (np.allclose(flat[b][:, kept], 1.0 / n, atol=1e-15) and (flat[b][:, ~kept] == 0).all()):
            return False
    return True


CHECKS = [check_vs_torch, check_consistency, check_closed_forms]


def _oracle(q, k, lens, scale, starts, mask):
    return decode_probabilities(q, k, lens, scale, kv_start=starts, mask=mask)


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes(check):
    assert check(_oracle)


def _mutant_head_map(q, k, lens, scale, starts, mask):
    idx = np.arange(q.shape[1]) % k.shape[1]
    return decode_probabilities(q, k[:, idx], lens, scale, kv_start=starts, mask=mask)


def _mutant_inclusive_end(q, k, lens, scale, starts, mask):
    return decode_probabilities(q, k, np.minimum(np.asarray(lens) + 1, k.shape[2]), scale, kv_start=starts, mask=mask)


def _mutant_no_scale(q, k, lens, scale, starts, mask):
    return decode_probabilities(q, k, lens, 1.0, kv_start=starts, mask=mask)


def _mutant_unnormalised(q, k, lens, scale, starts, mask):
    p = decode_probabilities(q, k, lens, scale, kv_start=starts, mask=mask)
    return p * np.maximum(1, np.count_nonzero(p, axis=-1, keepdims=True)) ** 0.5


def _mutant_wrong_row(q, k, lens, scale, starts, mask):
    return decode_probabilities(q, k[::-1].copy(), lens, scale, kv_start=starts, mask=mask)


@pytest.mark.parametrize("mutant", [_mutant_head_map, _mutant_inclusive_end, _mutant_no_scale, _mutant_unnormalised,
                                    _mutant_wrong_row], ids=lambda m: m.__name__)
def test_planted_mistakes_are_caught(mutant):
    assert not all(check(mutant) for check in CHECKS)
