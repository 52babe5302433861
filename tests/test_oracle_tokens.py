"""Pins of oracle.attention.decode_attention_tokens (T query tokens per row, causal among themselves): torch's SDPA
with a causal mask built from the query positions (a different statement of the same rule), closed forms of the
depth transformer's first step, and planted mistakes that the SDPA pin must reject."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import _row_range, decode_attention, decode_attention_tokens


def sdpa_tokens(q, k, v, seq_lens, scale, kv_start=None):
    """Token t of row b sits at position end_b - T + t and sees key j iff start_b <= j <= its position."""
    q, k, v = (torch.as_tensor(np.asarray(x), dtype=torch.float32) for x in (q, k, v))
    B, NH, T, D = q.shape
    G = NH // k.shape[1]
    out = torch.zeros(B, T, NH, D)
    for b in range(B):
        start, end = _row_range(b, seq_lens, kv_start, k.shape[2])
        qpos = torch.arange(T) + end - T
        j = torch.arange(k.shape[2])
        allowed = (j[None, :] >= start) & (j[None, :] <= qpos[:, None])  # [T, cap]
        kh = k[b].repeat_interleave(G, dim=0)
        vh = v[b].repeat_interleave(G, dim=0)
        for t in range(T):
            if allowed[t].any():
                o = F.scaled_dot_product_attention(q[b, :, t:t + 1], kh[:, allowed[t]], vh[:, allowed[t]], scale=scale)
                out[b, t] = o[:, 0]
    return out.numpy()


def _case(seed, B=2, NH=8, NKV=2, T=2, D=128, cap=16):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, NH, T, D)).astype(np.float32)
    k = rng.standard_normal((B, NKV, cap, D)).astype(np.float32)
    v = rng.standard_normal((B, NKV, cap, D)).astype(np.float32)
    return q, k, v


@pytest.mark.parametrize("T,lens,starts", [(2, [2, 2], None), (2, [9, 16], [0, 3]), (3, [5, 12], [1, 0]),
                                            (4, [16, 7], [2, 2]), (4, [3, 8], [0, 6])])
def test_matches_sdpa_with_causal_mask(T, lens, starts):
    q, k, v = _case(T * 7 + lens[0], T=T)
    st = None if starts is None else np.array(starts)
    got = decode_attention_tokens(q, k, v, np.array(lens), 128 ** -0.5, kv_start=st)
    ref = sdpa_tokens(q, k, v, np.array(lens), 128 ** -0.5, kv_start=st)
    assert np.allclose(got, ref, atol=2e-5, rtol=1e-5)


def test_depth_first_step_closed_forms():
    # step 0 of the depth transformer: two tokens at positions 0 and 1 (depth_frame.cu:221-227)
    q, k, v = _case(5)
    out = decode_attention_tokens(q, k, v, np.array([2, 2]), 128 ** -0.5)
    G = 4
    for h in range(8):
        assert np.array_equal(out[:, 0, h], v[:, h // G, 0].astype(np.float64))  # token 0 sees only position 0
    # the last token of any T equals the single-token decode over the whole row
    q4, k4, v4 = _case(6, T=4)
    lens = np.array([11, 16])
    last = decode_attention_tokens(q4, k4, v4, lens, 0.1)[:, 3]
    assert np.array_equal(last, decode_attention(q4[:, :, 3], k4, v4, lens, 0.1))


def _shifted(shift):
    """A mutant of the oracle whose token t ends `shift(T, t)` positions before the row end."""
    def f(q, k, v, seq_lens, scale, kv_start=None):
        q = np.asarray(q, dtype=np.float64)
        B, NH, T, D = q.shape
        out = np.zeros((B, T, NH, D))
        for t in range(T):
            ends = np.array([max(0, int(seq_lens[b]) - shift(T, t)) for b in range(B)])
            out[:, t] = decode_attention(q[:, :, t], k, v, ends, scale, kv_start=kv_start)
        return out
    return f


@pytest.mark.parametrize("mutant", [
    _shifted(lambda T, t: T - t),        # off by one: token t misses its own position
    _shifted(lambda T, t: t),            # tokens reversed
    _shifted(lambda T, t: 0),            # no causality among the tokens
])
def test_planted_mistakes_caught(mutant):
    q, k, v = _case(8, T=3)
    lens = np.array([9, 14])
    ref = sdpa_tokens(q, k, v, lens, 128 ** -0.5)
    assert not np.allclose(mutant(q, k, v, lens, 128 ** -0.5), ref, atol=1e-3)
