"""GPU: bz_mask_interval (breeze_tts_2_flash_amd.mask_interval) against oracle.attention.mask_interval: per row the
first and last + 1 position whose additive mask value is > -1e30, read from bf16 and fp32 masks of shape
[B, 1, 1, S] and [B, S], a broadcast [1, 1, 1, S] mask, rows with holes and finite biases inside the interval, a row
with nothing attended ([0, 0)), intervals touching both ends, and a mask longer than the capacity (positions past the
capacity are not read). Integer results: bit-exact."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import mask_interval
from oracle.attention import mask_interval as mask_interval_ref

pytestmark = pytest.mark.gpu

NEG = float(torch.finfo(torch.bfloat16).min)


def make_mask(rows, S, rng):
    m = np.full((len(rows), S), NEG, dtype=np.float32)
    for i, (lo, hi) in enumerate(rows):
        if hi > lo:
            m[i, lo:hi] = rng.standard_normal(hi - lo) * 0.5       # finite biases inside the interval
            if hi - lo > 4:
                m[i, lo + 1 + (hi - lo) // 3] = NEG                  # a hole: the interval spans it
    return m


ROWS = [(0, 1), (5, 100), (0, 512), (511, 512), (0, 0), (37, 38), (100, 400), (1, 511)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["b11s", "bs"])
def test_intervals(device, dtype, layout):
    rng = np.random.default_rng(7)
    S = 512
    m = make_mask(ROWS, S, rng)
    t = torch.from_numpy(m).to(dtype)
    ref_start, ref_end = mask_interval_ref(t.float().numpy())
    t = t.to(device)
    if layout == "b11s":
        t = t.view(len(ROWS), 1, 1, S)
    seq_lens, kv_start = mask_interval(t, S)
    torch.cuda.synchronize()
    assert np.array_equal(seq_lens.cpu().numpy(), ref_end)
    assert np.array_equal(kv_start.cpu().numpy(), ref_start)
    assert ref_end[4] == 0 and ref_start[4] == 0


def test_broadcast_and_capacity(device):
    rng = np.random.default_rng(8)
    S = 1024
    m = make_mask([(10, 900)], S, rng)
    t = torch.from_numpy(m).to(torch.bfloat16).to(device).view(1, 1, 1, S)
    seq_lens, kv_start = mask_interval(t, 600, batch=4)      # one mask row for 4 batch rows; capacity 600 < S
    torch.cuda.synchronize()
    assert seq_lens.tolist() == [600] * 4 and kv_start.tolist() == [10] * 4
    out_l = torch.empty(4, dtype=torch.int32, device=device)
    out_s = torch.empty(4, dtype=torch.int32, device=device)
    r = mask_interval(t, S, batch=4, seq_lens=out_l, kv_start=out_s)
    torch.cuda.synchronize()
    assert r[0] is out_l and r[1] is out_s
    assert out_l.tolist() == [900] * 4 and out_s.tolist() == [10] * 4


def test_argument_errors(device):
    t = torch.zeros(2, 64, dtype=torch.float16, device=device)
    with pytest.raises(RuntimeError):
        mask_interval(t, 64)                                  # fp16 mask
    with pytest.raises(RuntimeError):
        mask_interval(torch.zeros(2, 32, dtype=torch.bfloat16, device=device), 64)   # shorter than the capacity
    with pytest.raises(RuntimeError):
        mask_interval(torch.zeros(3, 64, dtype=torch.bfloat16, device=device), 64, batch=2)  # batch mismatch
