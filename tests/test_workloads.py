"""Host logic: the seeded workloads and the algorithmic byte counts the roofline uses."""
import torch

from breeze_tts_2_flash_amd import workloads


def test_algorithmic_bytes_match_published_counts():
    # BASELINE byte counts per call (K+V of valid positions + q + out + seq_lens)
    assert workloads.algorithmic_bytes([256, 256], 16, 8, 128) == 2_113_544
    assert workloads.algorithmic_bytes([1024, 1024], 16, 8, 128) == 8_405_000
    assert workloads.algorithmic_bytes([4096, 4096], 16, 8, 128) == 33_570_824
    lens = [300, 300, 2000, 2000]
    assert workloads.algorithmic_bytes(lens, 16, 8, 128) == 4096 * sum(lens) + 4 * 16 * 128 * 2 * 2 + 16
    frame = sum(workloads.algorithmic_bytes([L, L], 16, 8, 64) for L in range(1, 33))
    assert frame == 2_425_088
    assert workloads.flops([1024, 1024], 16, 128) == 16_777_216
    # fused step: + raw k and v (2 rows x 2 x 8 heads x 128 x 2 B), 2 norm weights, cos/sin [2, 128], the slot write
    # of k and v (same size as the raw reads) and the int64 cache_pos
    assert workloads.fused_algorithmic_bytes([1024, 1024], 16, 8, 128) == 8_405_000 + 8192 + 512 + 1024 + 8192 + 8


def test_config_shapes_and_determinism():
    a, b = workloads.make(1), workloads.make(1)
    assert torch.equal(a.q.view(torch.int16), b.q.view(torch.int16))
    assert tuple(a.k.shape) == (2, 8, 256, 128) and a.k.dtype == torch.bfloat16
    w2 = workloads.make(2)
    assert tuple(w2.k.shape) == (2, 8, 2048, 128) and w2.seq_lens.tolist() == [1024, 1024]
    w5 = workloads.make(5)
    assert tuple(w5.q.shape) == (32, 2, 16, 64) and w5.seq_lens[:, 0].tolist() == list(range(1, 33))


def test_long_config_hot_positions():
    w = workloads.make(3)
    hot = w.extras["hot"]
    assert tuple(w.k.shape) == (2, 8, 4096, 128)
    assert 0.005 < hot.float().mean().item() < 0.015
    # hot positions carry K scaled by 8: their mean |K| is ~8x the others'
    kabs = w.k.float().abs().mean(dim=(1, 3))
    ratio = kabs[hot].mean() / kabs[~hot].mean()
    assert 7.0 < ratio.item() < 9.0


def test_ragged_config_nan_tails():
    w = workloads.make(4)
    lens = w.seq_lens.tolist()
    assert len(lens) == 16 and all(lens[2 * i] == lens[2 * i + 1] for i in range(8))
    assert all(128 <= L <= 2048 for L in lens)
    for b, L in enumerate(lens):
        assert not torch.isnan(w.k[b, :, :L].float()).any()
        assert torch.isnan(w.k[b, :, L:].float()).all() and torch.isnan(w.v[b, :, L:].float()).all()
