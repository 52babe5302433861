"""GPU parity of T query tokens per row (causal among themselves) against oracle.attention.decode_attention_tokens:
the depth transformer's first step (8 q / 2 KV heads, head_dim 128, two tokens at positions 0 and 1,
flash/csrc/depth_frame.cu:221-227) with the query read from the reference's [B * T, NH * D] projection rows, and
longer rows at the backbone shape with split-K, left padding, the interval mask and both output layouts.
Tolerance |out - ref| <= 2e-3 + 1e-2 |ref|."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import gqa_decode, gqa_decode_masked
from oracle.attention import decode_attention_tokens, interval_mask

pytestmark = pytest.mark.gpu


def bf16(x, device):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).to(device)


def check(got, q, k, v, lens, scale, starts=None, what=""):
    ref = decode_attention_tokens(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                  np.asarray(lens), scale, kv_start=None if starts is None else np.asarray(starts))
    g = got.float().cpu().numpy()
    assert np.isfinite(g).all(), what
    excess = np.abs(g - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert excess.max() <= 0, f"{what}: excess {excess.max():.3e}"


def test_depth_first_step(device):
    rng = np.random.default_rng(21)
    B, T, NH, NKV, D, cap = 2, 2, 8, 2, 128, 16
    qb = bf16(rng.standard_normal((B * T, NH * D)), device)          # row m = b * T + t, as the reference's qb
    q = qb.view(B, T, NH, D).permute(0, 2, 1, 3)                      # [B, NH, T, D] view, token stride NH * D
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    lens = torch.tensor([2, 2], dtype=torch.int32, device=device)
    out = gqa_decode(q, k, v, lens, D ** -0.5)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (B, T, NH, D)
    check(out, q, k, v, [2, 2], D ** -0.5, what="depth step 0")
    # token 0 sees position 0 only: its output is that V row, bit for bit
    for h in range(NH):
        assert torch.equal(out[:, 0, h], v[:, h // 4, 0])


@pytest.mark.parametrize("T", [2, 3, 4])
@pytest.mark.parametrize("splits", [0, 1, 7, 16])
@pytest.mark.parametrize("combine", ["last_block", "kernel"])
def test_backbone_tokens(device, T, splits, combine):
    rng = np.random.default_rng(T * 100 + splits)
    B, NH, NKV, D, cap = 2, 16, 8, 128, 1024
    q = bf16(rng.standard_normal((B, NH, T, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    lens, starts = [1000, 613], [0, 41]
    out = gqa_decode(q, k, v, torch.tensor(lens, dtype=torch.int32, device=device), D ** -0.5,
                     kv_start=torch.tensor(starts, dtype=torch.int32, device=device), num_splits=splits,
                     combine=combine)
    torch.cuda.synchronize()
    check(out, q, k, v, lens, D ** -0.5, starts, f"T={T} splits={splits} {combine}")


def test_tokens_interval_mask_and_layouts(device):
    rng = np.random.default_rng(33)
    B, T, NH, NKV, D, cap = 2, 3, 16, 8, 64, 512
    q = bf16(rng.standard_normal((B, NH, T, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    pos, pad = 300, [0, 57]                                   # last token at position 300, left padding on row 1
    mask = interval_mask(pad, pos, cap).to(device)
    out_tn = torch.empty(B, T, NH, D, dtype=torch.bfloat16, device=device)
    out_nt = torch.empty(B, NH, T, D, dtype=torch.bfloat16, device=device)
    gqa_decode_masked(q, k, v, mask, D ** -0.5, out_tn)
    gqa_decode_masked(q, k, v, mask, D ** -0.5, out_nt)
    torch.cuda.synchronize()
    check(out_tn, q, k, v, [pos + 1] * B, D ** -0.5, pad, "interval mask, [B, T, NH, D]")
    assert torch.equal(out_nt.permute(0, 2, 1, 3), out_tn)


def test_rows_shorter_than_tokens(device):
    # a row of one position with T = 3: tokens 0 and 1 have no position (output 0), token 2 sees position 0
    rng = np.random.default_rng(44)
    B, T, NH, NKV, D, cap = 2, 3, 4, 2, 128, 64
    q = bf16(rng.standard_normal((B, NH, T, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    out = gqa_decode(q, k, v, torch.tensor([1, 2], dtype=torch.int32, device=device), D ** -0.5)
    torch.cuda.synchronize()
    check(out, q, k, v, [1, 2], D ** -0.5, what="short rows")
    assert torch.count_nonzero(out[0, :2]) == 0 and torch.count_nonzero(out[1, 0]) == 0


def test_golden_tokens_fixtures(device):
    """tests/golden/fused_and_tokens.npz: the several-token cases through gqa_decode."""
    from tests.golden.make_golden import OUT2, load

    for name, c in sorted(load(OUT2).items()):
        if not name.startswith("tokens"):
            continue
        t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)  # noqa: E731
        out = gqa_decode(t(c["q"]), t(c["k"]), t(c["v"]), torch.from_numpy(c["lens"]).to(device), float(c["scale"]),
                         kv_start=torch.from_numpy(c["starts"]).to(device))
        torch.cuda.synchronize()
        g = out.float().cpu().numpy()
        excess = np.abs(g - c["out"]) - (2e-3 + 1e-2 * np.abs(c["out"]))
        assert excess.max() <= 0, f"golden {name}: excess {excess.max():.3e}"
