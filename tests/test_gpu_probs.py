"""GPU parity of the softmax probabilities (bz_gqa_decode_probs, bz_gqa_decode_fused_probs; the reference's dbg output
of attn_decode / attn_decode_fused, flash/csrc/bb_attn.cu:288-289) against oracle.attention.decode_probabilities:
every value within one bf16 ulp of the float64 probability (|got - ref| <= 2^-8 |ref| + 1e-7: the output is rounded
to bf16, and the fp32 score can sit on the other side of a rounding boundary), and exactly 0 outside each row's range
and at excluded positions. Through the C ABI."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import attn_decode, attn_decode_fused, gqa_decode_probs
from oracle.attention import decode_probabilities, interval_mask, mask_interval, qk_norm_rope, rope_cos_sin
from oracle.bf16 import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu


def bf(x, device):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).to(device)


def assert_probs(got, ref, what):
    got = np.asarray(got, np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite"
    excess = np.abs(got - ref) - (2.0 ** -8 * np.abs(ref) + 1e-7)
    assert excess.max() <= 0, f"{what}: excess {excess.max():.3e}"
    assert (got[ref == 0] == 0).all(), f"{what}: nonzero outside the range or at an excluded position"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_probs_over_ranges(device, D, G):
    rng = np.random.default_rng(D + G)
    B, NKV, cap = 4, 2, 300
    q = rng.standard_normal((B, NKV * G, D)) * 2
    k = rng.standard_normal((B, NKV, cap, D))
    lens = np.array([300, 1, 0, 257])
    starts = np.array([0, 0, 0, 40])
    kq = bf(k, device)
    for b in range(B):  # NaN outside each row's range must not leak
        kq[b, :, :starts[b]] = float("nan")
        kq[b, :, lens[b]:] = float("nan")
    qd = bf(q, device)
    got = gqa_decode_probs(qd, kq, torch.tensor(lens, dtype=torch.int32, device=device), D ** -0.5,
                           kv_start=torch.tensor(starts, dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    ref = decode_probabilities(qd.float().cpu().numpy(), bf(k, "cpu").float().numpy(), lens, D ** -0.5,
                               kv_start=starts)
    assert tuple(got.shape) == (B, NKV * G, cap)
    assert_probs(got.cpu().numpy(), ref, f"D={D} G={G}")
    assert (got[1, :, 0] == 1.0).all()  # one position: probability 1


@pytest.mark.parametrize("mdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_lens", [False, True])
def test_probs_with_mask(device, mdtype, with_lens):
    rng = np.random.default_rng(7)
    B, NH, NKV, D, cap = 2, 16, 8, 128, 520
    q = bf(rng.standard_normal((B, NH, D)), device)
    k = bf(rng.standard_normal((B, NKV, cap, D)), device)
    mask = interval_mask([0, 33], 480, cap, dtype=mdtype)
    mask[0, 0, 0, 100:140] = torch.finfo(mdtype).min   # excluded hole
    mask[1, 0, 0, 200] = 0.75                          # a finite bias
    m2 = mask[:, 0, 0, :].float().numpy()
    start, end = mask_interval(m2)
    lens = torch.tensor(end, dtype=torch.int32, device=device) if with_lens else None
    starts = torch.tensor(start, dtype=torch.int32, device=device) if with_lens else None
    got = gqa_decode_probs(q, k, lens, D ** -0.5, kv_start=starts, mask=mask.to(device))
    torch.cuda.synchronize()
    ref = decode_probabilities(q.float().cpu().numpy(), k.float().cpu().numpy(), end, D ** -0.5, kv_start=start,
                               mask=m2)
    assert_probs(got.cpu().numpy(), ref, f"mask {mdtype} lens={with_lens}")


def test_attn_decode_dbg(device):
    rng = np.random.default_rng(11)
    B, NH, NKV, D, cap = 2, 16, 8, 128, 2048
    q = bf(rng.standard_normal((B, NH, 1, D)), device)
    k = bf(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf(rng.standard_normal((B, NKV, cap, D)), device)
    mask = interval_mask([0, 9], 1023, cap).to(device)
    dbg = torch.full((B, NH, cap), -1.0, device=device)
    out = attn_decode(q, k, v, mask, D ** -0.5, dbg=dbg)
    plain = attn_decode(q, k, v, mask, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16)), "dbg changed the attention output"
    m2 = mask[:, 0, 0, :].float().cpu().numpy()
    start, end = mask_interval(m2)
    ref = decode_probabilities(q[:, :, 0].float().cpu().numpy(), k.float().cpu().numpy(), end, D ** -0.5,
                               kv_start=start, mask=m2)
    assert_probs(dbg.cpu().numpy(), ref, "attn_decode dbg")


def test_attn_decode_fused_dbg(device):
    rng = np.random.default_rng(12)
    B, NH, NKV, D, cap, pos = 2, 16, 8, 128, 1024, 700
    qkv = f32_to_bf16((rng.standard_normal((B, (NH + 2 * NKV) * D)) * 3).astype(np.float32))
    qn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    kn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    cos, sin = (f32_to_bf16(t) for t in rope_cos_sin([pos] * B, D))
    kc0 = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))
    vc0 = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))

    def t(b):
        return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(device)

    mask = interval_mask([0, 5], pos, cap).to(device)
    cp = torch.tensor([pos], dtype=torch.int64, device=device)
    cs, sn = t(cos).view(B, 1, D), t(sin).view(B, 1, D)
    kc, vc = t(kc0), t(vc0)
    dbg = torch.full((B, NH, cap), -1.0, device=device)
    out = attn_decode_fused(t(qkv), t(qn), t(kn), 1e-6, cs, sn, kc, vc, mask, cp, D ** -0.5, dbg=dbg)
    kc2, vc2 = t(kc0), t(vc0)
    plain = attn_decode_fused(t(qkv), t(qn), t(kn), 1e-6, cs, sn, kc2, vc2, mask, cp, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16)), "dbg changed the attention output"
    # q as the fused step computes it; K with the step's new k at pos (the cache the kernel left)
    heads = qkv.reshape(B, NH + 2 * NKV, D)
    q = bf16_to_f32(qk_norm_rope(heads[:, :NH], qn, 1e-6, cos.reshape(B, 1, D), sin.reshape(B, 1, D)))
    k_after = kc.float().cpu().numpy()
    m2 = mask[:, 0, 0, :].float().cpu().numpy()
    start, end = mask_interval(m2)
    ref = decode_probabilities(q, k_after, end, D ** -0.5, kv_start=start, mask=m2)
    assert_probs(dbg.cpu().numpy(), ref, "attn_decode_fused dbg")
    assert (dbg[:, :, pos] > 0).all()  # the step's own position is attended


def test_probs_argument_errors(device):
    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16, device=device)
    k = torch.zeros(2, 8, 64, 128, dtype=torch.bfloat16, device=device)
    lens = torch.tensor([4, 4], dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError):  # probs too small
        gqa_decode_probs(q, k, lens, 0.1, torch.empty(2, 16, 63, device=device))
    with pytest.raises(RuntimeError):  # probs not float32
        gqa_decode_probs(q, k, lens, 0.1, torch.empty(2, 16, 64, dtype=torch.bfloat16, device=device))
    with pytest.raises(RuntimeError):  # two query tokens per row
        gqa_decode_probs(torch.zeros(2, 16, 2, 128, dtype=torch.bfloat16, device=device), k, lens, 0.1)
    with pytest.raises(RuntimeError):  # neither seq_lens nor a mask
        gqa_decode_probs(q, k, None, 0.1)
