"""GPU: masks whose excluded holes cover whole chunks. With the range taken from the mask (bz_gqa_decode_masked, the
mask form of bz_gqa_decode_fused), a workgroup whose chunk the mask excludes entirely streams nothing and leaves an
empty partial, as the reference skips its fully masked 64-position chunks (bb_attn.cu:9-11, :151-154). The output
must still match the oracle (|d| <= 2e-3 + 1e-2 |ref|), with NaN in every excluded position of K and V, at every
split count and in both merge modes; the fused step must still write its cache slot when that slot lies in a
skipped chunk."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import gqa_decode_fused, gqa_decode_masked
from oracle.attention import decode_attention, fused_decode, rope_cos_sin
from oracle.bf16 import f32_to_bf16
from tests.test_gpu_parity import assert_close, oracle, rand_case

pytestmark = pytest.mark.gpu


def holey_mask(cap, B, dtype):
    """Row 0 attends [0, 100) and [3000, 3100); row 1 [40, 60), [1500, 1530) and [4000, 4096); everything else is
    excluded, so most chunks of both rows hold no attended position."""
    m = torch.full((B, 1, 1, cap), torch.finfo(dtype).min, dtype=dtype)
    for b, spans in enumerate([[(0, 100), (3000, 3100)], [(40, 60), (1500, 1530), (4000, 4096)]]):
        for lo, hi in spans:
            m[b, 0, 0, lo:hi] = 0.0
    m[1, 0, 0, 1510] = -0.5  # a finite bias inside a span
    return m


@pytest.mark.parametrize("splits", [0, 1, 4, 16, 64])
@pytest.mark.parametrize("combine", ["last_block", "kernel"])
@pytest.mark.parametrize("mdtype", [torch.bfloat16, torch.float32])
def test_holes_over_whole_chunks(device, splits, combine, mdtype):
    B, NH, NKV, D, cap = 2, 16, 8, 128, 4096
    w, _ = rand_case(61, B, NH, NKV, D, cap, [cap, cap])
    mask = holey_mask(cap, B, mdtype)
    m2 = mask[:, 0, 0, :].float().numpy()
    ref = oracle(w, mask=m2)
    g = w.to(device)
    kn, vn = g.k.clone(), g.v.clone()
    excluded = torch.from_numpy(m2 <= -1e30).to(device)
    for b in range(B):
        kn[b, :, excluded[b]] = float("nan")
        vn[b, :, excluded[b]] = float("nan")
    out = gqa_decode_masked(g.q, kn, vn, mask.to(device), g.scale, num_splits=splits, combine=combine)
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), ref, f"splits={splits} combine={combine}")


def test_fused_slot_in_a_skipped_chunk(device):
    """The new slot lies inside an excluded hole: nobody attends it, but it must be written."""
    B, NH, NKV, D, cap, pos = 2, 16, 8, 128, 4096, 2000
    rng = np.random.default_rng(62)
    qkv = f32_to_bf16((rng.standard_normal((B, (NH + 2 * NKV) * D)) * 3).astype(np.float32))
    qn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    kn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    cos, sin = (f32_to_bf16(t) for t in rope_cos_sin([pos] * B, D))
    kc0 = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))
    vc0 = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))
    mask = holey_mask(cap, B, torch.bfloat16)
    m2 = mask[:, 0, 0, :].float().numpy()

    def t(bits):
        return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)

    kc, vc = t(kc0), t(vc0)
    out = gqa_decode_fused(t(qkv), t(qn), t(kn), 1e-6, t(cos), t(sin), kc, vc,
                           torch.tensor([pos], dtype=torch.int64, device=device), D ** -0.5, mask=mask.to(device),
                           num_splits=16)
    torch.cuda.synchronize()
    ref, k_ref, v_ref = fused_decode(qkv, qn, kn, 1e-6, cos, sin, kc0, vc0, pos, np.full(B, cap), D ** -0.5, mask=m2)
    assert_close(out.float().cpu().numpy(), ref, "fused, slot in a hole")
    got_v = vc.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got_v[:, :, pos], v_ref[:, :, pos]), "the slot in the skipped chunk was not written"
