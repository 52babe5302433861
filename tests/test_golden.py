"""The committed golden fixtures (tests/golden/decode_attention.npz): the oracle still reproduces them, and they
agree with torch's fp32 scaled_dot_product_attention (a library routine) where no mask is involved."""
import numpy as np
import pytest
import torch

from oracle.attention import decode_attention, sdpa_fp32
from oracle.bf16 import bf16_to_f32
from tests.golden.make_golden import load

CASES = load()


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_reproduces_fixture(name):
    c = CASES[name]
    mask = bf16_to_f32(c["mask"]) if "mask" in c else None
    out = decode_attention(bf16_to_f32(c["q"]), bf16_to_f32(c["k"]), bf16_to_f32(c["v"]), c["lens"],
                           float(c["scale"]), kv_start=c["starts"], mask=mask)
    assert np.allclose(out, c["out"], rtol=1e-6, atol=1e-7)
    assert np.isfinite(c["out"]).all()


@pytest.mark.parametrize("name", [n for n in sorted(CASES) if "mask" not in CASES[n]])
def test_fixture_matches_torch_sdpa(name):
    c = CASES[name]
    t = lambda a: torch.from_numpy(bf16_to_f32(a))  # noqa: E731
    ref = sdpa_fp32(t(c["q"]), t(c["k"]), t(c["v"]), c["lens"], float(c["scale"]), c["starts"]).numpy()
    assert np.allclose(c["out"], ref, atol=2e-6, rtol=2e-5)
