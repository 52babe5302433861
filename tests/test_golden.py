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


# ---------------------------------------------------------------------------------------------- fused step, tokens
from oracle.attention import decode_attention_tokens, fused_decode  # noqa: E402
from tests.golden.make_golden import OUT2  # noqa: E402

CASES2 = load(OUT2)


@pytest.mark.parametrize("name", sorted(n for n in CASES2 if n.startswith("fused")))
def test_oracle_reproduces_fused_fixture(name):
    c = CASES2[name]
    out, k2, v2 = fused_decode(c["qkv"], c["qn"], c["kn"], float(c["eps"]), c["cos"], c["sin"], c["k"], c["v"],
                               int(c["pos"]), c["lens"], float(c["scale"]), kv_start=c["starts"])
    assert np.allclose(out, c["out"], rtol=1e-6, atol=1e-7)
    assert np.array_equal(k2[:, :, int(c["pos"])], c["k_slot"]) and np.array_equal(v2[:, :, int(c["pos"])], c["v_slot"])


@pytest.mark.parametrize("name", sorted(n for n in CASES2 if n.startswith("fused")))
def test_fused_fixture_k_slot_matches_transformers(name):
    """The new k of the fixture against transformers' own Qwen3RMSNorm + apply_rotary_pos_emb in bf16."""
    pytest.importorskip("transformers.models.qwen3.modeling_qwen3")
    from tests.test_oracle_prologue import _transformers

    c = CASES2[name]
    B, NKV = c["k"].shape[0], c["k"].shape[1]
    D = c["k"].shape[3]
    NH = c["qkv"].shape[1] // D - 2 * NKV
    heads = c["qkv"].reshape(B, NH + 2 * NKV, D)[:, NH:NH + NKV].reshape(B * NKV, D)
    cos = np.repeat(c["cos"], NKV, axis=0)
    sin = np.repeat(c["sin"], NKV, axis=0)
    ref = _transformers(heads, c["kn"], float(c["eps"]), cos, sin).reshape(B, NKV, D)
    got, want = bf16_to_f32(c["k_slot"]).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    assert (np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30).all()
    assert (c["k_slot"] == ref).mean() > 0.99


@pytest.mark.parametrize("name", sorted(n for n in CASES2 if n.startswith("tokens")))
def test_tokens_fixture(name):
    from tests.test_oracle_tokens import sdpa_tokens

    c = CASES2[name]
    q, k, v = bf16_to_f32(c["q"]), bf16_to_f32(c["k"]), bf16_to_f32(c["v"])
    out = decode_attention_tokens(q, k, v, c["lens"], float(c["scale"]), kv_start=c["starts"])
    assert np.allclose(out, c["out"], rtol=1e-6, atol=1e-7)
    ref = sdpa_tokens(q, k, v, c["lens"], float(c["scale"]), kv_start=c["starts"])
    assert np.allclose(c["out"], ref, atol=2e-5, rtol=1e-5)
