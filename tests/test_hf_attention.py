"""Host logic of the transformers registration (breeze_tts_2_flash_amd.hf_attention): the name is registered for the
attention function and for the eager mask builder, and every call the kernel cannot take (here: CPU tensors) goes to
the model's own eager attention with the eager mask, so a CPU model gives bit-identical logits to
attn_implementation="eager"."""
import pytest
import torch

from breeze_tts_2_flash_amd import hf_attention

qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


def tiny_qwen3(impl: str):
    from transformers import Qwen3Config

    cfg = Qwen3Config(vocab_size=256, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=64, max_position_embeddings=256)
    torch.manual_seed(0)
    model = qwen3.Qwen3ForCausalLM(cfg).eval()
    model.config._attn_implementation = impl
    return model


def test_install_registers_attention_and_mask():
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, eager_mask

    name = hf_attention.install()
    assert name == hf_attention.NAME
    assert AttentionInterface._global_mapping[name] is hf_attention.mi355_decode_attention
    assert ALL_MASK_ATTENTION_FUNCTIONS._global_mapping[name] is eager_mask
    assert AttentionInterface._global_mapping[hf_attention.EAGER_NAME] is hf_attention.eager_attention
    assert hf_attention.install() == name  # idempotent


def test_cpu_model_routes_to_eager_bit_identically():
    hf_attention.install()
    ids = torch.randint(0, 256, (2, 9), generator=torch.Generator().manual_seed(1))
    am = torch.ones(2, 9, dtype=torch.long)
    am[1, :3] = 0  # left padding on row 1
    before = dict(hf_attention.calls)
    with torch.no_grad():
        ours = tiny_qwen3(hf_attention.NAME).generate(ids, attention_mask=am, max_new_tokens=3, do_sample=False,
                                                       output_logits=True, return_dict_in_generate=True)
        ref = tiny_qwen3("eager").generate(ids, attention_mask=am, max_new_tokens=3, do_sample=False,
                                           output_logits=True, return_dict_in_generate=True)
    assert torch.equal(ours.sequences, ref.sequences)
    for a, b in zip(ours.logits, ref.logits):
        assert torch.equal(a, b)
    assert hf_attention.calls["hip"] == before["hip"]
    assert hf_attention.calls["eager"] == before["eager"] + 3 * 2  # prefill + 2 decode steps, 2 layers


@pytest.mark.parametrize("q_len,G", [(1, 2), (7, 2), (7, 1), (5, 4)])
def test_eager_attention_matches_transformers_eager(q_len, G):
    """eager_attention (the GPU route for prefill and other non-decode calls) gives transformers' eager attention bit
    for bit: same rounding points, only the operands' memory layout differs."""
    g = torch.Generator().manual_seed(q_len * 10 + G)
    B, NKV, L, D = 2, 2, 19, 64
    q = torch.randn(B, NKV * G, q_len, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, NKV, L, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, NKV, L, D, generator=g).to(torch.bfloat16)
    mask = torch.zeros(B, 1, q_len, L, dtype=torch.bfloat16)
    mask[1, :, :, :4] = torch.finfo(torch.bfloat16).min
    mask[0, :, :, 10:12] = -1.5
    mod = torch.nn.Module()
    mod.num_key_value_groups = G
    mod.eval()
    want, want_w = qwen3.eager_attention_forward(mod, q, k, v, mask, scaling=D ** -0.5)
    got, got_w = hf_attention.eager_attention(mod, q, k, v, mask, scaling=D ** -0.5)
    assert torch.equal(got, want) and torch.equal(got_w, want_w)


def test_install_declines_other_gpus(monkeypatch, capsys):
    """A visible GPU other than gfx950: nothing is registered, "eager" is returned with the reason, and calls that
    reach the function anyway take eager attention (the reference's pre-flight, flash/support.py:67-84)."""
    from breeze_tts_2_flash_amd import kernels

    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(kernels, "device_unsupported", lambda index=None: "Fake GPU (gfx000): the kernels are gfx950 only")
    assert hf_attention.install() == "eager"
    assert "not installed: Fake GPU" in capsys.readouterr().out
    q = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16)
    assert not hf_attention._hip_route(None, q, q, q, None, 0.0)
