"""GPU: the kernel inside a transformers model (breeze_tts_2_flash_amd.hf_attention). A tiny random-weight Qwen3
(the reference backbone's layer type: q_norm / k_norm, RoPE, GQA 16 q / 8 KV heads, head_dim 128), bf16 on the GPU,
left-padded batch of 2, greedy generation with a StaticCache and with a DynamicCache. Every q_len == 1 call must take
the HIP route and match the fp32 oracle on the exact tensors the model passed (|d| <= 2e-3 + 1e-2 |ref|); the
end-to-end logits must stay close to the same model run with eager attention (hf_attention.EAGER_NAME: transformers'
eager rounding points with contiguous operands, so no bf16 batched product takes a transposed view on the GPU)."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import hf_attention
from oracle.attention import decode_attention, mask_interval

pytestmark = pytest.mark.gpu
qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")

REC = "mi355_decode_recording"
records = []


def recording_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    before = hf_attention.calls["hip"]
    out, w = hf_attention.mi355_decode_attention(module, query, key, value, attention_mask, scaling=scaling,
                                                 dropout=dropout, **kwargs)
    if hf_attention.calls["hip"] > before:
        records.append(tuple(t.detach().float().cpu() for t in (query, key, value, attention_mask[:, :, -1], out)) +
                       (scaling,))
    return out, w


def tiny_qwen3(impl, device):
    from transformers import Qwen3Config

    cfg = Qwen3Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128, max_position_embeddings=512)
    torch.manual_seed(0)
    model = qwen3.Qwen3ForCausalLM(cfg).to(device=device, dtype=torch.bfloat16).eval()
    model.config._attn_implementation = impl
    return model


def generate(model, ids, am, cache):
    kw = dict(cache_implementation="static") if cache == "static" else {}
    with torch.no_grad():
        return model.generate(ids, attention_mask=am, max_new_tokens=5, do_sample=False, output_logits=True,
                              return_dict_in_generate=True, **kw)


@pytest.mark.parametrize("cache", ["static", "dynamic"])
def test_qwen3_decode_through_registered_attention(device, cache):
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, eager_mask

    hf_attention.install()
    AttentionInterface.register(REC, recording_attention)
    ALL_MASK_ATTENTION_FUNCTIONS.register(REC, eager_mask)
    records.clear()
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 512, (2, 24), generator=g).to(device)
    am = torch.ones(2, 24, dtype=torch.long, device=device)
    am[1, :9] = 0  # left padding: row 1 attends from position 9
    hip0 = hf_attention.calls["hip"]
    ours = generate(tiny_qwen3(REC, device), ids, am, cache)
    ref = generate(tiny_qwen3(hf_attention.EAGER_NAME, device), ids, am, cache)

    # 4 decode forwards (the first new token comes from prefill) x 2 layers, all on the HIP route
    assert hf_attention.calls["hip"] - hip0 == 8 and len(records) == 8
    for i, (q, k, v, m, out, scale) in enumerate(records):
        start, end = mask_interval(m.numpy())
        assert start[0] == 0 and start[1] == 9, (i, start)
        oracle = decode_attention(q[:, :, 0].numpy(), k.numpy(), v.numpy(), end, scale, kv_start=start,
                                  mask=m.reshape(m.shape[0], -1).numpy())
        got = out[:, 0].numpy()
        excess = np.abs(got - oracle) - (2e-3 + 1e-2 * np.abs(oracle))
        assert excess.max() <= 0, f"call {i}: excess {excess.max():.3e}"

    # end to end against eager bf16 attention: the prefill logits are the same computation; decode
    # logits differ only by the attention's rounding (eager rounds scores and probabilities to bf16)
    assert torch.equal(ours.logits[0], ref.logits[0])
    steps = 1
    while steps < len(ours.logits) and torch.equal(ours.sequences[:, 24:24 + steps], ref.sequences[:, 24:24 + steps]):
        a, b = ours.logits[steps].float(), ref.logits[steps].float()
        assert (a - b).abs().max() <= 0.05 * b.abs().max() + 0.05, f"decode step {steps}"
        steps += 1
    assert steps >= 2  # at least the first decode step had identical inputs and was compared
