"""Host side of the backbone decode step (breeze_tts_2_flash_amd.backbone) and the oracle of the whole step.

- The oracle step (tests/mini_backbone_graph.oracle_step: the embedding and rotary tables of the graph, then
  oracle.gemv.decoder_layer per layer and the final RMSNorm) against the stand-in BackboneGraph's own eager step on
  the CPU, with transformers computing attention in fp32 over the interval mask: the hidden state and every layer's
  new cache slot. Planted mistakes (RoPE positions not shifted by the left padding, a doubled final-norm weight)
  fail.
- A graph the kernels cannot take (CPU tensors, batch 5) keeps its original step, bit for bit, with the reason
  printed once.
"""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import backbone
from mini_backbone_graph import MiniBackboneGraph, bits, build_graph, oracle_step
from oracle.bf16 import bf16_to_f32

pytest.importorskip("transformers.models.qwen3.modeling_qwen3")

FP32_ATTN = "bz_test_fp32_masked"


def _fp32_masked_attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
    G = query.shape[1] // key.shape[1]
    k = key.float().repeat_interleave(G, dim=1)
    v = value.float().repeat_interleave(G, dim=1)
    s = query.float() @ k.transpose(-1, -2) * scaling
    if attention_mask is not None:
        m = attention_mask[:, :, :, :k.shape[-2]].float()
        s = s.masked_fill(m <= -1e30, float("-inf")) + m.clamp_min(0)
    p = torch.softmax(s, dim=-1)
    return (p @ v).to(query.dtype).transpose(1, 2).contiguous(), None


@pytest.fixture(scope="module")
def fp32_attention():
    from transformers import AttentionInterface

    AttentionInterface.register(FP32_ATTN, _fp32_masked_attention)
    return FP32_ATTN


def _close(got_bits, ref_bits, rms_frac=1e-2):
    g, r = bf16_to_f32(got_bits).astype(np.float64), bf16_to_f32(ref_bits).astype(np.float64)
    rms = np.sqrt((r ** 2).mean())
    return bool((np.abs(g - r) <= 2.0 ** -6 * np.abs(r) + rms_frac * rms).all())


def _step_inputs(graph, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 64, (graph.batch_size, 1, 2), generator=g)


def test_oracle_step_matches_eager_graph(fp32_attention):
    graph = build_graph("cpu", attn_implementation=fp32_attention, prefill=100)
    pads, pos = [0, 7], 100
    graph.set_step(_step_inputs(graph), pads, pos)
    want_hidden, want_slots = oracle_step(graph, pads, pos)
    with torch.no_grad():
        graph._decode_step()
    got = bits(graph.hidden_buf.reshape(graph.batch_size, -1))
    assert _close(got, want_hidden), "hidden state"
    assert (got == want_hidden).mean() >= 0.9
    for li, (c, (k_slot, v_slot)) in enumerate(zip(graph.static_cache.layers, want_slots)):
        assert np.array_equal(bits(c.values)[:, :, pos], v_slot), f"layer {li} v slot"
        kd = bf16_to_f32(bits(c.keys)[:, :, pos]) - bf16_to_f32(k_slot)
        assert (np.abs(kd) <= np.abs(bf16_to_f32(k_slot)) * 2.0 ** -7 + 1e-30).all(), f"layer {li} k slot"


def test_oracle_step_planted_mistakes(fp32_attention):
    graph = build_graph("cpu", attn_implementation=fp32_attention, prefill=60)
    pads, pos = [0, 9], 60
    graph.set_step(_step_inputs(graph, 2), pads, pos)
    with torch.no_grad():
        graph._decode_step()
    got = bits(graph.hidden_buf.reshape(graph.batch_size, -1))
    # the first row has no padding, so a RoPE position that ignores the padding only moves the second row
    graph.position_ids.fill_(pos)
    wrong_pos, _ = oracle_step(graph, pads, pos)
    graph.position_ids.copy_(torch.tensor([[pos], [pos - 9]]))
    assert _close(got[:1], wrong_pos[:1]) and not _close(got[1:], wrong_pos[1:])
    # the final norm's weight taken twice
    right, _ = oracle_step(graph, pads, pos)
    assert _close(got, right)
    with torch.no_grad():
        w = graph.model.norm.weight.clone()
        graph.model.norm.weight.mul_(2)
    doubled, _ = oracle_step(graph, pads, pos)
    with torch.no_grad():
        graph.model.norm.weight.copy_(w)
    assert not _close(got, doubled)


class _PatchedGraph(MiniBackboneGraph):
    """A subclass, so that install() patches this class only."""


def test_unsupported_graph_keeps_original_step(capsys):
    graph = build_graph("cpu", prefill=40)
    graph.__class__ = _PatchedGraph
    ids = _step_inputs(graph, 3)
    graph.set_step(ids, [0, 4], 40)
    snapshot = [(c.keys.clone(), c.values.clone()) for c in graph.static_cache.layers]
    with torch.no_grad():
        MiniBackboneGraph._decode_step(graph)
    want = graph.cfg_logits_buf.clone(), graph.hidden_buf.clone()
    for c, (k, v) in zip(graph.static_cache.layers, snapshot):
        c.keys.copy_(k)
        c.values.copy_(v)
    backbone.install(_PatchedGraph)
    try:
        assert _PatchedGraph._decode_step is backbone.fused_decode_step
        with torch.no_grad():
            for _ in range(2):
                graph.set_step(ids, [0, 4], 40)
                graph._decode_step()
    finally:
        backbone.uninstall(_PatchedGraph)
    assert _PatchedGraph._decode_step is MiniBackboneGraph._decode_step
    assert torch.equal(graph.cfg_logits_buf, want[0]) and torch.equal(graph.hidden_buf, want[1])
    out = capsys.readouterr().out
    assert out.count("backbone decode step not taken") == 1, out
    assert "not a contiguous bf16 device tensor" in out


def test_prepare_reasons():
    graph = build_graph("cpu", batch=2, prefill=8)
    assert backbone.prepare(graph) is None
    assert "device tensor" in graph._bz_unsupported
    graph.batch_size = 5
    assert backbone.prepare(graph) is None
    assert graph._bz_unsupported.startswith("batch 5")


def test_install_declines_other_gpus(monkeypatch, capsys):
    """A visible GPU other than gfx950: install() returns False, prints the reason and keeps the original step."""
    from breeze_tts_2_flash_amd import kernels

    class _Declined(_PatchedGraph):
        pass

    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(kernels, "device_unsupported", lambda index=None: "Fake GPU (gfx000): the kernels are gfx950 only")
    before = _Declined._decode_step
    assert backbone.install(_Declined) is False
    assert _Declined._decode_step is before
    assert "not installed: Fake GPU" in capsys.readouterr().out
