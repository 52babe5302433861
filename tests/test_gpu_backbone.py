"""GPU: the whole backbone decode step through breeze_tts_2_flash_amd.backbone (the reference's fused step,
flash/backbone.py:112-136, in place of BackboneGraph._decode_step) on the stand-in BackboneGraph of
tests/mini_backbone_graph.py: a random-init bf16 Qwen3 backbone (head_dim 128, 2 layers), a 256-slot static cache
holding 100 prefilled positions (and a 1024-slot cache holding 600, whose rows span many splits), left padding,
codebook embeddings, the fp32 lm_head and CFG.

- Against the CPU oracle of the step (oracle_step: oracle.gemv.decoder_layer per layer + the final RMSNorm):
  |hidden - ref| <= 2^-5 |ref| + 1e-2 rms(ref) (the attention output's 2e-3 + 1e-2 |ref| carried through o_proj and
  the MLP, plus bf16 rounding differences of the GEMVs), the new v slot of every layer bit for bit and the new k slot
  within one bf16 ulp.
- Against the graph's own eager step (eager attention rounding scores and probabilities to bf16): the CFG logits
  within 5% of their largest magnitude.
- install() on the graph class, then capture() into one HIP graph as BackboneGraph does: three replays with the
  position, mask and token ids advanced on the host between them, each equal bit for bit to the same step run
  eagerly through the library.
"""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import backbone, hf_attention
from mini_backbone_graph import MiniBackboneGraph, bits, build_graph, oracle_step
from oracle.bf16 import bf16_to_f32

pytestmark = pytest.mark.gpu
pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


@pytest.fixture(scope="module")
def eager_name():
    hf_attention.install()
    return hf_attention.EAGER_NAME


def _ids(graph, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 64, (graph.batch_size, 1, 2), generator=g).to(graph.device)


def _snapshot(graph):
    return [(c.keys.clone(), c.values.clone()) for c in graph.static_cache.layers]


def _restore(graph, snap):
    for c, (k, v) in zip(graph.static_cache.layers, snap):
        c.keys.copy_(k)
        c.values.copy_(v)


# the last case spreads each row over many splits: a 1024-slot cache, 600 filled, left padding up to 250
@pytest.mark.parametrize("batch,pads,cap,pos", [(2, [0, 7], 256, 100), (1, [3], 256, 100),
                                               (4, [0, 5, 0, 12], 256, 100), (2, [250, 0], 1024, 600)])
def test_step_matches_oracle_and_eager(device, eager_name, batch, pads, cap, pos):
    graph = build_graph(device, batch=batch, max_seq_len=cap, prefill=pos, attn_implementation=eager_name,
                        seed=batch)
    print(f"backbone step: batch {batch}, pads {pads}, cache_pos {pos}", flush=True)
    ids = _ids(graph, 5)
    graph.set_step(ids, pads, pos)
    snap = _snapshot(graph)
    want_hidden, want_slots = oracle_step(graph, pads, pos)
    with torch.no_grad():
        graph._decode_step()
    eager_cfg = graph.cfg_logits_buf.clone()
    _restore(graph, snap)
    graph.set_step(ids, pads, pos)
    with torch.no_grad():
        backbone.fused_decode_step(graph)
    torch.cuda.synchronize()
    assert backbone.prepare(graph) is not None, getattr(graph, "_bz_unsupported", "")

    got = bits(graph.hidden_buf.reshape(batch, -1))
    g, r = bf16_to_f32(got).astype(np.float64), bf16_to_f32(want_hidden).astype(np.float64)
    rms = np.sqrt((r ** 2).mean())
    err = np.abs(g - r)
    print(f"  hidden: max |d| {err.max():.3e}, rms(ref) {rms:.3f}, exact {(got == want_hidden).mean():.3f}", flush=True)
    assert (err <= 2.0 ** -5 * np.abs(r) + 1e-2 * rms).all()
    for li, (c, (k_slot, v_slot)) in enumerate(zip(graph.static_cache.layers, want_slots)):
        assert np.array_equal(bits(c.values)[:, :, pos], v_slot), f"layer {li} v slot"
        kd = np.abs(bf16_to_f32(bits(c.keys)[:, :, pos]) - bf16_to_f32(k_slot))
        assert (kd <= np.abs(bf16_to_f32(k_slot)) * 2.0 ** -7 + 1e-30).all(), f"layer {li} k slot"
    # the other slots are untouched
    for c, (k0, v0) in zip(graph.static_cache.layers, snap):
        keep = torch.ones(c.keys.size(2), dtype=torch.bool, device=device)
        keep[pos] = False
        assert torch.equal(c.keys[:, :, keep], k0[:, :, keep]) and torch.equal(c.values[:, :, keep], v0[:, :, keep])

    d = (graph.cfg_logits_buf - eager_cfg).abs().max().item()
    assert d <= 0.05 * eager_cfg.abs().max().item(), f"CFG logits vs the eager step: {d:.3e}"


class _CapturedGraph(MiniBackboneGraph):
    """A subclass, so that install() patches this class only."""


@pytest.mark.parametrize("pads,cap,pos0", [([0, 7], 256, 100), ([250, 0], 1024, 600)])
def test_installed_step_in_a_hip_graph(device, eager_name, pads, cap, pos0):
    graph = build_graph(device, batch=2, max_seq_len=cap, prefill=pos0, attn_implementation=eager_name, seed=11)
    graph.__class__ = _CapturedGraph
    backbone.install(_CapturedGraph)
    try:
        graph.set_step(_ids(graph, 1), pads, pos0)
        with torch.no_grad():
            graph.capture()
        snap = _snapshot(graph)
        replays = []
        for i in range(3):
            print(f"replay {i}: cache_pos {pos0 + i}", flush=True)
            graph.set_step(_ids(graph, 20 + i), pads, pos0 + i)
            graph.graph.replay()
            torch.cuda.synchronize()
            replays.append((graph.hidden_buf.clone(), graph.cfg_logits_buf.clone()))
        _restore(graph, snap)
        for i in range(3):
            graph.set_step(_ids(graph, 20 + i), pads, pos0 + i)
            with torch.no_grad():
                graph._decode_step()
            torch.cuda.synchronize()
            assert torch.equal(graph.hidden_buf.view(torch.int16), replays[i][0].view(torch.int16)), f"replay {i}"
            assert torch.equal(graph.cfg_logits_buf, replays[i][1]), f"replay {i} logits"
    finally:
        backbone.uninstall(_CapturedGraph)
