"""The workspace contract of bz_gqa_decode on the GPU: a workspace starts with one arrival counter per (row, kv head),
which every call leaves at zero, and the rest (the split partials) is written before it is read. One zero-filled
workspace therefore serves every call with the same rows * kv heads, whatever its split count, length, mask or
entry point.

Tolerance as in test_gpu_parity: |out - ref| <= 2e-3 + 1e-2 * |ref| against the float64 oracle.
"""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import attention, gqa_decode, gqa_decode_fused, gqa_decode_masked, workspace_bytes
from oracle.attention import interval_mask
from tests.test_gpu_parity import assert_close, oracle, rand_case

pytestmark = pytest.mark.gpu

COUNTER_BYTES = 256  # one 256-byte line per (row, kv head) at the start of the workspace


def _counters_clear(ws, groups, what):
    torch.cuda.synchronize()
    nz = int(torch.count_nonzero(ws[:groups * COUNTER_BYTES]))
    assert nz == 0, f"{what}: {nz} counter bytes left nonzero"


def test_alternating_split_counts_on_one_workspace(device):
    """num_splits 32 and 8 (and the default) in turn on one workspace, with lengths that change every call: the
    partial slots of one layout overlap the other's, and the counters stay in place and at zero."""
    w, _ = rand_case(71, 2, 16, 8, 128, 2048, [2048, 2048])
    g = w.to(device)
    ws = torch.zeros(workspace_bytes(2, 16, 8, 128, 2048, 32), dtype=torch.uint8, device=device)
    for i, (splits, L) in enumerate([(32, 2048), (8, 1500), (32, 700), (0, 1024), (8, 2048), (32, 65), (8, 333)]):
        print(f"call {i}: splits={splits} L={L}", flush=True)
        lens = torch.tensor([L, max(1, L - 17)], dtype=torch.int32)
        out = gqa_decode(g.q, g.k, g.v, lens.to(device), g.scale, num_splits=splits, workspace=ws)
        _counters_clear(ws, 2 * 8, f"call {i}")
        assert_close(out.float().cpu(), oracle(w, lens=lens), f"call {i} splits={splits} L={L}")


@pytest.mark.parametrize("combine", ["last_block", "kernel"])
def test_entries_share_one_workspace(device, combine):
    """Plain, masked and fused calls, one after another on one workspace (same rows * kv heads), each correct and
    each leaving the counters at zero; the two-token causal step on a workspace of its own (twice the rows)."""
    B, NH, NKV, D, cap = 2, 16, 8, 128, 2048
    w, st = rand_case(73, B, NH, NKV, D, cap, [1800, 1700], [0, 9])
    g = w.to(device)
    ws = torch.zeros(workspace_bytes(B, NH, NKV, D, cap, 64), dtype=torch.uint8, device=device)
    kw = dict(combine=combine, workspace=ws)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device), num_splits=24, **kw)
    _counters_clear(ws, B * NKV, "plain")
    assert_close(out.float().cpu(), oracle(w, kv_start=st), "plain")

    mask = interval_mask([0, 9], 1699, cap).to(device)
    mask[0, 0, 0, 1700:1800] = 0.0  # row 0 attends [0, 1800)
    out = gqa_decode_masked(g.q, g.k, g.v, mask, g.scale, num_splits=40, **kw)
    _counters_clear(ws, B * NKV, "masked")
    ref = oracle(w, kv_start=np.array([0, 9]), lens=torch.tensor([1800, 1700], dtype=torch.int32),
                 mask=mask[:, 0, 0, :].float().cpu().numpy())
    assert_close(out.float().cpu(), ref, "masked")

    qkv = (torch.randn(B, (NH + 2 * NKV) * D, generator=torch.Generator().manual_seed(6)) * 2).bfloat16().to(device)
    ones = torch.ones(D, dtype=torch.bfloat16, device=device)
    cos = torch.ones(B, D, dtype=torch.bfloat16, device=device)
    sin = torch.zeros(B, D, dtype=torch.bfloat16, device=device)
    kc, vc = g.k.clone(), g.v.clone()
    pos = torch.tensor([1799], dtype=torch.int64, device=device)
    gqa_decode_fused(qkv, ones, ones, 1e-6, cos, sin, kc, vc, pos, g.scale, seq_lens=g.seq_lens, num_splits=16, **kw)
    _counters_clear(ws, B * NKV, "fused")

    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device), num_splits=24, **kw)
    _counters_clear(ws, B * NKV, "plain again")
    assert_close(out.float().cpu(), oracle(w, kv_start=st), "plain again")

    ws2 = torch.zeros(workspace_bytes(2 * B, NH, NKV, D, cap, 24), dtype=torch.uint8, device=device)
    q2 = torch.randn(B, NH, 2, D, generator=torch.Generator().manual_seed(5)).bfloat16()
    out = gqa_decode(q2.to(device), g.k, g.v, g.seq_lens, g.scale, num_splits=24, combine=combine, workspace=ws2)
    _counters_clear(ws2, 2 * B * NKV, "two tokens")
    for t in range(2):
        ref = oracle(w, q=q2[:, :, t], lens=w.seq_lens - (1 - t))
        assert_close(out[:, t].float().cpu(), ref, f"two tokens, token {t}")


def test_cached_workspace_stays_bounded(device):
    """The DynamicCache route: the key length grows by one every step. The cached workspace of the stream grows
    geometrically instead of one new workspace per length, and its counters stay at zero between calls."""
    B, NH, NKV, D = 2, 16, 8, 128
    g = torch.Generator().manual_seed(77)
    q = torch.randn(B, NH, D, generator=g).bfloat16().to(device)
    k = torch.randn(B, NKV, 1200, D, generator=g).bfloat16().to(device)
    v = torch.randn(B, NKV, 1200, D, generator=g).bfloat16().to(device)
    before = len(attention._WS) + len(attention._WS_RETIRED)
    for L in range(64, 1200, 7):
        kk, vv = k[:, :, :L].contiguous(), v[:, :, :L].contiguous()
        lens = torch.full((B,), L, dtype=torch.int32, device=device)
        gqa_decode(q, kk, vv, lens, D ** -0.5)
    torch.cuda.synchronize()
    grown = len(attention._WS) + len(attention._WS_RETIRED) - before
    assert grown <= 8, f"{grown} workspaces allocated over 163 growing lengths"
    ws = attention._WS[(device.index, torch.cuda.current_stream(device).cuda_stream, B * NKV)]
    _counters_clear(ws, B * NKV, "cached workspace")


def test_capture_without_workspace_allocates_nothing(device):
    """A call recorded into a HIP graph without a workspace runs on the library's static scratch
    (bz_gqa_decode_noalloc): the capture adds no cached workspace, and every replay, with eager calls of other sizes
    in between, equals the eager result bit for bit; the masked form likewise (its range comes from the mask)."""
    w, st = rand_case(79, 2, 16, 8, 128, 1024, [1000, 640], [0, 17])
    g = w.to(device)
    starts = st.to(device)
    mask = interval_mask([0, 17], 639, 1024).to(device)
    mask[0, 0, 0, 640:1000] = 0.0
    ref = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=starts, num_splits=16)
    ref_m = gqa_decode_masked(g.q, g.k, g.v, mask, g.scale, num_splits=16)
    out = torch.empty_like(ref)
    out_m = torch.empty_like(ref_m)
    keys = set(attention._WS)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, out, kv_start=starts, num_splits=16)
            gqa_decode_masked(g.q, g.k, g.v, mask, g.scale, out_m, num_splits=16)
    assert set(attention._WS) == keys, "the capture allocated a workspace"
    small = gqa_decode(g.q[:1], g.k[:1], g.v[:1], g.seq_lens[:1], g.scale, num_splits=8)
    for i in range(3):
        out.zero_()
        out_m.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
        assert torch.equal(out_m.view(torch.int16), ref_m.view(torch.int16)), f"replay {i} (masked)"
        again = gqa_decode(g.q[:1], g.k[:1], g.v[:1], g.seq_lens[:1], g.scale, num_splits=8)
        assert torch.equal(again.view(torch.int16), small.view(torch.int16)), f"eager call after replay {i}"


def _step_inputs(device, B=2, NH=16, NKV=8, D=128, cap=1024, L=700, seed=81):
    """Raw q | k | v projections, norm weights, RoPE tables, caches and the cache slot of one fused decode step."""
    gen = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(B, (NH + 2 * NKV) * D, generator=gen) * 2).bfloat16().to(device)
    qn = (1 + 0.2 * torch.randn(D, generator=gen)).bfloat16().to(device)
    kn = (1 + 0.2 * torch.randn(D, generator=gen)).bfloat16().to(device)
    ang = torch.linspace(0, 3, D)
    cos = ang.cos().bfloat16().expand(B, D).contiguous().to(device)
    sin = ang.sin().bfloat16().expand(B, D).contiguous().to(device)
    kc = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(device)
    vc = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(device)
    pos = torch.tensor([L - 1], dtype=torch.int64, device=device)
    lens = torch.full((B,), L, dtype=torch.int32, device=device)
    return qkv, qn, kn, cos, sin, kc, vc, pos, lens


def test_fused_capture_allocates_nothing(device):
    """The fused entry under capture: without workspace= it raises before launching anything (it has no static-scratch
    form, and a capture must not allocate); with a workspace made before the capture it records, allocates nothing,
    and every replay equals the eager step bit for bit (caches included)."""
    qkv, qn, kn, cos, sin, kc0, vc0, pos, lens = _step_inputs(device)
    kc, vc = kc0.clone(), vc0.clone()
    ref = gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc, vc, pos, 128 ** -0.5, seq_lens=lens)
    torch.cuda.synchronize()
    ref_k, ref_v = kc.clone(), vc.clone()
    ws = attention.get_workspace(device, 2, 16, 8, 128, 1024)
    out = torch.empty_like(ref)
    keys = set(attention._WS)
    kc2, vc2 = kc0.clone(), vc0.clone()
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="workspace"):
            with torch.cuda.graph(graph, stream=side):
                gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc2, vc2, pos, 128 ** -0.5, out, seq_lens=lens)
        torch.cuda.synchronize()
        assert set(attention._WS) == keys, "the refused capture allocated a workspace"
        before = torch.cuda.memory_allocated(device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc2, vc2, pos, 128 ** -0.5, out, seq_lens=lens,
                             workspace=ws)
        assert torch.cuda.memory_allocated(device) == before, "the capture allocated device memory"
    assert set(attention._WS) == keys, "the capture added a cached workspace"
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
        assert torch.equal(kc2.view(torch.int16), ref_k.view(torch.int16)), f"replay {i}: k cache"
        assert torch.equal(vc2.view(torch.int16), ref_v.view(torch.int16)), f"replay {i}: v cache"
        _counters_clear(ws, 2 * 8, f"replay {i}")


def test_reference_fused_entry_capture_allocates_nothing(device):
    """compat.attn_decode_fused, the entry the reference's decode step calls (flash/backbone.py:123-124), in the
    reference's capture sequence (backbone_graph.py:288-315): eager warm-up calls with the reference's workspaces, then
    a capture on a side stream. The capture allocates nothing (the warm-up made the library workspace this call's
    `counters` buffer keys) and every replay equals the eager step; a capture with a `counters` buffer never seen
    eagerly raises instead of allocating."""
    from breeze_tts_2_flash_amd import compat

    qkv, qn, kn, cos, sin, kc0, vc0, pos, lens = _step_inputs(device, seed=82)
    B, NH, NKV, D, cap, L = 2, 16, 8, 128, 1024, 700
    mask = interval_mask([0, 0], L - 1, cap).to(device)
    scores = torch.empty(B, NH, cap, device=device)
    cmax = torch.empty(B, NH, cap // 64, device=device)
    part = torch.empty(B, NH, cap // 64, D, device=device)
    counters = torch.zeros(B, NKV, 4, dtype=torch.int32, device=device)
    kc, vc = kc0.clone(), vc0.clone()
    ref = torch.empty(B, 1, NH, D, dtype=torch.bfloat16, device=device)
    for _ in range(3):  # the reference's warm-up steps
        kc.copy_(kc0)
        vc.copy_(vc0)
        compat.attn_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc, vc, mask, pos, D ** -0.5, scores, cmax, part,
                                 counters, ref)
    torch.cuda.synchronize()
    ref_k, ref_v = kc.clone(), vc.clone()
    kc2, vc2 = kc0.clone(), vc0.clone()
    out = torch.empty_like(ref)
    other = torch.zeros_like(counters)  # a reference workspace never seen eagerly
    ws_keys, lib_keys = set(compat._WS), set(attention._WS)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        # torch's graph machinery itself allocates 1 KiB at the first capture on a stream (an empty capture does it
        # too), so one empty capture comes first
        warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(warm, stream=side):
            pass
        before = torch.cuda.memory_allocated(device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            compat.attn_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc2, vc2, mask, pos, D ** -0.5, scores, cmax, part,
                                     counters, out)
        assert torch.cuda.memory_allocated(device) == before, "the capture allocated device memory"
        with pytest.raises(RuntimeError, match="eagerly"):
            with torch.cuda.graph(torch.cuda.CUDAGraph(), stream=side):
                compat.attn_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc2, vc2, mask, pos, D ** -0.5, scores, cmax,
                                         part, other, out)
        assert torch.cuda.memory_allocated(device) == before, "the refused capture allocated device memory"
    torch.cuda.synchronize()
    assert set(compat._WS) == ws_keys and set(attention._WS) == lib_keys, "the captures added a workspace"
    for i in range(3):
        out.zero_()
        kc2.copy_(kc0)
        vc2.copy_(vc0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
        assert torch.equal(kc2.view(torch.int16), ref_k.view(torch.int16)), f"replay {i}: k cache"
        assert torch.equal(vc2.view(torch.int16), ref_v.view(torch.int16)), f"replay {i}: v cache"


def test_capture_beyond_the_static_scratch_raises(device):
    """A non-fused call captured without workspace= whose sizes exceed the static scratch (more than 1024 (row, kv
    head) groups) raises rather than allocate a workspace inside the capture; with workspace= it records."""
    B, NH, NKV, D, cap = 160, 16, 8, 64, 128  # 1280 groups
    gen = torch.Generator().manual_seed(83)
    q = torch.randn(B, NH, D, generator=gen).bfloat16().to(device)
    k = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(device)
    v = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(device)
    lens = torch.full((B,), cap, dtype=torch.int32, device=device)
    ref = gqa_decode(q, k, v, lens, D ** -0.5, num_splits=2)
    ws = attention.get_workspace(device, B, NH, NKV, D, cap, 2)
    out = torch.empty_like(ref)
    keys = set(attention._WS)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        with pytest.raises(RuntimeError, match="SCRATCH|scratch"):
            with torch.cuda.graph(torch.cuda.CUDAGraph(), stream=side):
                gqa_decode(q, k, v, lens, D ** -0.5, out, num_splits=2)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            gqa_decode(q, k, v, lens, D ** -0.5, out, num_splits=2, workspace=ws)
    assert set(attention._WS) == keys, "a capture added a cached workspace"
    for i in range(2):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
