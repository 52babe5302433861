"""GPU: the cross-workgroup merge under back-to-back calls at full size.

Hundreds of calls are captured into one HIP graph, cycling over K/V sets that hold different data and different row
lengths (so consecutive calls on the one workspace run different split counts, including one-split rows that skip the
merge), each call writing an output slot of its own. The graph is replayed several times and every output must equal,
bit for bit, a direct call on the same set made beforehand with a synchronisation around it. The merge is
deterministic (split order), so any partial or arrival counter left over from the previous call, or read before it
landed, shows as a difference. Covered: the default last-block merge at the serving shape (B2, 16/8, D128, capacity
2048) and the ragged batch (B16), the second merge kernel, the interval-mask entry and the fused step.
"""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import gqa_decode, gqa_decode_fused, gqa_decode_masked, workspace_bytes

pytestmark = pytest.mark.gpu

CALLS = 240       # calls per graph
REPLAYS = 4


def _bits(t):
    return t.view(torch.int16)


def _sets(device, B, NKV, G, D, cap, lens_per_set, seed):
    gen = torch.Generator().manual_seed(seed)
    sets = []
    for lens in lens_per_set:
        q = torch.randn(B, NKV * G, D, generator=gen).bfloat16().to(device)
        k = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(device)
        v = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(device)
        sl = torch.tensor(lens, dtype=torch.int32, device=device)
        sets.append((q, k, v, sl))
    return sets


def _interval_mask(lens, starts, cap, device):
    m = torch.full((len(lens), 1, 1, cap), torch.finfo(torch.bfloat16).min, dtype=torch.bfloat16)
    for b, (s, e) in enumerate(zip(starts, lens)):
        m[b, 0, 0, s:e] = 0
    return m.to(device)


def _check(device, run, nsets, out_shape):
    """run(i, out): call i (set i % nsets) into out. References first (direct, synchronised), then the graph."""
    refs = []
    for j in range(nsets):
        o = torch.empty(out_shape, dtype=torch.bfloat16, device=device)
        run(j, o)
        torch.cuda.synchronize()
        refs.append(o.clone())
    # consecutive sets give different outputs, so a result carried over from the previous call cannot pass
    for j in range(nsets):
        assert not torch.equal(_bits(refs[j]), _bits(refs[(j + 1) % nsets])), f"sets {j} and {j + 1} agree"
    outs = torch.empty((CALLS,) + tuple(out_shape), dtype=torch.bfloat16, device=device)
    run(0, outs[0])  # warm the stream's workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(CALLS):
            run(i, outs[i])
    for rep in range(REPLAYS):
        outs.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        bad = [i for i in range(CALLS) if not torch.equal(_bits(outs[i]), _bits(refs[i % nsets]))]
        print(f"replay {rep}: {len(bad)} of {CALLS} calls differ", flush=True)
        assert not bad, f"replay {rep}: calls {bad[:10]} differ from their direct calls"


SERVING_LENS = [[1024, 1024], [700, 1333], [2048, 1900], [100, 60], [33, 2048], [1500, 1], [0, 999], [1024, 512]]


def _workspace(device, B, NH, NKV, D, cap):
    return torch.zeros(workspace_bytes(B, NH, NKV, D, cap), dtype=torch.uint8, device=device)


# workspace "explicit": one caller workspace for the references and the graph; "none": the references use the
# stream's cached workspace and the captured calls the library's static scratch (bz_gqa_decode_noalloc)
@pytest.mark.parametrize("combine,ws_mode", [("auto", "explicit"), ("auto", "none"), ("kernel", "explicit")])
def test_serving_shape_back_to_back(device, combine, ws_mode):
    sets = _sets(device, 2, 8, 2, 128, 2048, SERVING_LENS, seed=71)
    ws = _workspace(device, 2, 16, 8, 128, 2048) if ws_mode == "explicit" else None
    print(f"B2 16/8 D128 cap 2048, {len(sets)} sets, combine={combine}, workspace {ws_mode}", flush=True)

    def run(i, out):
        q, k, v, sl = sets[i % len(sets)]
        gqa_decode(q, k, v, sl, 128 ** -0.5, out, combine=combine, workspace=ws)

    _check(device, run, len(sets), (2, 16, 128))


def test_ragged_batch_back_to_back(device):
    rng = np.random.default_rng(72)
    lens = [rng.integers(0, 2049, size=16).tolist() for _ in range(6)]
    sets = _sets(device, 16, 8, 2, 128, 2048, lens, seed=72)
    ws = _workspace(device, 16, 16, 8, 128, 2048)
    print("B16 16/8 D128 cap 2048, 6 ragged sets", flush=True)

    def run(i, out):
        q, k, v, sl = sets[i % len(sets)]
        gqa_decode(q, k, v, sl, 128 ** -0.5, out, workspace=ws)

    _check(device, run, len(sets), (16, 16, 128))


def test_masked_entry_back_to_back(device):
    starts_per_set = [[0, 7], [250, 0], [0, 0], [40, 13], [5, 900], [0, 0], [0, 0], [300, 100]]
    sets = _sets(device, 2, 8, 2, 128, 2048, SERVING_LENS, seed=73)
    masks = [_interval_mask([max(e, s) for e, s in zip(lens, st)], st, 2048, device)
             for lens, st in zip(SERVING_LENS, starts_per_set)]
    ws = _workspace(device, 2, 16, 8, 128, 2048)
    print("interval-mask entry, B2 16/8 D128 cap 2048, 8 sets", flush=True)

    def run(i, out):
        q, k, v, _ = sets[i % len(sets)]
        gqa_decode_masked(q, k, v, masks[i % len(sets)], 128 ** -0.5, out, workspace=ws)

    _check(device, run, len(sets), (2, 16, 128))


def test_fused_step_back_to_back(device):
    B, NH, NKV, D, cap = 2, 16, 8, 128, 2048
    sets = _sets(device, B, NKV, 2, D, cap, SERVING_LENS[:6], seed=74)
    gen = torch.Generator().manual_seed(75)
    extra = []
    for _, _, _, sl in sets:
        L = int(sl.max().item())
        qkv = (torch.randn(B, (NH + 2 * NKV) * D, generator=gen) * 3).bfloat16().to(device)
        ang = torch.randn(B, D, generator=gen)
        pos = torch.tensor([max(L - 1, 0)], dtype=torch.int64, device=device)
        extra.append((qkv, ang.cos().bfloat16().to(device), ang.sin().bfloat16().to(device), pos))
    qn = (1 + 0.2 * torch.randn(D, generator=gen)).bfloat16().to(device)
    kn = (1 + 0.2 * torch.randn(D, generator=gen)).bfloat16().to(device)
    ws = _workspace(device, B, NH, NKV, D, cap)
    print("fused step, B2 16/8 D128 cap 2048, 6 sets (each call rewrites its slot with the same values)", flush=True)

    def run(i, out):
        _, k, v, sl = sets[i % len(sets)]
        qkv, cos, sin, pos = extra[i % len(sets)]
        gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, k, v, pos, D ** -0.5, out, seq_lens=sl, workspace=ws)

    # the first direct call writes each set's slot; the reference is the second, made on the settled cache
    for i in range(len(sets)):
        run(i, torch.empty(B, NH, D, dtype=torch.bfloat16, device=device))
    torch.cuda.synchronize()
    _check(device, run, len(sets), (B, NH, D))
