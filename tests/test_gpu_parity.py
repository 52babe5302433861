"""GPU parity of the HIP decode attention (libbz_gqa_decode.so, called through its C ABI) against the CPU oracle.

Tolerance (north star): |out - ref| <= 2e-3 + 1e-2 * |ref| elementwise on the bf16 output, ref = the float64
oracle (oracle.attention.decode_attention). Range / split coverage is checked exactly through closed forms.
"""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import gqa_decode, gqa_decode_masked, attn_decode, workloads
from oracle.attention import decode_attention, interval_mask

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def assert_close(got, ref, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    excess = np.abs(got - ref) - (ATOL + RTOL * np.abs(ref))
    i = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess.max() <= 0, f"{what}: worst {i}: got {got[i]!r} ref {ref[i]!r} (excess {excess.max():.3e})"


def oracle(w, kv_start=None, mask=None, q=None, lens=None):
    q = w.q if q is None else q
    lens = w.seq_lens if lens is None else lens
    return decode_attention(q.float().numpy(), w.k.float().numpy(), w.v.float().numpy(), lens.numpy(), w.scale,
                            kv_start=None if kv_start is None else np.asarray(kv_start), mask=mask)


def rand_case(seed, B, NH, NKV, D, cap, lens, starts=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, NH, D, generator=g).bfloat16()
    k = torch.randn(B, NKV, cap, D, generator=g).bfloat16()
    v = torch.randn(B, NKV, cap, D, generator=g).bfloat16()
    w = workloads.Workload(0, B, NH, NKV, D, cap, q, k, v, torch.tensor(lens, dtype=torch.int32), D ** -0.5)
    return w, (None if starts is None else torch.tensor(starts, dtype=torch.int32))


# ---------------------------------------------------------------------------------------------- BASELINE configs

@pytest.mark.parametrize("cfg", [1, 2, 3, 4])
@pytest.mark.parametrize("combine", ["last_block", "kernel"])
def test_config_parity(device, cfg, combine):
    w = workloads.make(cfg)
    print(f"config {cfg} {workloads.NAMES[cfg]} combine={combine}", flush=True)
    ref = oracle(w)
    g = w.to(device)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, combine=combine)
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), ref, f"config {cfg}")


@pytest.mark.parametrize("splits", [1, 3, 16, 32, 64, 128])
def test_config3_split_counts(device, splits):
    w = workloads.make(3)
    ref = oracle(w)
    g = w.to(device)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, num_splits=splits)
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), ref, f"config 3 splits={splits}")


def test_config5_depth_frame(device):
    w = workloads.make(5)
    g = w.to(device)
    outs = []
    for step in range(w.q.shape[0]):
        outs.append(gqa_decode(g.q[step], g.k, g.v, g.seq_lens[step], g.scale))
    torch.cuda.synchronize()
    for step, out in enumerate(outs):
        assert_close(out.float().cpu(), oracle(w, q=w.q[step], lens=w.seq_lens[step]), f"depth step {step}")


def test_real_depth_shape(device):
    # the reference's depth transformer: 8 q / 2 KV heads (G = 4), head_dim 128, <= 16 positions
    w, _ = rand_case(55, 2, 8, 2, 128, 17, [1, 1])
    g = w.to(device)
    for L in range(1, 17):
        lens = torch.tensor([L, L], dtype=torch.int32)
        out = gqa_decode(g.q, g.k, g.v, lens.to(device), g.scale)
        torch.cuda.synchronize()
        assert_close(out.float().cpu(), oracle(w, lens=lens), f"depth L={L}")


# ---------------------------------------------------------------------------------------------- shapes and ranges

@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("NH,NKV", [(8, 8), (16, 8), (16, 4), (16, 2), (32, 4)])
def test_group_sizes(device, D, NH, NKV):
    w, st = rand_case(100 + NH + NKV + D, 3, NH, NKV, D, 700, [700, 333, 64], [0, 11, 0])
    g = w.to(device)
    for combine in ("last_block", "kernel"):
        out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device), combine=combine)
        torch.cuda.synchronize()
        assert_close(out.float().cpu(), oracle(w, kv_start=st), f"G={NH // NKV} D={D} {combine}")


EDGE_LENS = [0, 1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 257, 1000, 1023, 2047, 2048]


@pytest.mark.parametrize("splits", [0, 1, 2, 7, 32, 100])
def test_edge_lengths(device, splits):
    B = len(EDGE_LENS)
    starts = [(3 * i) % 5 if EDGE_LENS[i] > 5 else 0 for i in range(B)]
    w, st = rand_case(7 + splits, B, 16, 8, 128, 2048, EDGE_LENS, starts)
    g = w.to(device)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device), num_splits=splits)
    torch.cuda.synchronize()
    got = out.float().cpu()
    assert_close(got, oracle(w, kv_start=st), f"edge lengths splits={splits}")
    assert torch.all(got[0] == 0)  # empty row -> 0


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("splits", [0, 1, 3, 8, 33, 64])
def test_split_boundaries_exact(device, D, splits):
    """q = 0 -> uniform weights; V[p] is a one-hot at dim p % D, so out[d] = (#positions p in range with
    p % D == d) / len: a dropped or doubled position changes some out[d] by >= 1/len."""
    NH, NKV, cap = 16, 8, 4096
    cases = [(0, 1), (0, D), (5, 5 + D - 1), (100, 100 + D), (0, 4096), (17, 4000), (1, 2), (64, 1089), (3, 1234)]
    B = len(cases)
    q = torch.zeros(B, NH, D, dtype=torch.bfloat16)
    k = torch.randn(B, NKV, cap, D, generator=torch.Generator().manual_seed(3)).bfloat16()
    pos = torch.arange(cap)
    v = torch.zeros(B, NKV, cap, D, dtype=torch.bfloat16)
    v[:, :, pos, pos % D] = 1.0
    st = torch.tensor([c[0] for c in cases], dtype=torch.int32)
    en = torch.tensor([c[1] for c in cases], dtype=torch.int32)
    out = gqa_decode(q.to(device), k.to(device), v.to(device), en.to(device), D ** -0.5, kv_start=st.to(device),
                     num_splits=splits)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for b, (s, e) in enumerate(cases):
        counts = np.bincount(np.arange(s, e) % D, minlength=D) / (e - s)
        assert_close(got[b], np.broadcast_to(counts, (NH, D)), f"range [{s},{e}) splits={splits}")


def test_single_position_is_exact(device):
    w, _ = rand_case(9, 4, 16, 8, 128, 300, [1, 51, 300, 8], [0, 50, 299, 7])
    st = torch.tensor([0, 50, 299, 7], dtype=torch.int32)
    g = w.to(device)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device))
    torch.cuda.synchronize()
    heads = torch.arange(16) // 2
    for b in range(4):
        assert torch.equal(out[b].cpu().view(torch.int16), w.v[b, heads, int(st[b])].view(torch.int16))


def test_dominant_key(device):
    w, _ = rand_case(13, 2, 16, 8, 128, 1500, [1500, 1400])
    k = w.k.float()
    for b in range(2):
        for kvh in range(8):
            qd = w.q[b, 2 * kvh:2 * kvh + 2].float().sum(0)
            k[b, kvh, 777] = 40.0 * qd / qd.norm()
    w.k = k.bfloat16()
    g = w.to(device)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, 1.0)
    torch.cuda.synchronize()
    w.scale = 1.0
    assert_close(out.float().cpu(), oracle(w), "dominant key")


def test_nan_outside_range_never_leaks(device):
    w, st = rand_case(17, 4, 16, 8, 128, 1024, [1000, 513, 64, 1024], [10, 0, 33, 0])
    clean = gqa_decode(*[t.to(device) for t in (w.q, w.k, w.v, w.seq_lens)], w.scale, kv_start=st.to(device))
    k, v = w.k.clone(), w.v.clone()
    for b in range(4):
        k[b, :, :int(st[b])] = float("nan")
        v[b, :, :int(st[b])] = float("inf")
        k[b, :, int(w.seq_lens[b]):] = float("inf")
        v[b, :, int(w.seq_lens[b]):] = float("nan")
    dirty = gqa_decode(w.q.to(device), k.to(device), v.to(device), w.seq_lens.to(device), w.scale,
                       kv_start=st.to(device))
    torch.cuda.synchronize()
    assert torch.equal(clean.cpu().view(torch.int16), dirty.cpu().view(torch.int16))
    assert_close(dirty.float().cpu(), oracle(w, kv_start=st), "nan tails")


def test_out_of_range_lengths_are_clamped(device):
    # seq_lens beyond capacity clamp to capacity; negative lengths / start > end give empty rows (output 0)
    w, _ = rand_case(19, 4, 16, 8, 128, 256, [256, 256, 0, 256])
    lens = torch.tensor([10_000, -5, 100, 256], dtype=torch.int32)
    st = torch.tensor([0, 0, 200, -7], dtype=torch.int32)
    g = w.to(device)
    out = gqa_decode(g.q, g.k, g.v, lens.to(device), g.scale, kv_start=st.to(device)).float().cpu()
    torch.cuda.synchronize()
    ref = oracle(w, kv_start=[0, 0, 100, 0], lens=torch.tensor([256, 0, 100, 256], dtype=torch.int32))
    assert_close(out, ref, "clamped")
    assert torch.all(out[1] == 0) and torch.all(out[2] == 0)


# ---------------------------------------------------------------------------------------------- determinism

def test_deterministic_and_mode_independent(device):
    w = workloads.make(2)
    g = w.to(device)
    outs = [gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, combine=c).cpu().view(torch.int16)
            for c in ("last_block", "last_block", "kernel", "last_block", "kernel")]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_split_count_invariance(device):
    w = workloads.make(2)
    g = w.to(device)
    ref = oracle(w)
    outs = {s: gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, num_splits=s).float().cpu().numpy()
            for s in (1, 2, 5, 16, 31, 64, 256)}
    torch.cuda.synchronize()
    for s, o in outs.items():
        assert_close(o, ref, f"splits={s}")
        assert np.abs(o - outs[1]).max() <= 2 * 2 ** -7 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("D,cap", [(128, 128), (128, 136), (64, 256), (64, 264)])
def test_one_split_up_to_64_kib(device, D, cap):
    """The default split count is 1 while a row's K+V span (cap x 4 D bytes) is at most 64 KiB, several above; either
    way the default call matches the oracle and the explicit one-split call within tolerance."""
    from breeze_tts_2_flash_amd import default_splits

    one = cap * 4 * D <= 64 * 1024
    assert (default_splits(2, 8, D, cap) == 1) == one
    assert default_splits(16, 8, D, cap) == 1 or not one
    w, st = rand_case(cap + D, 2, 16, 8, D, cap, [cap, cap - 3], starts=[0, 2])
    g = w.to(device)
    starts = st.to(device)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=starts).float().cpu().numpy()
    out1 = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=starts, num_splits=1).float().cpu().numpy()
    torch.cuda.synchronize()
    ref = oracle(w, kv_start=[0, 2])
    assert_close(out, ref, f"D={D} cap={cap} default")
    assert_close(out1, ref, f"D={D} cap={cap} one split")
    if one:
        assert np.array_equal(out, out1)


def test_short_rows_run_as_one_split_in_a_wide_grid(device):
    """A grid sized for the capacity (16 splits) runs a row whose K+V span is at most 64 KiB (128 positions at head_dim
    128) as one chunk: bit-identical to the one-split launch. Longer rows in the same call are split and stay within
    tolerance of the oracle."""
    lens, starts = [100, 128, 129, 1500], [0, 0, 0, 37]
    w, st = rand_case(131, 4, 16, 8, 128, 2048, lens, starts)
    g = w.to(device)
    wide = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device), num_splits=16)
    one = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device), num_splits=1)
    torch.cuda.synchronize()
    assert torch.equal(wide[:2].view(torch.int16), one[:2].view(torch.int16))
    assert_close(wide.float().cpu(), oracle(w, kv_start=st), "wide grid")


# ---------------------------------------------------------------------------------------------- masks / compat

@pytest.mark.parametrize("mdtype", [torch.bfloat16, torch.float32])
def test_interval_mask_attn_decode(device, mdtype):
    """The reference's call form: attn_decode with its left-padded interval mask (backbone_graph.py:239-252)."""
    B, NH, NKV, D, cap = 4, 16, 8, 128, 2048
    w, _ = rand_case(23, B, NH, NKV, D, cap, [cap] * B)
    pad = [0, 37, 5, 500]
    position = 1300
    mask = interval_mask(pad, position, cap, mdtype)
    out = torch.full((B, 1, NH, D), 7.0, dtype=torch.bfloat16, device=device)
    scores = cmax = part = counters = None
    ret = attn_decode(w.q[:, :, None].to(device), w.k.to(device), w.v.to(device), mask.to(device), w.scale,
                      scores, cmax, part, counters, out)
    torch.cuda.synchronize()
    assert ret is out
    ref = oracle(w, kv_start=pad, lens=torch.full((B,), position + 1, dtype=torch.int32))
    assert_close(out[:, 0].float().cpu(), ref, f"attn_decode {mdtype}")


def test_general_mask_values_and_holes(device):
    """Finite mask values are added to the scores; a hole (<= -1e30) inside the range is excluded even when V holds
    NaN there; a broadcast (batch-1) mask row serves every batch row."""
    B, NH, NKV, D, cap = 3, 16, 8, 64, 600
    w, _ = rand_case(29, B, NH, NKV, D, cap, [600, 450, 7])
    g = torch.Generator().manual_seed(5)
    m = (torch.randn(B, 1, 1, cap, generator=g) * 2.0).float()
    m[:, :, :, 100:140] = torch.finfo(torch.float32).min
    m[2, :, :, 3] = float("-inf")
    w.v[:, :, 100:140] = float("nan")
    w.v[2, :, 3] = float("nan")
    gd = w.to(device)
    out = gqa_decode(gd.q, gd.k, gd.v, gd.seq_lens, gd.scale, mask=m.to(device))
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), oracle(w, mask=m.numpy().reshape(B, cap)), "general mask")
    mb = m[:1].bfloat16()
    mb[..., 3] = torch.finfo(torch.bfloat16).min  # row 2's NaN V at position 3 is excluded for every row
    out = gqa_decode(gd.q, gd.k, gd.v, gd.seq_lens, gd.scale, mask=mb.to(device))
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), oracle(w, mask=mb.float().numpy().reshape(1, cap)), "broadcast bf16 mask")
    # masked entry point: interval from the same mask (first..last > -1e30), holes still excluded
    out = gqa_decode_masked(gd.q, gd.k, gd.v, m.to(device), gd.scale)
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), oracle(w, mask=m.numpy().reshape(B, cap), lens=torch.full((B,), cap)),
                 "masked entry")


def test_fully_masked_row_is_zero(device):
    w, _ = rand_case(31, 2, 16, 8, 128, 128, [128, 128])
    m = torch.zeros(2, 1, 1, 128, dtype=torch.bfloat16)
    m[1] = torch.finfo(torch.bfloat16).min
    g = w.to(device)
    out = gqa_decode_masked(g.q, g.k, g.v, m.to(device), g.scale).float().cpu()
    torch.cuda.synchronize()
    assert torch.all(out[1] == 0)
    assert_close(out[0], oracle(w)[0], "unmasked row")


def test_strided_query_and_reference_out_layout(device):
    """q as a view into a fused qkv projection buffer [B, (NH + 2 NKV) D] and out in [B, 1, NH, D] (the
    reference's layout, flash/backbone.py:91-92, :122-125)."""
    B, NH, NKV, D, cap = 2, 16, 8, 128, 2048
    w, _ = rand_case(37, B, NH, NKV, D, cap, [1024, 999])
    qkv = torch.randn(B, (NH + 2 * NKV) * D).bfloat16()
    qkv[:, :NH * D] = w.q.reshape(B, NH * D)
    qv = qkv.to(device)[:, :NH * D].view(B, NH, D)
    assert not qv.is_contiguous() or qv.stride(0) == (NH + 2 * NKV) * D
    out = torch.empty(B, 1, NH, D, dtype=torch.bfloat16, device=device)
    gqa_decode(qv, w.k.to(device), w.v.to(device), w.seq_lens.to(device), w.scale, out=out)
    torch.cuda.synchronize()
    assert_close(out[:, 0].float().cpu(), oracle(w), "strided q")


def test_workspace_shared_across_calls_stays_clean(device):
    # the last-block counters reset themselves: many calls with changing lengths on one workspace stay correct
    w, _ = rand_case(41, 2, 16, 8, 128, 2048, [2048, 2048])
    g = w.to(device)
    for L in (2048, 1, 700, 64, 2000, 33, 1024):
        lens = torch.tensor([L, max(1, L // 2)], dtype=torch.int32)
        out = gqa_decode(g.q, g.k, g.v, lens.to(device), g.scale, num_splits=32)
        torch.cuda.synchronize()
        assert_close(out.float().cpu(), oracle(w, lens=lens), f"L={L}")


def test_hip_graph_replay(device):
    """Recorded into a HIP graph (torch.cuda.CUDAGraph): lengths change on the device between replays; every
    replay matches an eager call made between replays."""
    w, _ = rand_case(43, 2, 16, 8, 128, 2048, [1024, 1024])
    g = w.to(device)
    lens = g.seq_lens.clone()
    out = torch.empty(2, 16, 128, dtype=torch.bfloat16, device=device)
    gqa_decode(g.q, g.k, g.v, lens, g.scale, out=out)  # warm-up: workspace allocated outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gqa_decode(g.q, g.k, g.v, lens, g.scale, out=out)
    for L in (1024, 100, 2048, 1, 1500, 1024):
        lens.copy_(torch.tensor([L, max(1, L - 3)], dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = gqa_decode(g.q, g.k, g.v, lens, g.scale)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), f"replay L={L}"
        assert_close(got.float().cpu(), oracle(w, lens=lens.cpu()), f"replay L={L}")


def test_argument_errors(device):
    w, _ = rand_case(47, 2, 16, 8, 128, 64, [64, 64])
    g = w.to(device)
    with pytest.raises(RuntimeError, match="bf16"):
        gqa_decode(g.q.float(), g.k, g.v, g.seq_lens, g.scale)
    with pytest.raises(RuntimeError, match="int32"):
        gqa_decode(g.q, g.k, g.v, g.seq_lens.long(), g.scale)
    with pytest.raises(RuntimeError, match="unsupported"):
        q96 = torch.zeros(2, 16, 96, dtype=torch.bfloat16, device=device)
        kv96 = torch.zeros(2, 8, 64, 96, dtype=torch.bfloat16, device=device)
        gqa_decode(q96, kv96, kv96, g.seq_lens, 0.1)
    out = torch.zeros(2, 1, 16, 128, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError, match="dbg"):  # a dbg buffer smaller than B * NH * S, checked before any launch
        attn_decode(g.q[:, :, None], g.k, g.v, torch.zeros(2, 1, 1, 64, device=device), 0.1, None, None, None, None,
                    out, dbg=torch.empty(1, device=device))
    torch.cuda.synchronize()
    assert not out.any(), "attn_decode ran before refusing its dbg buffer"


# ---------------------------------------------------------------------------------------------- golden fixtures

def test_golden_fixtures(device):
    """The committed fixtures (tests/golden/decode_attention.npz), through gqa_decode and, for the masked case, also
    through the interval-mask entry point."""
    from tests.golden.make_golden import load

    for name, c in sorted(load().items()):
        t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)  # noqa: E731
        q, k, v = t(c["q"]), t(c["k"]), t(c["v"])
        lens = torch.from_numpy(c["lens"]).to(device)
        starts = torch.from_numpy(c["starts"]).to(device)
        mask = t(c["mask"]) if "mask" in c else None
        out = gqa_decode(q, k, v, lens, float(c["scale"]), kv_start=starts, mask=mask)
        torch.cuda.synchronize()
        assert_close(out.float().cpu(), c["out"], f"golden {name}")
        if mask is not None:
            out2 = gqa_decode_masked(q, k, v, mask, float(c["scale"]))
            torch.cuda.synchronize()
            assert_close(out2.float().cpu(), c["out"], f"golden {name} (masked entry)")


def test_concurrent_streams_and_threads(device):
    """Two host threads, each on its own stream with the default (per-stream) workspace, run decode calls at the same
    time on different data; every output matches the oracle (the op is stateless; the split counters and partials
    are per stream)."""
    import threading

    cases = [rand_case(60 + i, 2, 16, 8, 128, 2048, [1500 - 300 * i, 900 + 100 * i]) for i in range(2)]
    outs = [None, None]
    errors = []

    def worker(i):
        try:
            w, _ = cases[i]
            s = torch.cuda.Stream(device=device)
            with torch.cuda.stream(s):
                g = w.to(device)
                for _ in range(50):
                    o = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale)
                s.synchronize()
                outs[i] = o.float().cpu()
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for i in range(2):
        assert_close(outs[i], oracle(cases[i][0]), f"stream {i}")


@pytest.mark.parametrize("splits,combine", [(0, "auto"), (1, "auto"), (7, "auto"), (256, "auto"), (256, "last_block")])
def test_long_context(device, splits, combine):
    """A 32768-slot cache: a full row and a left-padded partial one, the default split count (chunks capped at 256
    positions), one workgroup streaming 32768 positions in 512 tiles, a ragged 7-way split, and the largest split
    count (256). At 256 splits the grid is 2 x 8 x 256 = 4096 workgroups, more than the GPU holds at once (256 CUs,
    at most 5 of these workgroups each), and the splits are still merged inside the one launch: no workgroup waits for
    another, the last of each (row, kv head) to count in merges."""
    lens, starts = [32768, 20001], [0, 5]
    w, st = rand_case(31 + splits, 2, 16, 8, 128, 32768, lens, starts)
    g = w.to(device)
    out = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=st.to(device), num_splits=splits, combine=combine)
    torch.cuda.synchronize()
    assert_close(out.float().cpu(), oracle(w, kv_start=st), f"long context splits={splits} combine={combine}")
