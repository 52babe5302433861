"""GPU parity of the one-wave-per-(row, q head) attention (bz_gqa_decode_wave through gqa_decode_wave; its wave is the device
function attend_wave of csrc/gqa_wave.cuh) against oracle.attention.decode_attention_tokens: head_dim 64 / 128 x
group sizes 1 / 2 / 4 / 8 over edge lengths (empty, one position, tile and two-tile boundaries, several hundred
positions) with non-zero starts; the depth transformer's shapes (the real 8 q / 2 KV heads at head_dim 128 and the
first step's two causal tokens; the head_dim-64 frame of 32 steps); NaN before the start and past the end; the golden
fixtures. Tolerance |out - ref| <= 2e-3 + 1e-2 |ref|, as for the split kernel."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import gqa_decode, gqa_decode_wave
from oracle.attention import decode_attention_tokens

pytestmark = pytest.mark.gpu

LENGTHS = [0, 1, 2, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 200]


def bf16(x, device):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).to(device)


def i32(x, device):
    return torch.tensor(x, dtype=torch.int32, device=device)


def check(got, q, k, v, lens, scale, starts=None, what=""):
    ref = decode_attention_tokens(q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                  np.asarray(lens), scale, kv_start=None if starts is None else np.asarray(starts))
    g = got.float().cpu().numpy()
    assert np.isfinite(g).all(), what
    excess = np.abs(g - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert excess.max() <= 0, f"{what}: excess {excess.max():.3e}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_lengths_and_groups(device, D, G):
    rng = np.random.default_rng(D * 10 + G)
    NKV, cap = 2, 256
    B = len(LENGTHS)
    q = bf16(rng.standard_normal((B, NKV * G, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    starts = [min(3 * i, L) for i, L in enumerate(LENGTHS)]
    ends = [s + L for s, L in zip(starts, LENGTHS)]
    out = gqa_decode_wave(q, k, v, i32(ends, device), D ** -0.5, kv_start=i32(starts, device))
    torch.cuda.synchronize()
    check(out[:, None], q[:, :, None], k, v, ends, D ** -0.5, starts, f"D={D} G={G}")
    empty = LENGTHS.index(0)
    assert (out[empty].float() == 0).all()
    one = LENGTHS.index(1)
    for h in range(NKV * G):  # one position: the output is its V row, bit for bit
        assert torch.equal(out[one, h], v[one, h // G, starts[one]])


def test_depth_first_step_tokens(device):
    rng = np.random.default_rng(41)
    B, T, NH, NKV, D, cap = 2, 2, 8, 2, 128, 16
    qb = bf16(rng.standard_normal((B * T, NH * D)), device)
    q = qb.view(B, T, NH, D).permute(0, 2, 1, 3)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    out = gqa_decode_wave(q, k, v, i32([2, 2], device), D ** -0.5)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (B, T, NH, D)
    check(out, q, k, v, [2, 2], D ** -0.5, what="depth step 0")
    for h in range(NH):
        assert torch.equal(out[:, 0, h], v[:, h // 4, 0])


@pytest.mark.parametrize("L", [1, 5, 16, 17])
def test_real_depth_shape(device, L):
    rng = np.random.default_rng(L)
    B, NH, NKV, D, cap = 2, 8, 2, 128, 17
    q = bf16(rng.standard_normal((B, NH, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    out = gqa_decode_wave(q, k, v, i32([L, L], device), D ** -0.5)
    torch.cuda.synchronize()
    check(out[:, :, None].transpose(1, 2), q[:, :, None], k, v, [L, L], D ** -0.5, what=f"depth L={L}")


def test_config5_frame_matches_split_kernel_within_tolerance(device):
    # the head_dim-64 depth frame: 32 sequential steps over lengths 1..32, each against the oracle and the split kernel
    rng = np.random.default_rng(5)
    B, NH, NKV, D, cap = 2, 16, 8, 64, 32
    q = bf16(rng.standard_normal((32, B, NH, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    for s in range(32):
        lens = i32([s + 1] * B, device)
        out = gqa_decode_wave(q[s], k, v, lens, D ** -0.5)
        split = gqa_decode(q[s], k, v, lens, D ** -0.5)
        torch.cuda.synchronize()
        check(out[:, :, None].transpose(1, 2), q[s][:, :, None], k, v, [s + 1] * B, D ** -0.5, what=f"step {s}")
        assert (out.float() - split.float()).abs().max().item() <= 2e-2


def test_nan_outside_the_range(device):
    rng = np.random.default_rng(9)
    B, NH, NKV, D, cap = 2, 16, 8, 128, 128
    q = bf16(rng.standard_normal((B, NH, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    starts, ends = [5, 40], [37, 101]
    clean = gqa_decode_wave(q, k, v, i32(ends, device), D ** -0.5, kv_start=i32(starts, device))
    kn, vn = k.clone(), v.clone()
    for b in range(B):
        for t in (kn, vn):
            t[b, :, :starts[b]] = float("nan")
            t[b, :, ends[b]:] = float("nan")
    dirty = gqa_decode_wave(q, kn, vn, i32(ends, device), D ** -0.5, kv_start=i32(starts, device))
    torch.cuda.synchronize()
    assert torch.equal(clean.view(torch.int16), dirty.view(torch.int16))


def test_golden_fixtures(device):
    """The unmasked cases of tests/golden/decode_attention.npz and the several-token cases of fused_and_tokens.npz."""
    from tests.golden.make_golden import OUT, OUT2, load

    cases = [(n, c) for n, c in sorted(load(OUT).items()) if "mask" not in c]
    cases += [(n, c) for n, c in sorted(load(OUT2).items()) if n.startswith("tokens")]
    assert len(cases) == 5
    for name, c in cases:
        t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)  # noqa: E731
        out = gqa_decode_wave(t(c["q"]), t(c["k"]), t(c["v"]), torch.from_numpy(c["lens"]).to(device),
                              float(c["scale"]), kv_start=torch.from_numpy(c["starts"]).to(device))
        torch.cuda.synchronize()
        excess = np.abs(out.float().cpu().numpy() - c["out"]) - (2e-3 + 1e-2 * np.abs(c["out"]))
        assert excess.max() <= 0, f"golden {name}: excess {excess.max():.3e}"


def test_argument_errors(device):
    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16, device=device)
    k = torch.zeros(2, 8, 64, 128, dtype=torch.bfloat16, device=device)
    lens = i32([4, 4], device)
    with pytest.raises(RuntimeError):  # output not 16-byte aligned
        buf = torch.empty(2 * 16 * 128 + 1, dtype=torch.bfloat16, device=device)
        gqa_decode_wave(q, k, k, lens, 0.1, buf[1:].view(2, 16, 128))
    with pytest.raises(RuntimeError):  # head_dim 96
        gqa_decode_wave(q[..., :96].contiguous(), k[..., :96].contiguous(), k[..., :96].contiguous(), lens, 0.1)


# (head_dim, q heads per kv head, capacity, routed): the wave kernel takes rows of at most 4096 / head_dim positions
# for 2 q heads per kv head and 8192 / head_dim for 4 or more; 1 q head per kv head always takes the split kernel
ROUTES = [(128, 4, 17, True), (128, 4, 64, True), (128, 4, 65, False), (128, 8, 64, True), (128, 2, 32, True),
          (128, 2, 33, False), (128, 1, 8, False), (64, 2, 64, True), (64, 2, 65, False), (64, 4, 128, True),
          (64, 4, 129, False)]


@pytest.mark.parametrize("D,G,cap,routed", ROUTES)
def test_gqa_decode_routes_short_wide_groups(device, D, G, cap, routed):
    """bz_gqa_decode runs the wave kernel on short rows in groups of two or more q heads when nothing is asked
    explicitly: its output is then bit-identical to bz_gqa_decode_wave's. Past the route's length, for single-head
    groups, or with an explicit split count, it runs the split kernel (one split at these sizes)."""
    rng = np.random.default_rng(77 + cap)
    B, NKV = 2, 2
    NH = NKV * G
    q = bf16(rng.standard_normal((B, NH, D)), device)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    lens = i32([cap, cap - 5], device)
    auto = gqa_decode(q, k, v, lens, D ** -0.5)
    wave = gqa_decode_wave(q, k, v, lens, D ** -0.5)
    one = gqa_decode(q, k, v, lens, D ** -0.5, num_splits=1)
    torch.cuda.synchronize()
    check(auto[:, None], q[:, :, None], k, v, [cap, cap - 5], D ** -0.5, what=f"auto cap={cap}")
    same = wave if routed else one
    assert torch.equal(auto.view(torch.int16), same.view(torch.int16)), f"D={D} G={G} cap={cap} routed={routed}"
    # the wave kernel needs no workspace and the split kernel does: a too-small one shows which route was taken
    tiny = torch.zeros(256, dtype=torch.uint8, device=device)
    if routed:
        gqa_decode(q, k, v, lens, D ** -0.5, workspace=tiny)
    else:
        with pytest.raises(RuntimeError, match="workspace"):
            gqa_decode(q, k, v, lens, D ** -0.5, workspace=tiny)
