"""GPU parity of the fused decode step (bz_gqa_decode_fused; the reference's attn_decode_fused) against the CPU
oracle (oracle.attention.fused_decode): attention output within |d| <= 2e-3 + 1e-2 |ref|, the new k (q_norm/k_norm +
RoPE at the eager bf16 rounding points) within one bf16 ulp of the oracle's, the new v bit-exact, every other cache
slot untouched."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import attn_decode_fused, gqa_decode_fused
from breeze_tts_2_flash_amd.attention import get_workspace
from oracle.attention import fused_decode, interval_mask, rope_cos_sin
from oracle.bf16 import bf16_to_f32, f32_to_bf16

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def tens(b: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(device)


def assert_close(got, ref, what):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite"
    excess = np.abs(got - ref) - (ATOL + RTOL * np.abs(ref))
    assert excess.max() <= 0, f"{what}: excess {excess.max():.3e}"


def assert_k_slot(got_bits, ref_bits, what):
    g, r = bf16_to_f32(got_bits).astype(np.float64), bf16_to_f32(ref_bits).astype(np.float64)
    assert (np.abs(g - r) <= np.abs(r) * 2.0 ** -7 + 1e-30).all(), f"{what}: new k differs by more than 1 bf16 ulp"
    assert (got_bits == ref_bits).mean() >= 0.98, f"{what}: too many bf16 rounding differences"


def make_step(seed, B=2, NH=16, NKV=8, D=128, cap=2048, pos=1000, fill=None):
    rng = np.random.default_rng(seed)
    qkv = f32_to_bf16((rng.standard_normal((B, (NH + 2 * NKV) * D)) * 3).astype(np.float32))
    qn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    kn = f32_to_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    cos, sin = (f32_to_bf16(t) for t in rope_cos_sin([pos] * B, D))
    kc = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))
    vc = f32_to_bf16(rng.standard_normal((B, NKV, cap, D)).astype(np.float32))
    return dict(qkv=qkv, qn=qn, kn=kn, cos=cos, sin=sin, kc=kc, vc=vc, D=D, NH=NH, NKV=NKV, B=B, cap=cap)


def run_fused(s, device, pos, seq_lens, kv_start=None, **kw):
    kc, vc = tens(s["kc"], device), tens(s["vc"], device)
    cp = torch.tensor([pos], dtype=torch.int64, device=device)
    lens = torch.tensor(seq_lens, dtype=torch.int32, device=device)
    st = None if kv_start is None else torch.tensor(kv_start, dtype=torch.int32, device=device)
    out = gqa_decode_fused(tens(s["qkv"], device), tens(s["qn"], device), tens(s["kn"], device), 1e-6,
                           tens(s["cos"], device), tens(s["sin"], device), kc, vc, cp, s["D"] ** -0.5,
                           seq_lens=lens, kv_start=st, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), bits(kc), bits(vc)


def check_against_oracle(s, pos, seq_lens, kv_start, out, kc, vc, what):
    ref, k2, v2 = fused_decode(s["qkv"], s["qn"], s["kn"], 1e-6, s["cos"], s["sin"], s["kc"], s["vc"], pos,
                               np.asarray(seq_lens), s["D"] ** -0.5,
                               kv_start=None if kv_start is None else np.asarray(kv_start))
    assert_close(out, ref, what)
    if 0 <= pos < s["cap"]:
        assert_k_slot(kc[:, :, pos], k2[:, :, pos], what)
        assert np.array_equal(vc[:, :, pos], v2[:, :, pos]), f"{what}: new v not written bit-exactly"
    other = np.ones(s["cap"], bool)
    if 0 <= pos < s["cap"]:
        other[pos] = False
    assert np.array_equal(kc[:, :, other], s["kc"][:, :, other]), f"{what}: K cache changed outside the slot"
    assert np.array_equal(vc[:, :, other], s["vc"][:, :, other]), f"{what}: V cache changed outside the slot"


@pytest.mark.parametrize("splits", [0, 1, 5, 16])
@pytest.mark.parametrize("combine", ["last_block", "kernel"])
def test_fused_backbone_step(device, splits, combine):
    s = make_step(1)
    pos = 1000
    out, kc, vc = run_fused(s, device, pos, [pos + 1, pos + 1], [0, 37], num_splits=splits, combine=combine)
    check_against_oracle(s, pos, [pos + 1, pos + 1], [0, 37], out, kc, vc, f"splits={splits} {combine}")


@pytest.mark.parametrize("pos,lens,what", [
    (0, [1, 1], "first slot"),
    (2047, [2048, 2048], "last slot"),
    (500, [400, 300], "slot past the attended range (written, not attended)"),
    (2048, [700, 2048], "slot outside the cache (nothing written)"),
])
def test_fused_slot_edges(device, pos, lens, what):
    s = make_step(2, pos=min(pos, 2047))
    out, kc, vc = run_fused(s, device, pos, lens)
    check_against_oracle(s, pos, lens, None, out, kc, vc, what)


def test_fused_depth_shape(device):
    # the reference's depth transformer: 8 q / 2 KV heads (G = 4), head_dim 128, <= 16 positions
    s = make_step(3, NH=8, NKV=2, cap=17, pos=9)
    out, kc, vc = run_fused(s, device, 9, [10, 10])
    check_against_oracle(s, 9, [10, 10], None, out, kc, vc, "depth 8/2")


def test_attn_decode_fused_reference_call(device):
    """The reference's argument order with its interval mask (left padding on row 1), as in
    flash/backbone.py:123-124; out [B, 1, NH, D]."""
    s = make_step(4, pos=1299)
    pos, pad = 1299, [0, 211]
    mask = interval_mask(pad, pos, s["cap"]).to(device)
    kc, vc = tens(s["kc"], device), tens(s["vc"], device)
    out = torch.empty(2, 1, 16, 128, dtype=torch.bfloat16, device=device)
    ret = attn_decode_fused(tens(s["qkv"], device), tens(s["qn"], device), tens(s["kn"], device), 1e-6,
                            tens(s["cos"], device)[:, None], tens(s["sin"], device)[:, None], kc, vc, mask,
                            torch.tensor([pos], dtype=torch.int64, device=device), 128 ** -0.5,
                            None, None, None, None, out)
    torch.cuda.synchronize()
    assert ret is out
    check_against_oracle(s, pos, [pos + 1, pos + 1], pad, out[:, 0].float().cpu().numpy(), bits(kc), bits(vc),
                         "attn_decode_fused")


def test_fused_decode_loop_in_hip_graph(device):
    """Five decode steps replayed from one HIP graph with cache_pos / seq_lens / cos / sin advanced on the device
    between replays; the caches evolve exactly as the oracle's, step after step."""
    s = make_step(5, cap=256, pos=100)
    B, D = s["B"], s["D"]
    kc, vc = tens(s["kc"], device), tens(s["vc"], device)
    qkv, qn, kn = tens(s["qkv"], device), tens(s["qn"], device), tens(s["kn"], device)
    cos, sin = tens(s["cos"], device), tens(s["sin"], device)
    cp = torch.tensor([100], dtype=torch.int64, device=device)
    lens = torch.tensor([101, 101], dtype=torch.int32, device=device)
    out = torch.empty(B, 16, D, dtype=torch.bfloat16, device=device)
    # a captured fused call needs its workspace made beforehand (nothing is allocated during a capture)
    ws = get_workspace(device, B, 16, 8, D, 256)
    call = lambda: gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc, vc, cp, D ** -0.5, out,  # noqa: E731
                                    seq_lens=lens, workspace=ws)
    call()  # eager step at slot 100
    torch.cuda.synchronize()
    ref_k, ref_v = s["kc"], s["vc"]
    _, ref_k, ref_v = fused_decode(s["qkv"], s["qn"], s["kn"], 1e-6, s["cos"], s["sin"], ref_k, ref_v, 100,
                                   np.array([101, 101]), D ** -0.5)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    rng = np.random.default_rng(55)
    for step, pos in enumerate(range(101, 106)):
        new_qkv = f32_to_bf16((rng.standard_normal((B, 32 * D)) * 3).astype(np.float32))
        c_np, s_np = (f32_to_bf16(t) for t in rope_cos_sin([pos] * B, D))
        qkv.copy_(tens(new_qkv, device))
        cos.copy_(tens(c_np, device))
        sin.copy_(tens(s_np, device))
        cp.fill_(pos)
        lens.fill_(pos + 1)
        graph.replay()
        torch.cuda.synchronize()
        ref, ref_k2, ref_v2 = fused_decode(new_qkv, s["qn"], s["kn"], 1e-6, c_np, s_np, ref_k, ref_v, pos,
                                           np.array([pos + 1, pos + 1]), D ** -0.5)
        assert_close(out.float().cpu().numpy(), ref, f"graph step {step}")
        got_k, got_v = bits(kc), bits(vc)
        assert_k_slot(got_k[:, :, pos], ref_k2[:, :, pos], f"graph step {step}")
        assert np.array_equal(got_v[:, :, pos], ref_v2[:, :, pos])
        # carry the GPU's own cache forward so that later steps compare like with like
        ref_k, ref_v = got_k, got_v


def test_golden_fused_fixtures(device):
    """tests/golden/fused_and_tokens.npz: the fused cases through gqa_decode_fused."""
    from tests.golden.make_golden import OUT2, load

    for name, c in sorted(load(OUT2).items()):
        if not name.startswith("fused"):
            continue
        pos = int(c["pos"])
        kc, vc = tens(c["k"], device), tens(c["v"], device)
        out = gqa_decode_fused(tens(c["qkv"], device), tens(c["qn"], device), tens(c["kn"], device), float(c["eps"]),
                               tens(c["cos"], device), tens(c["sin"], device), kc, vc,
                               torch.tensor([pos], dtype=torch.int64, device=device), float(c["scale"]),
                               seq_lens=torch.from_numpy(c["lens"]).to(device),
                               kv_start=torch.from_numpy(c["starts"]).to(device))
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), c["out"], f"golden {name}")
        assert_k_slot(bits(kc)[:, :, pos], c["k_slot"], f"golden {name}")
        assert np.array_equal(bits(vc)[:, :, pos], c["v_slot"]), f"golden {name}: v slot"
