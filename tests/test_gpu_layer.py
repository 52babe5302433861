"""GPU: one Qwen3 decoder layer of the reference's fused decode step at the backbone shape (hidden 2048, 16 q / 8 KV
heads of 128, intermediate 6144, the CFG pair), through this library's kernels in the reference's order
(flash/backbone.py:122-128: gemv_seg -> attn_decode_fused -> gemv_resid -> gemv_gateup -> gemv_resid), against the CPU
oracle of the same chain (oracle.gemv.decoder_layer), and the same step replayed from a HIP graph."""
import numpy as np
import pytest
import torch

import breeze_tts_2_flash_amd as bz
from oracle.attention import interval_mask, qk_norm_rope, rope_cos_sin
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.gemv import decoder_layer, gemv

pytestmark = pytest.mark.gpu

H, NQ, NK, INTER, D, CAP = 2048, 2048, 1024, 6144, 128, 2048


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def dev(b, device):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(device)


def make_layer(seed, x_scale=2.0):
    rng = np.random.default_rng(seed)
    r = lambda *s, scale=1.0: f32_to_bf16((rng.standard_normal(s) * scale).astype(np.float32))  # noqa: E731
    one = lambda n: f32_to_bf16((1 + 0.1 * rng.standard_normal(n)).astype(np.float32))  # noqa: E731
    p = dict(ln1=one(H), ln2=one(H), qn=one(D), kn=one(D), wq=r(NQ, H, scale=H ** -0.5), wk=r(NK, H, scale=H ** -0.5),
             wv=r(NK, H, scale=H ** -0.5), wo=r(H, NQ, scale=NQ ** -0.5), wg=r(INTER, H, scale=H ** -0.5),
             wu=r(INTER, H, scale=H ** -0.5), wd=r(H, INTER, scale=INTER ** -0.5), eps=1e-6, qk_eps=1e-6,
             scale=D ** -0.5)
    kc, vc = r(2, NK // D, CAP, D), r(2, NK // D, CAP, D)
    x = r(2, H, scale=x_scale)
    return p, kc, vc, x


def run_layer(p, x, kc, vc, cos, sin, mask, cache_pos, device, bufs):
    qkv, ao, h1, act, out = bufs
    bz.gemv_seg(x, p["ln1"], p["eps"], p["wq"], p["wk"], p["wv"], qkv)
    bz.attn_decode_fused(qkv, p["qn"], p["kn"], p["qk_eps"], cos, sin, kc, vc, mask, cache_pos, p["scale"],
                         None, None, None, None, ao)
    bz.gemv_resid(ao.view(2, NQ), p["wo"], x, h1)
    bz.gemv_gateup(h1, p["ln2"], p["eps"], p["wg"], p["wu"], act)
    bz.gemv_resid(act, p["wd"], h1, out)
    return out


@pytest.mark.parametrize("x_scale", [2.0, 0.05])
def test_decoder_layer_matches_oracle(device, x_scale):
    """x_scale 0.05: the residual is small next to the attention and MLP branches, so their errors reach the output."""
    p, kc, vc, x = make_layer(31, x_scale)
    pos, pad = 999, [0, 64]
    cos, sin = (f32_to_bf16(t) for t in rope_cos_sin([pos, pos], D))
    ref, _, _ = decoder_layer(x, p, cos, sin, kc, vc, pos, np.array([pos + 1, pos + 1]), kv_start=np.array(pad))

    pd = {k: (dev(v, device) if isinstance(v, np.ndarray) else v) for k, v in p.items()}
    kcd, vcd = dev(kc, device), dev(vc, device)
    mask = interval_mask(pad, pos, CAP).to(device)
    bufs = (torch.empty(2, NQ + 2 * NK, dtype=torch.bfloat16, device=device),
            torch.empty(2, 1, NQ // D, D, dtype=torch.bfloat16, device=device),
            torch.empty(2, H, dtype=torch.bfloat16, device=device),
            torch.empty(2, INTER, dtype=torch.bfloat16, device=device),
            torch.empty(2, H, dtype=torch.bfloat16, device=device))
    out = run_layer(pd, dev(x, device), kcd, vcd, dev(cos, device)[:, None], dev(sin, device)[:, None], mask,
                    torch.tensor([pos], dtype=torch.int64, device=device), device, bufs)
    torch.cuda.synchronize()
    got, want = bf16_to_f32(bits(out)).astype(np.float64), bf16_to_f32(ref).astype(np.float64)
    rms = np.sqrt((want ** 2).mean())
    err = np.abs(got - want)
    print(f"layer: max |d| {err.max():.4e}, rms(ref) {rms:.3f}, max |d|/rms {err.max() / rms:.4e}, "
          f"exact {(bits(out) == ref).mean():.4f}", flush=True)
    # the attention output carries |d| <= 2e-3 + 1e-2 |ref| into o_proj; the GEMVs add bf16 rounding differences
    assert (err <= 2.0 ** -5 * np.abs(want) + 1e-2 * rms).all()
    # q | k | v within the GEMV's rounding of the oracle's; the new v (raw) and k (normed, roped) written at slot pos are
    # the oracle prologue's of the device's own q | k | v, v bit for bit and k up to its last-place rounding (a k
    # value one bf16 ulp off the oracle's GEMV can move a roped k, a difference of two products, by more than that)
    qkv = bits(bufs[0])
    g_qkv, w_qkv = bf16_to_f32(qkv).astype(np.float64), bf16_to_f32(gemv(x, [p["wq"], p["wk"], p["wv"]], p["ln1"],
                                                                          p["eps"])).astype(np.float64)
    q_rms = np.sqrt((w_qkv ** 2).mean(axis=-1, keepdims=True))
    assert (np.abs(g_qkv - w_qkv) <= 2.0 ** -6 * np.abs(w_qkv) + 2.0 ** -6 * q_rms).all()
    k_raw = qkv[:, NQ:NQ + NK].reshape(2, NK // D, D)
    k_want = qk_norm_rope(k_raw, p["kn"], p["qk_eps"], cos[:, None], sin[:, None])
    kd = bits(kcd)[:, :, pos]
    assert np.array_equal(bits(vcd)[:, :, pos], qkv[:, NQ + NK:].reshape(2, NK // D, D))
    assert (np.abs(bf16_to_f32(kd) - bf16_to_f32(k_want)) <= np.abs(bf16_to_f32(k_want)) * 2 ** -7 + 1e-30).all()


def test_two_layers_in_a_hip_graph(device):
    """Two layers captured once and replayed for three decode steps, the position, lengths and RoPE tables advanced
    on the device between replays: every replay equals the same steps run eagerly, bit for bit."""
    layers = []
    for s in (41, 42):
        p, kc, vc, _ = make_layer(s)
        layers.append(({k: (dev(v, device) if isinstance(v, np.ndarray) else v) for k, v in p.items()},
                       dev(kc, device), dev(vc, device)))
    x0 = dev(make_layer(43)[3], device)
    pos0 = 500
    cos = torch.empty(2, 1, D, dtype=torch.bfloat16, device=device)
    sin = torch.empty_like(cos)
    cache_pos = torch.zeros(1, dtype=torch.int64, device=device)
    mask = torch.empty(2, 1, 1, CAP, dtype=torch.bfloat16, device=device)
    bufs = [(torch.empty(2, NQ + 2 * NK, dtype=torch.bfloat16, device=device),
             torch.empty(2, 1, NQ // D, D, dtype=torch.bfloat16, device=device),
             torch.empty(2, H, dtype=torch.bfloat16, device=device),
             torch.empty(2, INTER, dtype=torch.bfloat16, device=device),
             torch.empty(2, H, dtype=torch.bfloat16, device=device)) for _ in layers]

    def set_step(pos):
        c, s_ = (f32_to_bf16(t) for t in rope_cos_sin([pos, pos], D))
        cos.copy_(dev(c, device)[:, None])
        sin.copy_(dev(s_, device)[:, None])
        cache_pos.fill_(pos)
        mask.copy_(interval_mask([0, 32], pos, CAP).to(device))

    def step():
        x = x0
        for (p, kc, vc), b in zip(layers, bufs):
            x = run_layer(p, x, kc, vc, cos, sin, mask, cache_pos, device, b)
        return x

    # eager reference run on copies of the caches
    saved = [(kc.clone(), vc.clone()) for _, kc, vc in layers]
    eager = []
    for i in range(3):
        set_step(pos0 + i)
        eager.append(step().clone())
    torch.cuda.synchronize()
    for (_, kc, vc), (k0, v0) in zip(layers, saved):
        kc.copy_(k0)
        vc.copy_(v0)
    set_step(pos0)
    step()  # warm-up (workspaces) on the capture side as well
    for (_, kc, vc), (k0, v0) in zip(layers, saved):
        kc.copy_(k0)
        vc.copy_(v0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    for i in range(3):
        set_step(pos0 + i)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager[i].view(torch.int16)), f"replay {i}"
