"""Seeded random shapes through every attention entry against the oracle (oracle.attention.decode_attention_tokens).

Each case draws batch 1..6, kv heads 1/2/4/8, group 1/2/4/8, head_dim 64/128, a capacity of 1..600 slots, per-row
lengths 0..capacity and starts 0..length (empty and one-position rows included), 1 or 2 query tokens per row, a split
count (0 = default, 1, 3, 8, 17), a merge mode and, in about a third of the cases, an additive mask (bf16 or fp32,
values in [-2, 2] with excluded holes inside the range, in half of those also runs of 32..200 excluded positions), with
the K/V cache positions outside each row's range set to NaN. It runs bz_gqa_decode with the drawn options and, without
a mask, bz_gqa_decode_wave; with a mask and one query token also bz_gqa_decode_masked, whose range comes from the mask
(then also excluding what lies outside the row's range), so that chunks the mask excludes entirely are skipped. Tolerance
|out - ref| <= 2e-3 + 1e-2 |ref| (the north star's), every output finite, rows with nothing to attend exactly 0.
"""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import gqa_decode, gqa_decode_masked, gqa_decode_wave
from oracle.attention import decode_attention_tokens
from oracle.bf16 import f32_to_bf16

pytestmark = pytest.mark.gpu

SEEDS = list(range(400))


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 7))
    NKV = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 128]))
    cap = int(rng.integers(1, 601))
    T = int(rng.choice([1, 2]))
    lens = rng.integers(0, cap + 1, size=B)
    lens[rng.random(B) < 0.15] = 0
    lens[rng.random(B) < 0.15] = 1
    starts = np.array([int(rng.integers(0, L + 1)) if rng.random() < 0.5 else 0 for L in lens])
    splits = int(rng.choice([0, 1, 3, 8, 17]))
    combine = str(rng.choice(["auto", "last_block", "kernel"]))
    q = rng.standard_normal((B, NKV * G, T, D)).astype(np.float32)
    k = rng.standard_normal((B, NKV, cap, D)).astype(np.float32)
    v = rng.standard_normal((B, NKV, cap, D)).astype(np.float32)
    for b in range(B):  # NaN outside [start, end): never read, never leaks
        k[b, :, :starts[b]] = v[b, :, :starts[b]] = np.nan
        k[b, :, lens[b]:] = v[b, :, lens[b]:] = np.nan
    mask = None
    if rng.random() < 0.35:
        mask = rng.uniform(-2.0, 2.0, size=(B, cap)).astype(np.float32)
        excl = -np.inf if rng.random() < 0.5 else np.finfo(np.float32).min
        mask[rng.random((B, cap)) < 0.1] = excl
        if rng.random() < 0.5:  # runs of 32..200 excluded positions: whole chunks the masked entry skips
            for b in range(B):
                for _ in range(int(rng.integers(1, 4))):
                    lo = int(rng.integers(0, cap))
                    mask[b, lo:lo + int(rng.integers(32, 201))] = excl
    mask_dtype = torch.bfloat16 if rng.random() < 0.5 else torch.float32
    return dict(B=B, NKV=NKV, G=G, D=D, cap=cap, T=T, lens=lens.astype(np.int32), starts=starts.astype(np.int32),
                splits=splits, combine=combine, q=q, k=k, v=v, mask=mask, mask_dtype=mask_dtype)


def bf16(a, device):
    return torch.from_numpy(a).to(torch.bfloat16).to(device)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_case(device, seed):
    c = draw(seed)
    what = (f"seed {seed}: B={c['B']} NKV={c['NKV']} G={c['G']} D={c['D']} cap={c['cap']} T={c['T']} "
            f"lens={c['lens'].tolist()} starts={c['starts'].tolist()} splits={c['splits']} {c['combine']} "
            f"mask={None if c['mask'] is None else c['mask_dtype']}")
    print(what, flush=True)
    q, k, v = (bf16(c[n], device) for n in ("q", "k", "v"))
    lens = torch.from_numpy(c["lens"]).to(device)
    starts = torch.from_numpy(c["starts"]).to(device)
    scale = c["D"] ** -0.5
    qb, kb, vb = (t.float().cpu().numpy() for t in (q, k, v))  # the bf16-rounded inputs the kernels see
    mask = mb = None
    if c["mask"] is not None:
        mask = torch.from_numpy(c["mask"]).to(c["mask_dtype"]).to(device)[:, None, None, :]
        mb = mask[:, 0, 0].float().cpu().numpy()
    ref = decode_attention_tokens(qb, kb, vb, c["lens"], scale, kv_start=c["starts"], mask=mb)
    outs = {"gqa_decode": gqa_decode(q, k, v, lens, scale, kv_start=starts, mask=mask, num_splits=c["splits"],
                                     combine=c["combine"])}
    if mask is None:
        outs["gqa_decode_wave"] = gqa_decode_wave(q, k, v, lens, scale, kv_start=starts)
    elif c["T"] == 1:
        # the masked entry takes the range from the mask: exclude what lies outside [start, end) as well
        inside = np.zeros_like(c["mask"], dtype=bool)
        for b in range(c["B"]):
            inside[b, c["starts"][b]:c["lens"][b]] = True
        full = np.where(inside, c["mask"], np.float32(-np.inf))
        mfull = torch.from_numpy(full).to(c["mask_dtype"]).to(device)[:, None, None, :]
        outs["gqa_decode_masked"] = gqa_decode_masked(q, k, v, mfull, scale, num_splits=c["splits"],
                                                      combine=c["combine"])
    torch.cuda.synchronize()
    for name, out in outs.items():
        got = out.float().cpu().numpy().reshape(ref.shape)
        assert np.isfinite(got).all(), f"{name} {what}: non-finite output"
        excess = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
        assert excess.max() <= 0, f"{name} {what}: excess {excess.max():.3e}"
        for b in range(c["B"]):
            for t in range(c["T"]):
                s0, e0 = c["starts"][b], max(c["starts"][b], c["lens"][b] - (c["T"] - 1 - t))
                live = e0 > s0 and (mb is None or (mb[b, s0:e0] > -1e30).any())
                if not live:
                    assert not got[b, t].any(), f"{name} {what}: row {b} token {t} attends nothing but is not zero"


FUSED_SEEDS = list(range(120))


@pytest.mark.parametrize("seed", FUSED_SEEDS)
def test_random_fused_step(device, seed):
    """bz_gqa_decode_fused on seeded random shapes: batch 1..4, kv heads 1/2/4/8, group 1/2/4/8, head_dim 128, a
    capacity of 1..600 slots, the new slot anywhere in the cache, each row attending up to and including it from a
    random left-padding start (sometimes a shorter or longer row), random split count and merge mode. Checked with the
    fused-step test's rules: output within tolerance, new k within one bf16 ulp, new v exact, other slots untouched."""
    from tests.test_gpu_fused import check_against_oracle, make_step, run_fused

    rng = np.random.default_rng(5000 + seed)
    B = int(rng.integers(1, 5))
    NKV = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 4, 8]))
    cap = int(rng.integers(1, 601))
    pos = int(rng.integers(0, cap))
    lens = [pos + 1 if rng.random() < 0.8 else int(rng.integers(0, cap + 1)) for _ in range(B)]
    starts = [int(rng.integers(0, min(lens[b], pos + 1) + 1)) if rng.random() < 0.5 else 0 for b in range(B)]
    splits = int(rng.choice([0, 1, 3, 8, 17]))
    combine = str(rng.choice(["auto", "last_block", "kernel"]))
    what = (f"fused seed {seed}: B={B} NKV={NKV} G={G} cap={cap} pos={pos} lens={lens} starts={starts} "
            f"splits={splits} {combine}")
    print(what, flush=True)
    s = make_step(7000 + seed, B=B, NH=NKV * G, NKV=NKV, D=128, cap=cap, pos=pos)
    out, kc, vc = run_fused(s, device, pos, lens, starts, num_splits=splits, combine=combine)
    check_against_oracle(s, pos, lens, starts, out, kc, vc, what)


GEMV_SEEDS = list(range(64))


@pytest.mark.parametrize("seed", GEMV_SEEDS)
def test_random_gemv(device, seed):
    """bz_gemv on seeded random shapes: M 1..4, K a multiple of 8 in 8..7168 (x in registers or in LDS), 1..3 segments
    of 0..1500 rows (plain, optionally RMSNorm'ed), a residual epilogue, or gate/up + SiLU * up; x and y with padded row
    strides. Grids from one workgroup to hundreds (the paced and unpaced variants). Tolerance and bit-exact fraction as
    in the GEMV parity tests (the fraction only from 200 outputs up)."""
    from breeze_tts_2_flash_amd import gemv_gateup, gemv_resid, gemv_seg
    from oracle.gemv import gemv as gemv_ref
    from tests.test_gpu_gemv import assert_gemv_close, dev_bf16, host_bits, rand_bits

    rng = np.random.default_rng(9000 + seed)
    M = int(rng.integers(1, 5))
    K = 8 * int(rng.integers(1, 897))
    kind = str(rng.choice(["seg", "resid", "gateup"]))
    xpad = 8 * int(rng.integers(0, 3))
    x_full = rand_bits(rng, M, K + xpad, scale=2.0)
    x = dev_bf16(x_full, device)[:, :K]
    xb = x_full[:, :K]
    what = f"gemv seed {seed}: {kind} M={M} K={K} x_stride={K + xpad}"
    if kind == "seg":
        ns = [int(rng.integers(1, 1501))] + [int(rng.integers(0, 1501)) for _ in range(int(rng.integers(0, 3)))]
        ws = [rand_bits(rng, n, K, scale=K ** -0.5) for n in ns]
        norm = rng.random() < 0.5
        nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32)) if norm else None
        N = sum(ns)
        y = torch.empty(M, N + 8, dtype=torch.bfloat16, device=device)[:, :N]
        wd = [dev_bf16(w, device) for w in ws] + [torch.empty(0, K, dtype=torch.bfloat16, device=device)] * (3 - len(ws))
        gemv_seg(x, None if nw is None else dev_bf16(nw, device), 1e-6, wd[0], wd[1], wd[2], y)
        ref = gemv_ref(xb, ws, nw, 1e-6)
        frac = 0.98
        what += f" segments={ns} norm={norm}"
    elif kind == "resid":
        N = int(rng.integers(1, 3001))
        w = rand_bits(rng, N, K, scale=K ** -0.5)
        res = rand_bits(rng, M, N, scale=3.0)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=device)
        gemv_resid(x, dev_bf16(w, device), dev_bf16(res, device), y)
        ref = gemv_ref(xb, [w], epilogue="residual", res_bits=res)
        frac = 0.98
        what += f" N={N}"
    else:
        N = int(rng.integers(1, 2001))
        wg, wu = (rand_bits(rng, N, K, scale=K ** -0.5) for _ in range(2))
        nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
        y = torch.empty(M, N, dtype=torch.bfloat16, device=device)
        gemv_gateup(x, dev_bf16(nw, device), 1e-6, dev_bf16(wg, device), dev_bf16(wu, device), y)
        ref = gemv_ref(xb, [wg, wu], nw, 1e-6, epilogue="silu_mul")
        frac = 0.95
        what += f" N={N}"
    print(what, flush=True)
    torch.cuda.synchronize()
    if M * N < 200:  # too few outputs for a bit-exact fraction to mean anything: the tolerance alone
        frac = 0.0
    assert_gemv_close(host_bits(y), ref, what, frac)
