"""The native eager binding (breeze-tts-2-flash_amd/csrc/eager_ext.cpp, module _bz_eager): gqa_decode,
gqa_decode_masked and gqa_decode_fused call it first and fall back to the ctypes path only to make a stream's
workspace. CPU: the module is built from the sources next to it and exports its functions. GPU: once the stream's
workspace exists the native call runs (it returns the output instead of None), its results equal the ctypes path's
bit for bit (the same C ABI call), and for bad arguments it raises the ctypes path's RuntimeError messages."""
import ctypes

import pytest
import torch

from breeze_tts_2_flash_amd import attention, gqa_decode, gqa_decode_fused, gqa_decode_masked, kernels
from tests.test_gpu_parity import rand_case


def test_module_matches_its_sources():
    mod = kernels.eager()
    assert mod.build_id() == kernels.eager_id()
    for name in ("decode", "fused", "bind", "register_workspace", "build_id"):
        assert callable(getattr(mod, name))


def _bits(t):
    return t.view(torch.int16)


def _python_path(q, k, v, lens, scale, out, kv_start=None, mask=None, masked=False):
    """The ctypes path alone (what the package did before the native binding), with an explicit workspace."""
    a, out = attention._fill_args(q, k, v, scale, out, 0, 0, "auto")
    dev = q.device
    if masked:
        a.mask_dtype, a.mask_stride_b = attention._mask_view(mask, a.batch, a.capacity)
        a.mask = mask.data_ptr()
    else:
        a.seq_lens = lens.data_ptr()
        a.kv_start = kv_start.data_ptr() if kv_start is not None else None
    ws = attention.get_workspace(dev, a.batch * max(1, a.tokens_per_row), a.num_q_heads, a.num_kv_heads, a.head_dim,
                                 a.capacity)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    entry = "bz_gqa_decode_masked" if masked else "bz_gqa_decode"
    kernels.run_on(dev, lambda s: kernels.check(getattr(kernels.load(), entry)(ctypes.byref(a), ctypes.c_void_p(s)),
                                                entry))
    return out


@pytest.mark.gpu
def test_native_call_runs_and_equals_the_ctypes_path(device):
    w, st = rand_case(71, 2, 16, 8, 128, 512, [400, 333], [0, 9])
    g = w.to(device)
    starts = st.to(device)
    ref = _python_path(g.q, g.k, g.v, g.seq_lens, w.scale, None, kv_start=starts)
    gqa_decode(g.q, g.k, g.v, g.seq_lens, w.scale, kv_start=starts)  # makes this stream's workspace if needed
    got = kernels.eager().decode(g.q, g.k, g.v, g.seq_lens, starts, None, None, w.scale, 0, 0, "auto", None, False)
    assert got is not None, "the native call fell back although the stream's workspace exists"
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(ref))
    # the package function returns the same bits, into a caller's output too
    out = torch.empty_like(ref)
    assert gqa_decode(g.q, g.k, g.v, g.seq_lens, w.scale, out, kv_start=starts) is out
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(ref))


@pytest.mark.gpu
def test_native_masked_and_fused_equal_the_ctypes_path(device):
    from oracle.attention import interval_mask

    w, _ = rand_case(72, 2, 16, 8, 128, 256, [200, 200])
    g = w.to(device)
    mask = interval_mask([0, 7], 199, 256).to(device)
    ref = _python_path(g.q, g.k, g.v, None, w.scale, None, mask=mask, masked=True)
    got = gqa_decode_masked(g.q, g.k, g.v, mask, w.scale)
    got2 = kernels.eager().decode(g.q, g.k, g.v, None, None, mask, None, w.scale, 0, 0, "auto", None, True)
    assert got2 is not None
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(ref)) and torch.equal(_bits(got2), _bits(ref))
    # fused: the native call against the ctypes path's argument block, on fresh copies of the caches
    B, NH, NKV, D = 2, 16, 8, 128
    gen = torch.Generator(device=device).manual_seed(73)
    qkv = (torch.randn(B, (NH + 2 * NKV) * D, generator=gen, device=device)).bfloat16()
    qn, kn = (1 + 0.1 * torch.randn(D, generator=gen, device=device)).bfloat16(), \
        (1 + 0.1 * torch.randn(D, generator=gen, device=device)).bfloat16()
    cos, sin = torch.randn(B, D, generator=gen, device=device).bfloat16(), \
        torch.randn(B, D, generator=gen, device=device).bfloat16()
    pos = torch.tensor([150], dtype=torch.int64, device=device)
    lens = torch.full((B,), 151, dtype=torch.int32, device=device)
    k1, v1, k2, v2 = g.k.clone(), g.v.clone(), g.k.clone(), g.v.clone()
    ws = attention.get_workspace(device, B, NH, NKV, D, 256)
    native = gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, k1, v1, pos, w.scale, seq_lens=lens, workspace=ws)
    f, out = attention._fused_args(qkv, qn, kn, 1e-6, cos, sin, k2, v2, pos, w.scale, None, lens, None, None, 0, 0,
                                   "auto")
    f.base.workspace, f.base.workspace_bytes = ws.data_ptr(), ws.numel()
    kernels.run_on(device, lambda s: kernels.check(kernels.load().bz_gqa_decode_fused(ctypes.byref(f),
                                                                                     ctypes.c_void_p(s)),
                                                   "bz_gqa_decode_fused"))
    torch.cuda.synchronize()
    assert torch.equal(_bits(native), _bits(out))
    assert torch.equal(_bits(k1), _bits(k2)) and torch.equal(_bits(v1), _bits(v2))


def _message(fn):
    with pytest.raises(RuntimeError) as e:
        fn()
    return str(e.value)


@pytest.mark.gpu
def test_native_errors_are_the_ctypes_paths(device):
    """For each bad call the native binding's RuntimeError carries the message of the ctypes path's own check."""
    w, _ = rand_case(74, 2, 16, 8, 128, 64, [64, 64])
    g = w.to(device)
    E = kernels.eager()

    def native(q=g.q, k=g.k, v=g.v, lens=g.seq_lens, starts=None, mask=None, out=None, combine="auto"):
        return E.decode(q, k, v, lens, starts, mask, out, 0.1, 0, 0, combine, None, False)

    cases = [
        (lambda: native(q=g.q.float()), lambda: attention._check_args(g.q.float(), g.k, g.v, 0.1, None, 0, 0, "auto")),
        (lambda: native(q=g.q.cpu()), lambda: attention._check_args(g.q.cpu(), g.k, g.v, 0.1, None, 0, 0, "auto")),
        (lambda: native(q=g.q[0]), lambda: attention._check_args(g.q[0], g.k, g.v, 0.1, None, 0, 0, "auto")),
        (lambda: native(k=g.k[:, :, :32]), lambda: attention._check_args(g.q, g.k[:, :, :32], g.v, 0.1, None, 0, 0,
                                                                          "auto")),
        (lambda: native(k=g.k[:1], v=g.v[:1]), lambda: attention._check_args(g.q, g.k[:1], g.v[:1], 0.1, None, 0, 0,
                                                                              "auto")),
        (lambda: native(out=torch.empty(2, 16, 64, dtype=torch.bfloat16, device=device)),
         lambda: attention._check_args(g.q, g.k, g.v, 0.1, torch.empty(2, 16, 64, dtype=torch.bfloat16,
                                                                        device=device), 0, 0, "auto")),
        (lambda: native(out=torch.empty(2, 16, 128, device=device)),
         lambda: attention._check_args(g.q, g.k, g.v, 0.1, torch.empty(2, 16, 128, device=device), 0, 0, "auto")),
        (lambda: native(lens=g.seq_lens.long()), lambda: attention._int32_rows(g.seq_lens.long(), 2, "seq_lens",
                                                                                g.q.device)),
        (lambda: native(starts=torch.zeros(3, dtype=torch.int32, device=device)),
         lambda: attention._int32_rows(torch.zeros(3, dtype=torch.int32, device=device), 2, "kv_start", g.q.device)),
        (lambda: native(mask=torch.zeros(2, 1, 1, 32, device=device)),
         lambda: attention._mask_view(torch.zeros(2, 1, 1, 32, device=device), 2, 64)),
        (lambda: native(mask=torch.zeros(3, 1, 1, 64, device=device)),
         lambda: attention._mask_view(torch.zeros(3, 1, 1, 64, device=device), 2, 64)),
        (lambda: native(mask=torch.zeros(2, 2, 1, 64, device=device)),
         lambda: attention._mask_view(torch.zeros(2, 2, 1, 64, device=device), 2, 64)),
        (lambda: native(combine="fast"), lambda: attention._combine_code("fast")),
    ]
    for i, (nat, py) in enumerate(cases):
        assert _message(nat) == _message(py), f"case {i}"
    # a status from the C ABI (head_dim 96 has no kernel): the ctypes path's "what: status (status n)" form
    q96 = torch.zeros(2, 16, 96, dtype=torch.bfloat16, device=device)
    kv96 = torch.zeros(2, 8, 64, 96, dtype=torch.bfloat16, device=device)
    m = _message(lambda: gqa_decode(q96, kv96, kv96, g.seq_lens, 0.1))
    assert m.startswith("bz_gqa_decode") and "unsupported" in m and "(status -3)" in m
