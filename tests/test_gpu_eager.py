"""The native eager binding (breeze-tts-2-flash_amd/csrc/eager_ext.cpp, module _bz_eager): gqa_decode,
gqa_decode_masked and gqa_decode_fused call it first and fall back to the ctypes path only to make a stream's
workspace; gemv_seg, gemv_resid, gemv_gateup and rmsnorm go through it alone. CPU: the module is built from the
sources next to it and exports its functions. GPU: once the stream's workspace exists the native call runs (it
returns the output instead of None), its results equal the ctypes path's bit for bit (the same C ABI call), and for
bad arguments it raises the ctypes path's RuntimeError messages; the GEMVs equal a direct bz_gemv / bz_rmsnorm call
bit for bit and raise their argument checks' messages."""
import ctypes

import pytest
import torch

from breeze_tts_2_flash_amd import attention, gqa_decode, gqa_decode_fused, gqa_decode_masked, kernels
from tests.test_gpu_parity import rand_case


def test_module_matches_its_sources():
    mod = kernels.eager()
    assert mod.build_id() == kernels.eager_id()
    for name in ("decode", "fused", "gemv", "rmsnorm", "bind", "register_workspace", "build_id"):
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


def _bf16(shape, gen, device, scale=1.0):
    return (torch.randn(*shape, generator=gen, device=device) * scale).bfloat16()


def _c_gemv(x, y, epilogue, w, n, nw=None, eps=0.0, res=None):
    """bz_gemv called directly through ctypes: the reference result for the native binding."""
    a = kernels.GemvArgs()
    a.x, a.x_stride, a.y, a.y_stride = x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0)
    a.m, a.k, a.epilogue = x.size(0), x.size(1), epilogue
    for i, (t, rows) in enumerate(zip(w, n)):
        a.w[i], a.n[i] = t.data_ptr(), rows
    if nw is not None:
        a.norm_weight, a.eps = nw.data_ptr(), eps
    if res is not None:
        a.res, a.res_stride = res.data_ptr(), res.stride(0)
    kernels.run_on(x.device, lambda s: kernels.check(kernels.load().bz_gemv(ctypes.byref(a), ctypes.c_void_p(s)),
                                                     "bz_gemv"))


@pytest.mark.gpu
@pytest.mark.parametrize("M,K", [(2, 2048), (4, 2048), (2, 6144), (1, 1000)])
def test_native_gemvs_equal_the_c_abi(device, M, K):
    from breeze_tts_2_flash_amd import gemv_gateup, gemv_resid, gemv_seg, rmsnorm

    gen = torch.Generator(device=device).manual_seed(M * 10000 + K)
    x = _bf16((M, K), gen, device, 2.0)
    nw = (1 + 0.1 * torch.randn(K, generator=gen, device=device)).bfloat16()
    W0, W1, W2 = (_bf16((n, K), gen, device, K ** -0.5) for n in (96, 40, 24))
    res = _bf16((M, 96), gen, device)
    # gemv_seg with the norm and three segments
    got, want = torch.empty(M, 160, dtype=torch.bfloat16, device=device), torch.empty(M, 160, dtype=torch.bfloat16,
                                                                                    device=device)
    assert gemv_seg(x, nw, 1e-6, W0, W1, W2, got) is got
    _c_gemv(x, want, kernels.GEMV_PLAIN, (W0, W1, W2), (96, 40, 24), nw, 1e-6)
    # gemv_resid
    got2, want2 = torch.empty_like(res), torch.empty_like(res)
    assert gemv_resid(x, W0, res, got2) is got2
    _c_gemv(x, want2, kernels.GEMV_RESIDUAL, (W0,), (96,), res=res)
    # gemv_gateup
    got3, want3 = torch.empty(M, 40, dtype=torch.bfloat16, device=device), torch.empty(M, 40, dtype=torch.bfloat16,
                                                                                     device=device)
    Wu = _bf16((40, K), gen, device, K ** -0.5)
    assert gemv_gateup(x, nw, 1e-6, W1, Wu, got3) is got3
    _c_gemv(x, want3, kernels.GEMV_SILU_MUL, (W1, Wu), (40, 40), nw, 1e-6)
    # rmsnorm
    got4, want4 = torch.empty_like(x), torch.empty_like(x)
    assert rmsnorm(x, nw, 1e-6, got4) is got4
    kernels.run_on(x.device, lambda s: kernels.check(kernels.load().bz_rmsnorm(
        x.data_ptr(), x.stride(0), nw.data_ptr(), 1e-6, want4.data_ptr(), want4.stride(0), M, K, ctypes.c_void_p(s)),
        "bz_rmsnorm"))
    torch.cuda.synchronize()
    for g_, w_ in ((got, want), (got2, want2), (got3, want3), (got4, want4)):
        assert torch.equal(_bits(g_), _bits(w_))


@pytest.mark.gpu
def test_native_gemv_errors(device):
    from breeze_tts_2_flash_amd import gemv_gateup, gemv_resid, gemv_seg, rmsnorm

    x = torch.zeros(2, 64, dtype=torch.bfloat16, device=device)
    W = torch.zeros(32, 64, dtype=torch.bfloat16, device=device)
    y = torch.empty(2, 32, dtype=torch.bfloat16, device=device)
    nw = torch.ones(64, dtype=torch.bfloat16, device=device)
    e = torch.empty(0)
    cases = [
        (lambda: gemv_seg(x.float(), None, 0.0, W, e, e, y), "x must be a bf16 [M, K] device tensor with a contiguous "
                                                              "last dim"),
        (lambda: gemv_seg(torch.zeros(5, 64, dtype=torch.bfloat16, device=device), None, 0.0, W, e, e, y),
         "x: M must be 1..4, got 5"),
        (lambda: gemv_seg(x[:, :60], None, 0.0, W[:, :60].contiguous(), e, e, y),
         "x: K and the row stride must be multiples of 8"),
        (lambda: gemv_seg(x, None, 0.0, W.t(), e, e, y), "W0 must be a contiguous bf16 [N, 64] device tensor"),
        (lambda: gemv_seg(x, None, 0.0, W, W[:, :32].contiguous(), e, y),
         "W1 must be a contiguous bf16 [N, 64] device tensor"),
        (lambda: gemv_seg(x, None, 0.0, W, e, e, y[:, :31]), "y must be a bf16 [2, 32] device tensor with a contiguous "
                                                             "last dim"),
        (lambda: gemv_seg(x, nw[:63], 1e-6, W, e, e, y), "the norm weight must be a contiguous bf16 [64] device tensor"),
        (lambda: gemv_resid(x, W, y[:1], y), "res must be a bf16 [2, 32] device tensor with a contiguous last dim"),
        (lambda: gemv_gateup(x, nw, 1e-6, W, W[:16], y), "Wg and Wu must have the same number of rows"),
        (lambda: rmsnorm(x, nw, 1e-6, y), "y must be a bf16 [2, 64] device tensor with a contiguous last dim"),
    ]
    for i, (fn, msg) in enumerate(cases):
        assert _message(fn) == msg, f"case {i}"
    # a status from the C ABI: x's stride not a multiple of 8 passes the Python-level checks only through the
    # C ABI's own alignment check (x not 16-byte aligned)
    xs = torch.zeros(2, 72, dtype=torch.bfloat16, device=device)[:, 4:68]
    m = _message(lambda: gemv_seg(xs, None, 0.0, W, e, e, y))
    assert m.startswith("gemv_seg: ") and "(status -4)" in m
