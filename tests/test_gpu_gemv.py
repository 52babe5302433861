"""GPU parity of the backbone decode GEMVs (bz_gemv / bz_rmsnorm through gemv_seg, gemv_resid, gemv_gateup and
rmsnorm) against oracle.gemv at the reference backbone's shapes (hidden 2048, q / k / v 2048 / 1024 / 1024,
intermediate 6144, the CFG pair M = 2) and at edge shapes (M = 1..4, K not a multiple of the tile, output rows not a
multiple of the workgroup's, strided x, missing segments), on both kernels: the wave-per-row kernel and the
block-ordered one (4096 < K <= 6144 at any M, 1024 < K <= 2048 at M >= 3).

Tolerance: the outputs are bf16 roundings of fp32 sums whose order differs from the float64 oracle's, so a value on a
rounding boundary can move by one bf16 ulp (two through the SiLU chain): |got - ref| <= 2^-6 |ref| + 2^-6 rms(ref row),
with at least 98% of the outputs bit-exact (95% for SILU_MUL)."""
import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import gemv_gateup, gemv_resid, gemv_seg, rmsnorm
from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.gemv import gemv as gemv_ref
from oracle.gemv import rmsnorm as rmsnorm_ref

pytestmark = pytest.mark.gpu


def dev_bf16(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def host_bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def rand_bits(rng, *shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def assert_gemv_close(got_bits, ref_bits, what, frac_exact=0.98):
    g, r = bf16_to_f32(got_bits).astype(np.float64), bf16_to_f32(ref_bits).astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite"
    rms = np.sqrt((r ** 2).mean(axis=-1, keepdims=True))
    excess = np.abs(g - r) - (2.0 ** -6 * np.abs(r) + 2.0 ** -6 * rms)
    assert excess.max() <= 0, f"{what}: excess {excess.max():.3e}"
    exact = (got_bits == ref_bits).mean()
    assert exact >= frac_exact, f"{what}: only {exact:.4f} bit-exact"


def backbone_weights(rng, H=2048, nq=2048, nk=1024, inter=6144):
    s = H ** -0.5
    return dict(ln1=f32_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)),
                ln2=f32_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32)),
                wq=rand_bits(rng, nq, H, scale=s), wk=rand_bits(rng, nk, H, scale=s), wv=rand_bits(rng, nk, H, scale=s),
                wo=rand_bits(rng, H, nq, scale=nq ** -0.5), wg=rand_bits(rng, inter, H, scale=s),
                wu=rand_bits(rng, inter, H, scale=s), wd=rand_bits(rng, H, inter, scale=inter ** -0.5))


@pytest.fixture(scope="module")
def bb():
    return backbone_weights(np.random.default_rng(7))


def test_backbone_qkv_with_norm(device, bb):
    rng = np.random.default_rng(1)
    x = rand_bits(rng, 2, 2048, scale=3.0)
    y = torch.empty(2, 4096, dtype=torch.bfloat16, device=device)
    gemv_seg(dev_bf16(x, device), dev_bf16(bb["ln1"], device), 1e-6, dev_bf16(bb["wq"], device),
             dev_bf16(bb["wk"], device), dev_bf16(bb["wv"], device), y)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), gemv_ref(x, [bb["wq"], bb["wk"], bb["wv"]], bb["ln1"], 1e-6), "qkv")


def test_backbone_o_proj_residual(device, bb):
    rng = np.random.default_rng(2)
    a, res = rand_bits(rng, 2, 2048), rand_bits(rng, 2, 2048, scale=4.0)
    y = torch.empty(2, 2048, dtype=torch.bfloat16, device=device)
    gemv_resid(dev_bf16(a, device), dev_bf16(bb["wo"], device), dev_bf16(res, device), y)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), gemv_ref(a, [bb["wo"]], epilogue="residual", res_bits=res), "o_proj")


def test_backbone_gate_up(device, bb):
    rng = np.random.default_rng(3)
    h = rand_bits(rng, 2, 2048, scale=3.0)
    y = torch.empty(2, 6144, dtype=torch.bfloat16, device=device)
    gemv_gateup(dev_bf16(h, device), dev_bf16(bb["ln2"], device), 1e-6, dev_bf16(bb["wg"], device),
                dev_bf16(bb["wu"], device), y)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), gemv_ref(h, [bb["wg"], bb["wu"]], bb["ln2"], 1e-6, epilogue="silu_mul"),
                      "gate/up", frac_exact=0.95)


def test_backbone_down_residual(device, bb):
    rng = np.random.default_rng(4)
    act, res = rand_bits(rng, 2, 6144, scale=0.5), rand_bits(rng, 2, 2048, scale=4.0)
    y = torch.empty(2, 2048, dtype=torch.bfloat16, device=device)
    gemv_resid(dev_bf16(act, device), dev_bf16(bb["wd"], device), dev_bf16(res, device), y)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), gemv_ref(act, [bb["wd"]], epilogue="residual", res_bits=res), "down")


@pytest.mark.parametrize("M", [1, 2, 3, 4])
# K 1000 and 3072: the wave-per-row kernel (x in registers, x in LDS); K 1032, 1800 and 2048 at M >= 3 and K 4104
# and 6144 at any M: the block-ordered kernel, with rows past k's last full vector block (1032, 1800, 4104) and output
# rows that are not a multiple of a workgroup's (37, 129, 130, 300, 520)
@pytest.mark.parametrize("K,N", [(1000, 37), (1032, 129), (3072, 520), (1800, 130), (2048, 300), (4104, 37),
                                 (6144, 520)])
@pytest.mark.parametrize("kind", ["plain", "norm", "residual", "silu"])
def test_edge_shapes(device, M, K, N, kind):
    rng = np.random.default_rng(M * 1000 + K + N)
    xs = rand_bits(rng, M, K + 24, scale=2.0)          # a strided x: rows of K + 24 elements, the first K used
    x = xs[:, :K]
    W = [rand_bits(rng, N, K, scale=K ** -0.5)]
    nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    res = rand_bits(rng, M, N)
    xd = dev_bf16(xs, device)[:, :K]
    y = torch.empty(M, N, dtype=torch.bfloat16, device=device)
    if kind == "plain":
        gemv_seg(xd, None, 0.0, dev_bf16(W[0], device), torch.empty(0), torch.empty(0), y)
        ref = gemv_ref(x, W)
    elif kind == "norm":
        gemv_seg(xd, dev_bf16(nw, device), 1e-5, dev_bf16(W[0], device), torch.empty(0), torch.empty(0), y)
        ref = gemv_ref(x, W, nw, 1e-5)
    elif kind == "residual":
        gemv_resid(xd, dev_bf16(W[0], device), dev_bf16(res, device), y)
        ref = gemv_ref(x, W, epilogue="residual", res_bits=res)
    else:
        Wu = rand_bits(rng, N, K, scale=K ** -0.5)
        gemv_gateup(xd, dev_bf16(nw, device), 1e-5, dev_bf16(W[0], device), dev_bf16(Wu, device), y)
        ref = gemv_ref(x, [W[0], Wu], nw, 1e-5, epilogue="silu_mul")
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), ref, f"{kind} M={M} K={K} N={N}", 0.95 if kind == "silu" else 0.98)


def test_segments_split_anywhere(device):
    # q | k | v segments whose boundaries fall inside a wave's rows and a workgroup's rows
    rng = np.random.default_rng(9)
    K = 512
    x = rand_bits(rng, 2, K)
    W = [rand_bits(rng, n, K, scale=K ** -0.5) for n in (13, 7, 30)]
    y = torch.empty(2, 50, dtype=torch.bfloat16, device=device)
    gemv_seg(dev_bf16(x, device), None, 0.0, *(dev_bf16(w, device) for w in W), y)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), gemv_ref(x, W), "segments")
    # the second segment absent: only W0 and W2 (empty W1)
    y2 = torch.empty(2, 43, dtype=torch.bfloat16, device=device)
    gemv_seg(dev_bf16(x, device), None, 0.0, dev_bf16(W[0], device), torch.empty(0), dev_bf16(W[2], device), y2)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y2), gemv_ref(x, [W[0], W[2]]), "segments without W1")


@pytest.mark.parametrize("M,K", [(2, 6144), (4, 6144), (1, 2048), (3, 2048), (4, 2048)])
def test_block_kernel_segments_and_strides(device, M, K):
    # the block-ordered kernel's row groups and slots across q | k | v segment boundaries (inside a workgroup's rows
    # and inside a row group), a strided x and y, and the norm prologue
    rng = np.random.default_rng(M * 7 + K)
    xs = rand_bits(rng, M, K + 40, scale=2.0)
    W = [rand_bits(rng, n, K, scale=K ** -0.5) for n in (21, 6, 35)]
    nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    ys = torch.empty(M, 70, dtype=torch.bfloat16, device=device)
    y = ys[:, :62]
    gemv_seg(dev_bf16(xs, device)[:, :K], dev_bf16(nw, device), 1e-6, *(dev_bf16(w, device) for w in W), y)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), gemv_ref(xs[:, :K], W, nw, 1e-6), f"segments M={M} K={K}")


def _random_block_cases(n=24, seed=2024):
    """(M, K, N, kind) drawn with a fixed seed from the block kernel's two routes: 4096 < K <= 6144 at any M and
    1024 < K <= 2048 at M >= 3, K any multiple of 8 in the range, N from 1 to 700."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        if i % 2:
            M, K = int(rng.integers(1, 5)), 8 * int(rng.integers(4096 // 8 + 1, 6144 // 8 + 1))
        else:
            M, K = int(rng.integers(3, 5)), 8 * int(rng.integers(1024 // 8 + 1, 2048 // 8 + 1))
        cases.append((M, K, int(rng.integers(1, 701)), ["plain", "norm", "residual", "silu"][i % 4]))
    return cases


@pytest.mark.parametrize("M,K,N,kind", _random_block_cases())
def test_random_block_shapes(device, M, K, N, kind):
    rng = np.random.default_rng(M * 100003 + K * 7 + N)
    x = rand_bits(rng, M, K, scale=2.0)
    W = rand_bits(rng, N, K, scale=K ** -0.5)
    nw = f32_to_bf16((1 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    xd, Wd, nwd = dev_bf16(x, device), dev_bf16(W, device), dev_bf16(nw, device)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=device)
    if kind == "plain":
        gemv_seg(xd, None, 0.0, Wd, torch.empty(0), torch.empty(0), y)
        ref = gemv_ref(x, [W])
    elif kind == "norm":
        gemv_seg(xd, nwd, 1e-6, Wd, torch.empty(0), torch.empty(0), y)
        ref = gemv_ref(x, [W], nw, 1e-6)
    elif kind == "residual":
        res = rand_bits(rng, M, N)
        gemv_resid(xd, Wd, dev_bf16(res, device), y)
        ref = gemv_ref(x, [W], epilogue="residual", res_bits=res)
    else:
        Wu = rand_bits(rng, N, K, scale=K ** -0.5)
        gemv_gateup(xd, nwd, 1e-6, Wd, dev_bf16(Wu, device), y)
        ref = gemv_ref(x, [W, Wu], nw, 1e-6, epilogue="silu_mul")
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), ref, f"{kind} M={M} K={K} N={N}", 0.95 if kind == "silu" else 0.98)


def test_identity_weights_exact(device):
    # W = I: every output is its x element, bit for bit (one nonzero product per output)
    K = 1024
    rng = np.random.default_rng(10)
    x = rand_bits(rng, 2, K, scale=5.0)
    eye = f32_to_bf16(np.eye(K, dtype=np.float32))
    y = torch.empty(2, K, dtype=torch.bfloat16, device=device)
    gemv_seg(dev_bf16(x, device), None, 0.0, dev_bf16(eye, device), torch.empty(0), torch.empty(0), y)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(y), x)


@pytest.mark.parametrize("M,K", [(1, 2048), (2, 2048), (4, 1000)])
def test_rmsnorm(device, M, K):
    rng = np.random.default_rng(M + K)
    x = rand_bits(rng, M, K, scale=3.0)
    w = f32_to_bf16((1 + 0.2 * rng.standard_normal(K)).astype(np.float32))
    y = torch.empty(M, K, dtype=torch.bfloat16, device=device)
    rmsnorm(dev_bf16(x, device), dev_bf16(w, device), 1e-6, y)
    torch.cuda.synchronize()
    assert_gemv_close(host_bits(y), rmsnorm_ref(x, w, 1e-6), f"rmsnorm M={M} K={K}", 0.99)


def test_argument_errors(device):
    x = torch.zeros(2, 64, dtype=torch.bfloat16, device=device)
    W = torch.zeros(32, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(RuntimeError):
        gemv_seg(x, None, 0.0, W, torch.empty(0), torch.empty(0), torch.empty(2, 31, dtype=torch.bfloat16,
                                                                             device=device))
    with pytest.raises(RuntimeError):
        gemv_resid(torch.zeros(5, 64, dtype=torch.bfloat16, device=device), W, torch.zeros(5, 32, dtype=torch.bfloat16,
                   device=device), torch.empty(5, 32, dtype=torch.bfloat16, device=device))
    with pytest.raises(RuntimeError):
        gemv_gateup(x, torch.ones(64, dtype=torch.bfloat16, device=device), 1e-6, W, W[:16],
                    torch.empty(2, 32, dtype=torch.bfloat16, device=device))
