"""The C ABI library on the CPU: it loads, exports exactly what include/*.h declares, its argument struct matches the
C layout, and its host-side checks return the documented status codes before anything reaches the GPU.
No call here launches a kernel (every case fails validation first)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADERS = sorted((REPO / "include").glob("*.h"))


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg.load()


@pytest.fixture(scope="module")
def K(pkg):
    from breeze_tts_2_flash_amd import kernels
    return kernels


def _declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(bz_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_exports_match_header(K):
    declared = _declared_functions()
    assert declared == set(K.EXPORTS)
    res = subprocess.run(["nm", "-D", "--defined-only", str(K.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = {ln.split()[-1] for ln in res.stdout.splitlines() if " T " in ln}
    assert exported == declared


def test_every_symbol_resolves(lib, K):
    for name in K.EXPORTS:
        assert getattr(lib, name) is not None


def test_abi_version(lib, K):
    assert lib.bz_gqa_decode_abi_version() == K.ABI_VERSION


def test_struct_layout_matches_c(K, tmp_path):
    fields = [f for f, _ in K.GqaDecodeArgs._fields_]
    src = ["#include <stddef.h>", "#include <stdio.h>", '#include "bz_gqa_decode.h"', "int main(void) {",
           '  printf("size %zu\\n", sizeof(bz_gqa_decode_args));']
    src += [f'  printf("{f} %zu\\n", offsetof(bz_gqa_decode_args, {f}));' for f in fields]
    src += ["  return 0;", "}"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{REPO / 'include'}",
                    str(c), "-o", str(exe)], check=True)
    got = dict(ln.split() for ln in subprocess.run([str(exe)], capture_output=True, text=True,
                                                   check=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(K.GqaDecodeArgs)
    for f in fields:
        assert int(got[f]) == getattr(K.GqaDecodeArgs, f).offset, f


def test_fused_struct_layout_matches_c(K, tmp_path):
    fields = [f for f, _ in K.GqaDecodeFusedArgs._fields_]
    src = ["#include <stddef.h>", "#include <stdio.h>", '#include "bz_gqa_decode.h"', "int main(void) {",
           '  printf("size %zu\\n", sizeof(bz_gqa_decode_fused_args));']
    src += [f'  printf("{f} %zu\\n", offsetof(bz_gqa_decode_fused_args, {f}));' for f in fields]
    src += ["  return 0;", "}"]
    c = tmp_path / "layout_fused.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout_fused"
    subprocess.run(["gcc", "-std=c11", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{REPO / 'include'}",
                    str(c), "-o", str(exe)], check=True)
    got = dict(ln.split() for ln in subprocess.run([str(exe)], capture_output=True, text=True,
                                                   check=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(K.GqaDecodeFusedArgs)
    for f in fields:
        assert int(got[f]) == getattr(K.GqaDecodeFusedArgs, f).offset, f


def test_status_strings(lib):
    for code in range(0, -10, -1):
        s = lib.bz_status_string(code).decode()
        assert s and s != "unknown status"
    assert lib.bz_status_string(-99).decode() == "unknown status"


def _good_args(K, **over):
    """Plausible sizes with fake (never dereferenced) device addresses; every test below breaks one check."""
    a = K.GqaDecodeArgs()
    a.q, a.q_stride_b, a.q_stride_h = 0x10000, 16 * 128, 128
    a.k_cache, a.v_cache = 0x100000, 0x200000
    a.kv_stride_b, a.kv_stride_h, a.kv_stride_s = 8 * 256 * 128, 256 * 128, 128
    a.seq_lens = 0x30000
    a.scale = 128 ** -0.5
    a.out, a.out_stride_b, a.out_stride_h = 0x40000, 16 * 128, 128
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.capacity = 2, 16, 8, 128, 256
    a.num_splits = 4
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,code", [
    (dict(q=None), -1), (dict(k_cache=None), -1), (dict(out=None), -1), (dict(seq_lens=None), -1),
    (dict(num_kv_heads=3), -2), (dict(batch=0), -2), (dict(capacity=0), -2), (dict(kv_stride_s=64), -2),
    (dict(head_dim=96), -3), (dict(num_q_heads=24, num_kv_heads=8), -3), (dict(num_q_heads=32, num_kv_heads=2), -3),
    (dict(k_cache=0x100008), -4), (dict(kv_stride_s=132), -4), (dict(kv_stride_h=256 * 128 + 4), -4),
    (dict(q=0x10004), -4), (dict(q_stride_h=132), -4), (dict(q_stride_b=16 * 128 + 2), -4),
    (dict(tokens_per_row=2, q_stride_t=68), -4), (dict(tokens_per_row=1, q_stride_t=68), -5),
    (dict(mask=0x50000, mask_dtype=0), -6), (dict(mask_dtype=7), -6),
    (dict(num_splits=-1), -2), (dict(num_splits=257), -2),
    (dict(combine=3), -9),
    (dict(workspace=None), -5), (dict(workspace=0x60000, workspace_bytes=16), -5),
    (dict(workspace=0x60010, workspace_bytes=1 << 30), -4),
    # 31-bit byte offsets inside one (row, kv head) span: (capacity + 1024) * kv_stride_s * 2 < 2^31
    (dict(capacity=(1 << 23) - 1024, num_splits=4), -2), (dict(capacity=1 << 20, kv_stride_s=1024), -2),
    (dict(capacity=(1 << 23) - 1025, num_splits=4), -5),   # just inside the bound: fails later, on the workspace
    # query tokens per row: >= 0, and batch * tokens within the grid's z limit
    (dict(tokens_per_row=-1), -2), (dict(batch=16384, tokens_per_row=4), -2),
    (dict(batch=16383, tokens_per_row=4), -5), (dict(tokens_per_row=0), -5), (dict(tokens_per_row=3), -5),
])
def test_host_validation(lib, K, over, code):
    a = _good_args(K, **over)
    assert lib.bz_gqa_decode(ctypes.byref(a), None) == code
    assert lib.bz_gqa_decode(None, None) == -1


def test_masked_validation(lib, K):
    a = _good_args(K)
    assert lib.bz_gqa_decode_masked(ctypes.byref(a), None) == -1            # mask required
    a = _good_args(K, mask=0x50000, mask_dtype=0)
    assert lib.bz_gqa_decode_masked(ctypes.byref(a), None) == -6
    a = _good_args(K, mask=0x50000, mask_dtype=1, workspace=None)
    assert lib.bz_gqa_decode_masked(ctypes.byref(a), None) == -5


def _ws(lib, *args):
    n = ctypes.c_size_t(0)
    rc = lib.bz_gqa_decode_workspace_size(*args, ctypes.byref(n))
    return rc, n.value


def test_workspace_size(lib):
    def layout(B, NH, NKV, D, S):
        # the arrival counters (one 256-byte line per row and kv head), the (m, l) pairs, then the accumulators
        a = lambda x: (x + 255) // 256 * 256  # noqa: E731
        acc = a(B * NKV * 256 + B * NH * S * 8)
        return a(acc + B * NH * S * D * 4)
    for B, NH, NKV, D, cap, S in [(2, 16, 8, 128, 2048, 32), (16, 16, 8, 128, 2048, 1), (2, 8, 2, 64, 17, 3),
                                  (1, 8, 8, 128, 4096, 256)]:
        rc, n = _ws(lib, B, NH, NKV, D, cap, S, 0)
        assert rc == 0 and n == layout(B, NH, NKV, D, S) and n % 256 == 0
    assert _ws(lib, 2, 16, 8, 96, 2048, 4, 0)[0] == -3
    assert _ws(lib, 2, 16, 8, 128, 2048, 300, 0)[0] == -2
    assert lib.bz_gqa_decode_workspace_size(2, 16, 8, 128, 2048, 4, 0, None) == -1


def _good_fused(K, **over):
    f = K.GqaDecodeFusedArgs()
    f.base = _good_args(K, q=None, workspace=None)
    f.qkv, f.qkv_stride_b = 0x70000, (16 + 2 * 8) * 128
    f.q_norm_weight, f.k_norm_weight, f.eps = 0x71000, 0x72000, 1e-6
    f.cos, f.sin, f.rope_stride_b = 0x73000, 0x74000, 128
    f.cache_pos = 0x75000
    for k, v in over.items():
        if k.startswith("base_"):
            setattr(f.base, k[5:], v)
        else:
            setattr(f, k, v)
    return f


@pytest.mark.parametrize("over,code", [
    (dict(qkv=None), -1), (dict(q_norm_weight=None), -1), (dict(cos=None), -1), (dict(cache_pos=None), -1),
    (dict(base_head_dim=64, base_kv_stride_s=64, base_kv_stride_h=256 * 64, base_kv_stride_b=8 * 256 * 64), -3),
    (dict(qkv_stride_b=100), -2), (dict(rope_stride_b=64), -2),
    (dict(qkv=0x70008), -4), (dict(cos=0x73004), -4), (dict(qkv_stride_b=32 * 128 + 4), -4),
    (dict(cache_pos=0x75004), -4),
    (dict(base_tokens_per_row=2), -3),                        # the fused step has one query token per row
    (dict(), -5),                                             # no workspace (checked before any launch)
    (dict(base_seq_lens=None), -1),                           # interval form needs a mask
])
def test_fused_validation(lib, K, over, code):
    f = _good_fused(K, **over)
    assert lib.bz_gqa_decode_fused(ctypes.byref(f), None) == code
    assert lib.bz_gqa_decode_fused(None, None) == -1


def test_gemv_struct_layout_matches_c(K, tmp_path):
    fields = [f for f, _ in K.GemvArgs._fields_]
    src = ["#include <stddef.h>", "#include <stdio.h>", '#include "bz_gemv.h"', "int main(void) {",
           '  printf("size %zu\\n", sizeof(bz_gemv_args));']
    src += [f'  printf("{f} %zu\\n", offsetof(bz_gemv_args, {f}));' for f in fields]
    src += ["  return 0;", "}"]
    c = tmp_path / "layout_gemv.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout_gemv"
    subprocess.run(["gcc", "-std=c11", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{REPO / 'include'}",
                    str(c), "-o", str(exe)], check=True)
    got = dict(ln.split() for ln in subprocess.run([str(exe)], capture_output=True, text=True,
                                                   check=True).stdout.splitlines())
    assert int(got["size"]) == ctypes.sizeof(K.GemvArgs)
    for f in fields:
        assert int(got[f]) == getattr(K.GemvArgs, f).offset, f


def _good_gemv(K, **over):
    """Backbone q|k|v projection sizes with fake (never dereferenced) addresses and no workspace-free launch: every
    case below breaks one check, so nothing is launched."""
    a = K.GemvArgs()
    a.x, a.x_stride = 0x10000, 2048
    a.w[0], a.w[1], a.w[2] = 0x100000, 0x200000, 0x300000
    a.n[0], a.n[1], a.n[2] = 2048, 1024, 1024
    a.y, a.y_stride = 0x40000, 4096
    a.m, a.k, a.epilogue = 2, 2048, K.GEMV_PLAIN
    for key, v in over.items():
        if key.startswith("w") and key[1:].isdigit():
            a.w[int(key[1:])] = v
        elif key.startswith("n") and key[1:].isdigit():
            a.n[int(key[1:])] = v
        else:
            setattr(a, key, v)
    return a


@pytest.mark.parametrize("over,code", [
    (dict(x=None), -1), (dict(y=None), -1), (dict(w0=None), -1), (dict(w1=None), -1),
    (dict(m=0), -2), (dict(m=5), -2), (dict(k=0), -2), (dict(k=2044), -2), (dict(n1=-1), -2),
    (dict(n0=0, n1=0, n2=0), -2), (dict(x_stride=1024), -2), (dict(y_stride=4000), -2),
    (dict(epilogue=3), -3), (dict(epilogue=1), -1), (dict(epilogue=1, res=0x50000, norm_weight=0x60000), -3),
    (dict(epilogue=2, n1=2048, n2=0, w1=None), -1), (dict(epilogue=2, n1=1024, n2=0), -2),
    (dict(epilogue=2, n1=2048, n2=1), -2),
    (dict(x=0x10008), -4), (dict(x_stride=2052), -4), (dict(w2=0x300004), -4), (dict(norm_weight=0x60002), -4),
    (dict(k=32768, x_stride=32768), -3),                      # x does not fit 64 KiB of LDS at m = 2
])
def test_gemv_validation(lib, K, over, code):
    a = _good_gemv(K, **over)
    assert lib.bz_gemv(ctypes.byref(a), None) == code
    assert lib.bz_gemv(None, None) == -1


def test_rmsnorm_validation(lib):
    P = 0x10000
    assert lib.bz_rmsnorm(None, 2048, P, 1e-6, P, 2048, 2, 2048, None) == -1
    assert lib.bz_rmsnorm(P, 2048, P, 1e-6, P, 2048, 0, 2048, None) == -2
    assert lib.bz_rmsnorm(P, 2048, P, 1e-6, P, 2048, 2, 2044, None) == -2
    assert lib.bz_rmsnorm(P, 1024, P, 1e-6, P, 2048, 2, 2048, None) == -2
    assert lib.bz_rmsnorm(P + 2, 2048, P, 1e-6, P, 2048, 2, 2048, None) == -4
    assert lib.bz_rmsnorm(P, 2048, P, 1e-6, P, 2052, 2, 2048, None) == -4


@pytest.mark.parametrize("over,code", [
    (dict(q=None), -1), (dict(seq_lens=None), -1), (dict(head_dim=96), -3), (dict(num_kv_heads=3), -2),
    (dict(mask=0x50000, mask_dtype=1), -3),                         # the wave entry takes no mask
    (dict(out=0x40008), -4), (dict(out_stride_h=132), -4), (dict(out_stride_b=16 * 128 + 4), -4),
    (dict(tokens_per_row=2, q_stride_t=128 * 16, out_stride_t=68), -4),
    (dict(k_cache=0x100008), -4),
    (dict(batch=65536), -2),  # rows > 65535: the grid's z dimension
])
def test_wave_validation(lib, K, over, code):
    a = _good_args(K, **over)
    assert lib.bz_gqa_decode_wave(ctypes.byref(a), None) == code
    assert lib.bz_gqa_decode_wave(None, None) == -1


@pytest.mark.parametrize("over,probs,code", [
    (dict(), None, -1),                                        # no output buffer
    (dict(seq_lens=None), 0x80000, -1),                        # neither seq_lens nor a mask
    (dict(tokens_per_row=2, q_stride_t=128), 0x80000, -3),     # one query token per row
    (dict(), 0x80002, -4),                                     # probs not 4-byte aligned
    (dict(mask=0x50000, mask_dtype=0), 0x80000, -6),           # mask without a dtype
    (dict(head_dim=96), 0x80000, -3),
    (dict(q=None), 0x80000, -1),
])
def test_probs_validation(lib, K, over, probs, code):
    a = _good_args(K, **over)
    assert lib.bz_gqa_decode_probs(ctypes.byref(a), probs, None) == code
    assert lib.bz_gqa_decode_probs(None, 0x80000, None) == -1
    f = _good_fused(K, **{"base_" + k: v for k, v in over.items() if k != "q"})
    if "q" not in over and "head_dim" not in over and "tokens_per_row" not in over:
        assert lib.bz_gqa_decode_fused_probs(ctypes.byref(f), probs, None) == code
    assert lib.bz_gqa_decode_fused_probs(None, 0x80000, None) == -1


def test_mask_interval_validation(lib, K):
    f = lib.bz_mask_interval
    ok = (0x50000, K.MASK_BF16, 2048, 2, 2048, 0x60000, 0x60010, None)
    for i, bad, code in [(0, None, -1), (5, None, -1), (6, None, -1),          # null mask / outputs
                         (1, K.MASK_NONE, -6), (1, 7, -6),                     # mask dtype
                         (3, 0, -2), (4, 0, -2), (2, -1, -2), (2, 100, -2),    # batch, capacity, row stride
                         (0, 0x50001, -4), (5, 0x60002, -4)]:                  # alignment
        args = list(ok)
        args[i] = bad
        assert f(*args) == code, (i, bad)
    args = list(ok)
    args[1], args[0] = K.MASK_F32, 0x50002
    assert f(*args) == -4                                                     # fp32 mask needs 4-byte alignment


def test_missing_library_fails_loudly(K, tmp_path, monkeypatch):
    """No build, no fallback: load() and every entry that needs the library raise."""
    from breeze_tts_2_flash_amd import backbone

    monkeypatch.setattr(K, "_LIB", None)
    monkeypatch.setattr(K, "LIB_PATH", tmp_path / "libbz_gqa_decode.so")
    with pytest.raises(RuntimeError, match="missing"):
        K.load()

    class Graph:
        def _decode_step(self):
            pass

    with pytest.raises(RuntimeError, match="missing"):
        backbone.install(Graph)
    assert Graph._decode_step is not backbone.fused_decode_step


def test_stale_build_is_refused(K, monkeypatch):
    """load() compares the library's build id with the hash of the sources next to it and refuses a library built from
    other sources or flags (the reference's loader rebuilds then, flash/kernels.py:1-4, :64-79)."""
    lib = K.load()
    assert lib.bz_gqa_decode_build_id().decode() == K.source_id()
    monkeypatch.setattr(K, "_LIB", None)
    monkeypatch.setattr(K, "source_id", lambda: "0123456789abcdef")
    with pytest.raises(RuntimeError, match="built from other sources"):
        K.load()
