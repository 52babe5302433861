"""Build and load the HIP library libbz_gqa_decode.so (the C ABI in include/bz_gqa_decode.h).

Counterpart of the reference's extension loader (flash/kernels.py:20-87): the reference JIT-builds a pybind
extension with nvcc under a process lock and caches it. Here hipcc builds one plain shared library for gfx950,
in-tree next to this file, ahead of time (build()); load() only opens it, under a lock, once per process, and
declares the C signatures for ctypes. There is no fallback: if the library is missing, load() raises.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import shutil
import subprocess
import tempfile
import threading
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
REPO_DIR = PKG_DIR.parent
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libbz_gqa_decode.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["gqa_decode.hip", "gqa_fused.hip", "gemv.hip"]  # translation units, compiled in parallel
HEADERS = ["gqa_kernels.cuh", "gqa_wave.cuh", "device_common.cuh"]
ARCH = "gfx950"
# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU ops (v_pk_*_f32)
# -falign-loops=64: loop heads on 64-byte boundaries (instruction fetch); the split kernels measured 1-4% faster with
# it, and their speed otherwise moved by a few percent with unrelated code changes that only shifted the loop
# -amdgpu-kernarg-preload-count=14: the first 56 bytes of scalar kernel arguments arrive in SGPRs with each wave (the
# kernels put the pointers their first loads need there), one round trip to the argument buffer fewer at every
# launch: the x-in-registers GEMVs 0.25-0.34 us faster each, the 28-layer backbone step 927 -> 901 us; the attention
# kernels measured the same either way
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-falign-loops=64",
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
ABI_VERSION = 9

# exported symbols and their ctypes signatures (include/bz_gqa_decode.h)
EXPORTS = (
    "bz_gqa_decode", "bz_gqa_decode_masked", "bz_gqa_decode_fused", "bz_gqa_decode_workspace_size",
    "bz_gqa_decode_default_splits", "bz_status_string", "bz_gqa_decode_abi_version", "bz_gemv", "bz_rmsnorm",
    "bz_mask_interval", "bz_gqa_decode_wave", "bz_gqa_decode_build_id", "bz_gqa_decode_noalloc",
    "bz_gqa_decode_probs", "bz_gqa_decode_fused_probs",
)


def source_id() -> str:
    """Hash of what build() compiles: the translation units, their headers, the C ABI headers, bench.py's timing
    helper (built in the same step) and the hipcc flags (sha256, first 16 hex digits). build() compiles it into the
    library (bz_gqa_decode_build_id) and load() refuses a library whose id differs from the sources next to it, as the
    reference's loader rebuilds when a source or a flag changes (flash/kernels.py:1-4, :64-79); a change to the
    timing helper's source without a rebuild is caught the same way."""
    h = hashlib.sha256()
    files = [CSRC / f for f in SOURCES + HEADERS + [STAMP_SOURCE]] + sorted(INCLUDE.glob("*.h"))
    for f in files:
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    h.update(" ".join(HIPCC_FLAGS).encode())
    return h.hexdigest()[:16]

MASK_NONE, MASK_BF16, MASK_F32 = 0, 1, 2
COMBINE_AUTO, COMBINE_LAST_BLOCK, COMBINE_KERNEL = 0, 1, 2
ERR_SCRATCH = -10  # BZ_ERR_SCRATCH: the sizes exceed bz_gqa_decode_noalloc's static scratch


class GqaDecodeArgs(ctypes.Structure):
    """Mirror of struct bz_gqa_decode_args (field order, types and C alignment)."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride_b", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("kv_stride_b", ctypes.c_int64), ("kv_stride_h", ctypes.c_int64), ("kv_stride_s", ctypes.c_int64),
        ("seq_lens", ctypes.c_void_p), ("kv_start", ctypes.c_void_p),
        ("mask", ctypes.c_void_p), ("mask_dtype", ctypes.c_int32), ("mask_stride_b", ctypes.c_int64),
        ("scale", ctypes.c_float),
        ("out", ctypes.c_void_p), ("out_stride_b", ctypes.c_int64), ("out_stride_h", ctypes.c_int64),
        ("batch", ctypes.c_int32), ("num_q_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("capacity", ctypes.c_int32),
        ("num_splits", ctypes.c_int32), ("max_seq_len", ctypes.c_int32), ("combine", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("tokens_per_row", ctypes.c_int32), ("q_stride_t", ctypes.c_int64), ("out_stride_t", ctypes.c_int64),
    ]


class GqaDecodeFusedArgs(ctypes.Structure):
    """Mirror of struct bz_gqa_decode_fused_args."""
    _fields_ = [
        ("base", GqaDecodeArgs),
        ("qkv", ctypes.c_void_p), ("qkv_stride_b", ctypes.c_int64),
        ("q_norm_weight", ctypes.c_void_p), ("k_norm_weight", ctypes.c_void_p), ("eps", ctypes.c_float),
        ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p), ("rope_stride_b", ctypes.c_int64),
        ("cache_pos", ctypes.c_void_p),
    ]


GEMV_PLAIN, GEMV_RESIDUAL, GEMV_SILU_MUL = 0, 1, 2


class GemvArgs(ctypes.Structure):
    """Mirror of struct bz_gemv_args (include/bz_gemv.h)."""
    _fields_ = [
        ("x", ctypes.c_void_p), ("x_stride", ctypes.c_int64),
        ("norm_weight", ctypes.c_void_p), ("eps", ctypes.c_float),
        ("w", ctypes.c_void_p * 3), ("n", ctypes.c_int32 * 3),
        ("res", ctypes.c_void_p), ("res_stride", ctypes.c_int64),
        ("y", ctypes.c_void_p), ("y_stride", ctypes.c_int64),
        ("m", ctypes.c_int32), ("k", ctypes.c_int32), ("epilogue", ctypes.c_int32),
    ]


_LOCK = threading.Lock()
_LIB = None


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libbz_gqa_decode.so)")


def compile_commands(objdir: Path) -> list[list[str]]:
    """One hipcc -c command per translation unit (objects into objdir)."""
    sid = source_id()
    return [[hipcc(), *HIPCC_FLAGS, f"-DBZ_BUILD_ID=\"{sid}\"", f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src),
             "-o", str(objdir / (Path(src).stem + ".o"))] for src in SOURCES]


def link_command(objdir: Path, out: Path) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out),
            *[str(objdir / (Path(src).stem + ".o")) for src in SOURCES]]


STAMP_SOURCE = "bench_stamp.hip"
STAMP_PATH = PKG_DIR / "libbz_bench_stamp.so"  # bench.py's GPU timestamp kernel; not part of the C ABI

# The native eager binding (csrc/eager_ext.cpp): a CPython extension module built with g++ against torch's headers,
# host code only, which calls the C ABI functions of the loaded library (eager()).
EAGER_SOURCE = "eager_ext.cpp"
EAGER_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM"]


def eager_path() -> Path:
    import sysconfig

    return PKG_DIR / ("_bz_eager" + sysconfig.get_config_var("EXT_SUFFIX"))


def eager_id() -> str:
    """Hash of what the eager module is built from: its source, the C ABI headers and its flags."""
    h = hashlib.sha256()
    for f in [CSRC / EAGER_SOURCE] + sorted(INCLUDE.glob("*.h")):
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    h.update(" ".join(EAGER_FLAGS).encode())
    return h.hexdigest()[:16]


def eager_command(out: Path) -> list[str]:
    """g++ command for the eager module: torch's headers and libraries, the HIP runtime's headers and library."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    torch_lib = cpp_extension.library_paths()[0]
    incs = [f"-I{d}" for d in cpp_extension.include_paths()] + [f"-I{sysconfig.get_paths()['include']}",
                                                                  f"-I{rocm}/include", f"-I{INCLUDE}"]
    return ["g++", *EAGER_FLAGS, f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
            f"-DBZ_EAGER_BUILD_ID=\"{eager_id()}\"", *incs, str(CSRC / EAGER_SOURCE), "-o", str(out),
            f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", f"-L{rocm}/lib",
            "-lamdhip64", f"-Wl,-rpath,{torch_lib}", f"-Wl,-rpath,{rocm}/lib"]


def build(verbose: bool = False) -> Path:
    """Compile libbz_gqa_decode.so for gfx950 in-tree (always recompiles), bench.py's timestamp helper
    libbz_bench_stamp.so and the native eager binding (_bz_eager). Returns the path of libbz_gqa_decode.so."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="bz_gqa_build_") as d:
        objdir = Path(d)
        cmds = compile_commands(objdir)
        stamp_tmp = STAMP_PATH.with_suffix(".so.tmp")
        cmds.append([hipcc(), *HIPCC_FLAGS, "-shared", str(CSRC / STAMP_SOURCE), "-o", str(stamp_tmp)])
        eager_tmp = objdir / eager_path().name
        cmds.append(eager_command(eager_tmp))

        def run(cmd):
            if verbose:
                print(" ".join(cmd), flush=True)
            return subprocess.run(cmd, capture_output=True, text=True)

        with ThreadPoolExecutor(max_workers=len(cmds)) as pool:
            results = list(pool.map(run, cmds))
        for cmd, res in zip(cmds, results):
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed ({res.returncode}) on {cmd[-3]}:\n{res.stderr[-4000:]}")
        os.replace(stamp_tmp, STAMP_PATH)
        shutil.copyfile(eager_tmp, eager_path().with_suffix(".tmp"))
        os.replace(eager_path().with_suffix(".tmp"), eager_path())
        res = run(link_command(objdir, tmp))
        if res.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{res.stderr[-4000:]}")
    os.replace(tmp, LIB_PATH)  # atomic: a concurrent load() sees the old or the new library, never half of one
    return LIB_PATH


def _declare(lib: ctypes.CDLL) -> None:
    P = ctypes.POINTER
    lib.bz_gqa_decode.argtypes = [P(GqaDecodeArgs), ctypes.c_void_p]
    lib.bz_gqa_decode.restype = ctypes.c_int
    lib.bz_gqa_decode_masked.argtypes = [P(GqaDecodeArgs), ctypes.c_void_p]
    lib.bz_gqa_decode_masked.restype = ctypes.c_int
    lib.bz_gqa_decode_fused.argtypes = [P(GqaDecodeFusedArgs), ctypes.c_void_p]
    lib.bz_gqa_decode_fused.restype = ctypes.c_int
    lib.bz_gqa_decode_workspace_size.argtypes = [ctypes.c_int32] * 7 + [P(ctypes.c_size_t)]
    lib.bz_gqa_decode_workspace_size.restype = ctypes.c_int
    lib.bz_gqa_decode_default_splits.argtypes = [ctypes.c_int32] * 5 + [P(ctypes.c_int32)]
    lib.bz_gqa_decode_default_splits.restype = ctypes.c_int
    lib.bz_status_string.argtypes = [ctypes.c_int]
    lib.bz_status_string.restype = ctypes.c_char_p
    lib.bz_gqa_decode_abi_version.argtypes = []
    lib.bz_gqa_decode_abi_version.restype = ctypes.c_int
    lib.bz_gemv.argtypes = [P(GemvArgs), ctypes.c_void_p]
    lib.bz_gemv.restype = ctypes.c_int
    lib.bz_rmsnorm.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                               ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p]
    lib.bz_rmsnorm.restype = ctypes.c_int
    lib.bz_mask_interval.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.bz_mask_interval.restype = ctypes.c_int
    lib.bz_gqa_decode_wave.argtypes = [P(GqaDecodeArgs), ctypes.c_void_p]
    lib.bz_gqa_decode_wave.restype = ctypes.c_int
    lib.bz_gqa_decode_noalloc.argtypes = [P(GqaDecodeArgs), ctypes.c_void_p]
    lib.bz_gqa_decode_noalloc.restype = ctypes.c_int
    lib.bz_gqa_decode_probs.argtypes = [P(GqaDecodeArgs), ctypes.c_void_p, ctypes.c_void_p]
    lib.bz_gqa_decode_probs.restype = ctypes.c_int
    lib.bz_gqa_decode_fused_probs.argtypes = [P(GqaDecodeFusedArgs), ctypes.c_void_p, ctypes.c_void_p]
    lib.bz_gqa_decode_fused_probs.restype = ctypes.c_int
    lib.bz_gqa_decode_build_id.argtypes = []
    lib.bz_gqa_decode_build_id.restype = ctypes.c_char_p


def load() -> ctypes.CDLL:
    """Open the built library once per process (thread-safe). Raises if it has not been built."""
    global _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; "
                               "g.build()'); there is no non-HIP fallback")
        lib = ctypes.CDLL(str(LIB_PATH))
        if not hasattr(lib, "bz_gqa_decode_build_id"):
            raise RuntimeError(f"{LIB_PATH} predates the build id: rebuild it")
        _declare(lib)
        ver = lib.bz_gqa_decode_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}: rebuild it")
        built, current = lib.bz_gqa_decode_build_id().decode(), source_id()
        if built != current:
            raise RuntimeError(f"{LIB_PATH} was built from other sources or flags (build id {built}, the sources next "
                               f"to it hash to {current}): rebuild it (python -c 'import __graft_entry__ as g; "
                               "g.build()')")
        _LIB = lib
        return lib


_EAGER = None


def eager():
    """The native eager binding, imported once per process and bound to the loaded library's C ABI functions.
    Raises if it is missing or was built from other sources (no fallback)."""
    global _EAGER
    if _EAGER is not None:
        return _EAGER
    with _LOCK:
        if _EAGER is not None:
            return _EAGER
    lib = load()
    import importlib.util

    import torch  # noqa: F401  (the module links against torch's libraries)

    path = eager_path()
    if not path.exists():
        raise RuntimeError(f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    spec = importlib.util.spec_from_file_location("_bz_eager", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    built, current = mod.build_id(), eager_id()
    if built != current:
        raise RuntimeError(f"{path} was built from other sources or flags (build id {built}, the sources next to it "
                           f"hash to {current}): rebuild it (python -c 'import __graft_entry__ as g; g.build()')")
    addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value  # noqa: E731
    mod.bind(addr(lib.bz_gqa_decode), addr(lib.bz_gqa_decode_masked), addr(lib.bz_gqa_decode_noalloc),
             addr(lib.bz_gqa_decode_fused), addr(lib.bz_status_string), addr(lib.bz_gqa_decode_workspace_size),
             addr(lib.bz_gemv), addr(lib.bz_rmsnorm))
    with _LOCK:
        if _EAGER is None:
            _EAGER = mod
    return _EAGER


_TC = None  # torch._C, bound on first use (this module does not import torch at load time)


def run_on(device, launch):
    """launch(stream) with `device` current and `stream` the raw handle of its current stream, as a torch kernel
    launches: what `with torch.cuda.device(device): launch(torch.cuda.current_stream(device).cuda_stream)` does,
    without building a stream object and switching the device only when another one is current (several us less host
    time per call). Returns what launch returns."""
    global _TC
    tc = _TC
    if tc is None:
        import torch

        tc = _TC = torch._C
    prev = tc._cuda_getDevice()
    idx = prev if device.index is None else device.index
    if prev == idx:
        return launch(tc._cuda_getCurrentRawStream(idx))
    tc._cuda_setDevice(idx)
    try:
        return launch(tc._cuda_getCurrentRawStream(idx))
    finally:
        tc._cuda_setDevice(prev)


_DEVICE_REASON: dict = {}


def device_unsupported(index: int | None = None) -> str | None:
    """None if GPU `index` (default: the current one) can run the kernels, else the reason: the library holds gfx950
    code only. The pre-flight of the reference's installer (flash/support.py:67-84), which declines a GPU other than
    the one its kernels were built for; cached per device."""
    import torch

    if not torch.cuda.is_available():
        return "no GPU is visible"
    idx = torch.cuda.current_device() if index is None else int(index)
    reason = _DEVICE_REASON.get(idx, False)
    if reason is False:
        props = torch.cuda.get_device_properties(idx)
        arch = getattr(props, "gcnArchName", "").split(":")[0]
        reason = None if arch == ARCH else f"{props.name} ({arch or 'unknown architecture'}): the kernels are {ARCH} only"
        _DEVICE_REASON[idx] = reason
    return reason


def status_string(code: int) -> str:
    return load().bz_status_string(code).decode()


def check(code: int, what: str) -> None:
    """Map a bz_status to the reference's error behaviour (TORCH_CHECK -> RuntimeError)."""
    if code != 0:
        raise RuntimeError(f"{what}: {status_string(code)} (status {code})")
