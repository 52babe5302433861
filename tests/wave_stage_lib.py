"""Build and load tests/csrc/libbz_test_wave_stage.so: the test kernel that runs the device function attend_wave as
one stage of a multi-stage kernel (tests/csrc/wave_stage.hip). __graft_entry__.build() compiles it in-tree next to the
library; load() refuses a build whose id differs from the sources (the test source and the library headers it
includes), so a test never runs a stale kernel."""
from __future__ import annotations

import ctypes
import hashlib
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
SOURCE = HERE / "csrc" / "wave_stage.hip"
LIB = HERE / "csrc" / "libbz_test_wave_stage.so"


def _kernels():
    import __graft_entry__

    __graft_entry__.package()
    from breeze_tts_2_flash_amd import kernels

    return kernels


def build_id() -> str:
    """sha256 (16 hex digits) of the test source, the library headers it includes and the hipcc flags."""
    k = _kernels()
    h = hashlib.sha256()
    for f in [SOURCE] + [k.CSRC / n for n in k.HEADERS] + sorted(k.INCLUDE.glob("*.h")):
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    h.update(" ".join(k.HIPCC_FLAGS).encode())
    return h.hexdigest()[:16]


def build(verbose: bool = False) -> Path:
    k = _kernels()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [k.hipcc(), *k.HIPCC_FLAGS, f"-DBZ_TEST_BUILD_ID=\"{build_id()}\"", f"-I{k.INCLUDE}", f"-I{k.CSRC}",
           "-shared", str(SOURCE), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}) on {SOURCE}:\n{res.stderr[-4000:]}")
    tmp.replace(LIB)
    return LIB


_LIB = None


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(str(LIB))
        lib.bz_test_wave_stage_build_id.restype = ctypes.c_char_p
        got, want = lib.bz_test_wave_stage_build_id().decode(), build_id()
        if got != want:
            raise RuntimeError(f"{LIB} was built from other sources (build id {got}, sources {want}): rebuild it")
        k = _kernels()
        args = ctypes.POINTER(k.GqaDecodeArgs)
        lib.bz_test_wave_stage.argtypes = [args, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        lib.bz_test_wave_stage.restype = ctypes.c_int
        lib.bz_test_wave_stage_busy_words.argtypes = [args, ctypes.c_uint32]
        lib.bz_test_wave_stage_busy_words.restype = ctypes.c_int64
        _LIB = lib
    return _LIB
