"""CPU: the parts of bench.py's output that do not need a GPU: the roofline's traffic figure read from the committed
counter summary, the algorithmic byte counts the bench divides by, the streaming-floor sizes of the backbone GEMVs,
and the refusal of more than one GPU."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (no GPU work at import)


def test_traffic_from_committed_profile():
    """The config 2 counter summary gives the HBM bytes per call: at least the algorithmic bytes (every valid K/V
    byte read once) and within 15% above them (split partials and counters only)."""
    from breeze_tts_2_flash_amd import workloads

    algo = workloads.algorithmic_bytes([1024, 1024], 16, 8, 128)
    assert algo == 8_405_000  # K and V of 2 x 8 x 1024 positions, q and out of 2 x 16 heads, 2 lengths
    traffic = bench.traffic_from_profile()
    assert traffic is not None, "profiles/ lacks the config 2 traffic summary"
    assert algo <= traffic <= 1.15 * algo


def test_backbone_gemv_floor_sizes_match_the_model():
    c = bench.BACKBONE
    H, nq, nk, inter = c["H"], c["nq"], c["nk"], c["inter"]
    sizes = bench.BACKBONE_GEMV_BYTES
    assert sizes["gemv_qkv_norm_bytes"] == 2 * (nq + 2 * nk) * H
    assert sizes["gemv_o_resid_bytes"] == 2 * H * nq
    assert sizes["gemv_gateup_norm_silu_bytes"] == 2 * 2 * inter * H
    assert sizes["gemv_down_resid_bytes"] == 2 * H * inter


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_default_arguments_and_modes(monkeypatch):
    """No flags: one GPU, 1000 timed calls after 50 warm-ups, config 2, the library's defaults; the diagnostic modes
    parse to their own flags (none of them is on by default)."""
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    a = bench.parse_args()
    assert (a.gpus, a.steps, a.warmup, a.config, a.splits, a.combine) == (1, 1000, 50, 2, 0, "auto")
    assert not (a.per_call or a.backbone_only or a.depth_only or a.fused or a.eager or a.no_extra or a.no_cpu)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--per-call", "400", "--config", "3"])
    a = bench.parse_args()
    assert (a.per_call, a.config) == (400, 3)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "1", "--steps", "20", "--warmup", "5"])  # the driver's
    a = bench.parse_args()
    assert (a.gpus, a.steps, a.warmup) == (1, 20, 5)
