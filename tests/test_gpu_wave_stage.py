"""GPU: the device function attend_wave (csrc/gqa_wave.cuh) as one stage of a multi-stage kernel, with other waves
of the same workgroups busy with unrelated work (tests/csrc/wave_stage.hip: streaming reads and read-modify-writes of a
scratch buffer, wave-local LDS traffic, VALU, no barrier), the way a kernel that runs a whole depth decode step would
call it (flash/csrc/depth_frame.cu:193-272). For every choice of attention waves in the four-wave workgroup, the
outputs equal bz_gqa_decode_wave's (the same function launched alone) bit for bit, and the oracle within the split
kernel's tolerance |out - ref| <= 2e-3 + 1e-2 |ref|; the busy waves' scratch words all change."""
import ctypes

import numpy as np
import pytest
import torch

from breeze_tts_2_flash_amd import attention, gqa_decode_wave
from oracle.attention import decode_attention_tokens
from tests import wave_stage_lib

MASKS = [0b0001, 0b1000, 0b0110, 0b1011, 0b1111]


def bf16(x, device):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).to(device)


def stage(q, k, v, lens, starts, scale, att_mask):
    """The test kernel's output for these inputs; also returns the scratch before and after."""
    lib = wave_stage_lib.load()
    a, out = attention._fill_args(q, k, v, scale, None, 0, 0, "auto")
    a.seq_lens = lens.data_ptr()
    a.kv_start = starts.data_ptr() if starts is not None else None
    words = lib.bz_test_wave_stage_busy_words(ctypes.byref(a), att_mask)
    assert words > 0
    busy = torch.randint(0, 2 ** 31 - 1, (words,), dtype=torch.int32, device=q.device)
    before = busy.clone()
    out.fill_(0)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    rc = lib.bz_test_wave_stage(ctypes.byref(a), att_mask, ctypes.c_void_p(busy.data_ptr()), words,
                                ctypes.c_void_p(stream))
    assert rc == 0
    torch.cuda.synchronize()
    return out, before, busy


def check_oracle(got, q, k, v, lens, starts, scale, what):
    q4 = q if q.dim() == 4 else q[:, :, None]
    g = got if got.dim() == 4 else got[:, None]
    ref = decode_attention_tokens(q4.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                                  lens.cpu().numpy(), scale,
                                  kv_start=None if starts is None else starts.cpu().numpy())
    r = g.float().cpu().numpy()
    excess = np.abs(r - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert excess.max() <= 0, f"{what}: excess {excess.max():.3e}"


CASES = {
    # the real depth shape (8 q / 2 KV heads, head_dim 128) at its longest step
    "depth_8q2kv_d128": dict(B=2, NH=8, NKV=2, D=128, cap=17, lens=[17, 9], starts=None, T=1),
    # config 5's frame shape (16 q / 8 KV heads, head_dim 64), last step
    "config5_16q8kv_d64": dict(B=2, NH=16, NKV=8, D=64, cap=32, lens=[32, 20], starts=None, T=1),
    # longer rows with a left-padding start: several tile pairs per wave
    "long_rows_d128": dict(B=3, NH=4, NKV=2, D=128, cap=320, lens=[300, 65, 0], starts=[7, 0, 0], T=1),
    # the depth transformer's first step: two causal query tokens per row
    "first_step_tokens": dict(B=2, NH=8, NKV=2, D=128, cap=16, lens=[2, 2], starts=None, T=2),
}


@pytest.mark.gpu
@pytest.mark.parametrize("att_mask", MASKS, ids=[f"mask{m:04b}" for m in MASKS])
@pytest.mark.parametrize("case", list(CASES))
def test_attention_stage_beside_busy_waves(device, case, att_mask):
    c = CASES[case]
    rng = np.random.default_rng(sum(map(ord, case)) + att_mask)
    B, NH, NKV, D, cap, T = c["B"], c["NH"], c["NKV"], c["D"], c["cap"], c["T"]
    if T == 1:
        q = bf16(rng.standard_normal((B, NH, D)), device)
    else:  # the transformers layout: [B, NH, T, D] as a view of [B, T, NH, D]
        q = bf16(rng.standard_normal((B, T, NH, D)), device).permute(0, 2, 1, 3)
    k = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    v = bf16(rng.standard_normal((B, NKV, cap, D)), device)
    lens = torch.tensor(c["lens"], dtype=torch.int32, device=device)
    starts = None if c["starts"] is None else torch.tensor(c["starts"], dtype=torch.int32, device=device)
    scale = D ** -0.5
    got, before, busy = stage(q, k, v, lens, starts, scale, att_mask)
    ref = gqa_decode_wave(q, k, v, lens, scale, kv_start=starts)
    torch.cuda.synchronize()
    assert got.shape == ref.shape
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"{case}: differs from bz_gqa_decode_wave"
    check_oracle(got, q, k, v, lens, starts, scale, case)
    # scratch words per (workgroup, wave): 48 per lane; the busy waves rewrote all of theirs, the attention waves none
    grid = busy.numel() // (4 * 48 * 64)
    view_b, view_a = before.view(grid, 4, 48 * 64), busy.view(grid, 4, 48 * 64)
    for w in range(4):
        changed = (view_a[:, w] != view_b[:, w]).float().mean().item()
        if (att_mask >> w) & 1:
            assert changed == 0.0, f"wave {w} runs attention but its scratch changed"
        else:
            assert changed > 0.99, f"busy wave {w}: only {changed:.3f} of its words changed"


@pytest.mark.gpu
def test_stage_argument_errors(device):
    lib = wave_stage_lib.load()
    q = torch.zeros(1, 2, 64, dtype=torch.bfloat16, device=device)
    k = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device=device)
    a, _ = attention._fill_args(q, k, k, 0.125, None, 0, 0, "auto")
    a.seq_lens = torch.ones(1, dtype=torch.int32, device=device).data_ptr()
    assert lib.bz_test_wave_stage_busy_words(ctypes.byref(a), 0) == -1  # no attention wave
    assert lib.bz_test_wave_stage_busy_words(ctypes.byref(a), 16) == -1  # a wave the workgroup does not have
    words = lib.bz_test_wave_stage_busy_words(ctypes.byref(a), 1)
    busy = torch.zeros(words, dtype=torch.int32, device=device)
    assert lib.bz_test_wave_stage(ctypes.byref(a), 1, ctypes.c_void_p(busy.data_ptr()), words - 1, None) == -1


def test_stage_library_loads_and_checks_masks():
    """CPU: the built test library matches its sources and rejects masks with no attention wave or a fifth wave (host
    code only; nothing is launched)."""
    from breeze_tts_2_flash_amd import kernels

    lib = wave_stage_lib.load()
    a = kernels.GqaDecodeArgs()
    a.q = a.k_cache = a.v_cache = a.out = a.seq_lens = 4096  # never dereferenced: only sizes are checked
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.capacity, a.tokens_per_row = 2, 8, 2, 128, 32, 1
    a.q_stride_b, a.q_stride_h, a.out_stride_b, a.out_stride_h = 8 * 128, 128, 8 * 128, 128
    a.kv_stride_b, a.kv_stride_h, a.kv_stride_s = 2 * 32 * 128, 32 * 128, 128
    assert lib.bz_test_wave_stage_busy_words(ctypes.byref(a), 0) == -1
    assert lib.bz_test_wave_stage_busy_words(ctypes.byref(a), 16) == -1
    # 16 items, two attention waves per workgroup: 8 workgroups of 4 waves x 48 words x 64 lanes
    assert lib.bz_test_wave_stage_busy_words(ctypes.byref(a), 0b0101) == 8 * 4 * 48 * 64
