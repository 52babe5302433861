"""GPU: bz_gqa_decode_noalloc, through the C ABI, against bz_gqa_decode (the same kernels with a caller workspace), bit
for bit: two calls in a row, the second with a smaller input (fewer rows, a shorter cache and fewer splits), so the
second call's counters and partials lie on what the first left in the static scratch; the mask form (seq_lens NULL)
against bz_gqa_decode_masked; sizes beyond the scratch are refused with BZ_ERR_SCRATCH before anything is launched."""
import ctypes

import pytest
import torch

from breeze_tts_2_flash_amd import attention, gqa_decode, gqa_decode_masked, kernels
from oracle.attention import interval_mask
from tests.test_gpu_parity import assert_close, oracle, rand_case

pytestmark = pytest.mark.gpu

BZ_ERR_SCRATCH = -10


def noalloc(q, k, v, seq_lens, scale, *, kv_start=None, mask=None, num_splits=0):
    """One bz_gqa_decode_noalloc call through the C ABI (no workspace). Returns (status, out)."""
    a, out = attention._fill_args(q, k, v, scale, None, num_splits, 0, "auto")
    if seq_lens is not None:
        a.seq_lens = seq_lens.data_ptr()
        a.kv_start = kv_start.data_ptr() if kv_start is not None else None
    if mask is not None:
        a.mask_dtype, a.mask_stride_b = attention._mask_view(mask, a.batch, a.capacity)
        a.mask = mask.data_ptr()
    a.workspace, a.workspace_bytes = None, 0
    stream = torch.cuda.current_stream(q.device).cuda_stream
    rc = kernels.load().bz_gqa_decode_noalloc(ctypes.byref(a), ctypes.c_void_p(stream))
    return rc, out


def _bits(t):
    return t.view(torch.int16)


def test_noalloc_matches_workspace_entry_twice_shrinking(device):
    big, st_big = rand_case(101, 4, 16, 8, 128, 2048, [2048, 1900, 1024, 333], [0, 7, 0, 100])
    small, _ = rand_case(102, 2, 16, 8, 128, 512, [512, 300])
    for i, (w, st, splits) in enumerate([(big, st_big, 24), (small, None, 4)]):
        print(f"call {i}: B={w.batch} cap={w.capacity} splits={splits}", flush=True)
        g = w.to(device)
        kvs = st.to(device) if st is not None else None
        rc, got = noalloc(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=kvs, num_splits=splits)
        assert rc == 0, kernels.status_string(rc)
        ref = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale, kv_start=kvs, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(ref)), f"call {i}: the no-alloc entry differs from bz_gqa_decode"
        assert_close(got.float().cpu(), oracle(w, kv_start=st), f"call {i}")


def test_noalloc_default_splits_and_mask_form(device):
    w, _ = rand_case(103, 2, 16, 8, 128, 2048, [1500, 1500])
    g = w.to(device)
    rc, got = noalloc(g.q, g.k, g.v, g.seq_lens, g.scale)
    ref = gqa_decode(g.q, g.k, g.v, g.seq_lens, g.scale)
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(_bits(got), _bits(ref))
    mask = interval_mask([0, 21], 1499, 2048).to(device)
    rc, got = noalloc(g.q, g.k, g.v, None, g.scale, mask=mask)
    ref = gqa_decode_masked(g.q, g.k, g.v, mask, g.scale)
    torch.cuda.synchronize()
    assert rc == 0 and torch.equal(_bits(got), _bits(ref))


def test_noalloc_refuses_sizes_beyond_its_scratch(device):
    # 1025 (row, kv head) groups: more counters than the scratch holds
    q = torch.zeros(1025, 8, 64, dtype=torch.bfloat16, device=device)
    kv = torch.zeros(1025, 1, 64, 64, dtype=torch.bfloat16, device=device)
    lens = torch.full((1025,), 64, dtype=torch.int32, device=device)
    rc, _ = noalloc(q, kv, kv, lens, 0.125, num_splits=2)
    assert rc == BZ_ERR_SCRATCH
    # 4 rows, 16 / 8 heads of 128, 256 splits: 4 * 16 * 256 * (128 + 2) * 4 B = 8.5 MB of partials > 8 MiB
    q = torch.zeros(4, 16, 128, dtype=torch.bfloat16, device=device)
    kv = torch.zeros(4, 8, 32768, 128, dtype=torch.bfloat16, device=device)
    lens = torch.full((4,), 32768, dtype=torch.int32, device=device)
    rc, _ = noalloc(q, kv, kv, lens, 0.125, num_splits=256)
    assert rc == BZ_ERR_SCRATCH
    assert "static" in kernels.status_string(rc)
