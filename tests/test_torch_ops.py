"""CPU: the torch operator registrations (torch_ops.py, namespace "bz"), without running a kernel.

Each entry point is an operator with a CUDA kernel and a fake kernel, whose schema declares exactly the arguments the
call writes as mutable (so that functionalization under torch.compile keeps the writes) and returns nothing. A call on
fake tensors (what dynamo traces with) runs the fake kernel and allocates nothing; a call on CPU tensors has no kernel
to run and fails in the dispatcher instead of reaching the library.
"""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import breeze_tts_2_flash_amd  # noqa: F401  (registers the operators)

# operator -> the arguments it writes
WRITES = {
    "gqa_decode": {"out", "workspace"},
    "gqa_decode_wave": {"out"},
    "gqa_decode_masked": {"out", "workspace"},
    "gqa_decode_fused": {"k_cache", "v_cache", "out", "workspace"},
    "gqa_decode_probs": {"probs"},
    "gemv_seg": {"y"},
    "gemv_resid": {"y"},
    "gemv_gateup": {"y"},
    "rmsnorm": {"y"},
}


@pytest.mark.parametrize("name", sorted(WRITES))
def test_schema_declares_the_writes(name):
    schema = getattr(torch.ops.bz, name).default._schema
    written = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
    assert written == WRITES[name]
    assert len(schema.returns) == 0


@pytest.mark.parametrize("name", sorted(WRITES))
def test_cuda_and_fake_kernels_registered(name):
    op = "bz::" + name
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op, "CUDA")
    assert not torch._C._dispatch_has_kernel_for_dispatch_key(op, "CPU")
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op, "Meta")
    assert torch._library.simple_registry.singleton.find(op).fake_impl.kernel is not None


def _gemv_args(device):
    x = torch.empty(2, 64, dtype=torch.bfloat16, device=device)
    W = torch.empty(32, 64, dtype=torch.bfloat16, device=device)
    res = torch.empty(2, 32, dtype=torch.bfloat16, device=device)
    y = torch.empty(2, 32, dtype=torch.bfloat16, device=device)
    return x, W, res, y


def test_fake_call_runs_without_the_library():
    with FakeTensorMode():
        x, W, res, y = _gemv_args("cpu")
        assert torch.ops.bz.gemv_resid(x, W, res, y) is None
        q = torch.empty(2, 16, 128, dtype=torch.bfloat16)
        kc = torch.empty(2, 8, 64, 128, dtype=torch.bfloat16)
        lens = torch.empty(2, dtype=torch.int32)
        out = torch.empty(2, 16, 128, dtype=torch.bfloat16)
        assert torch.ops.bz.gqa_decode(q, kc, kc, lens, 0.1, out, None, None, 0, 0, 0, None) is None


def test_cpu_tensors_do_not_reach_the_library():
    x, W, res, y = _gemv_args("cpu")
    with pytest.raises(NotImplementedError):
        torch.ops.bz.gemv_resid(x, W, res, y)
