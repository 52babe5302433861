"""GQA flash-decoding attention op: gqa_decode(q, k_cache, v_cache, seq_lens, scale) -> out.

The Python-side op shape the reference's call sites use (flash/csrc/bb_attn.cu:416-418: query, kc, vc, mask,
scaling, ...), with seq_lens in the mask's place. Every call goes through the C ABI of libbz_gqa_decode.so
(bz_gqa_decode, include/bz_gqa_decode.h); torch only provides device memory, the current stream and the device
guard. Workspaces are cached per (device, stream), as the reference caches its _workspace (flash/backbone.py:27-37),
so a call allocates nothing once its stream's workspace is large enough and can be recorded into a HIP graph.

Nothing here allocates device memory while the current stream is being captured into a HIP graph: a non-fused call
without a workspace then runs on the library's static scratch (bz_gqa_decode_noalloc), and a fused call without one
raises (pass workspace=, from get_workspace() made before the capture).

Errors follow the reference (TORCH_CHECK -> RuntimeError, bb_attn.cu:377-388, :420-447).
"""
from __future__ import annotations

import ctypes
import functools
import threading

import torch

from . import kernels

_WS: dict = {}            # (device index, raw stream handle, groups) -> workspace
_WS_RETIRED: list = []    # workspaces replaced by larger ones (kept: a captured graph may still use them)
_WS_LOCK = threading.Lock()

_COMBINE = {"auto": kernels.COMBINE_AUTO, "last_block": kernels.COMBINE_LAST_BLOCK, "kernel": kernels.COMBINE_KERNEL}


def _combine_code(combine) -> int:
    if isinstance(combine, int):
        return combine
    if combine not in _COMBINE:
        raise RuntimeError(f"combine must be one of {sorted(_COMBINE)}, got {combine!r}")
    return _COMBINE[combine]


@functools.lru_cache(maxsize=1024)
def _workspace_bytes(device_index: int, batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                     capacity: int, num_splits: int, max_seq_len: int) -> int:
    """bz_gqa_decode_workspace_size, computed with device device_index current (the default split count depends on
    its CU count; -1: an explicit split count, no device needed)."""
    n = ctypes.c_size_t(0)

    def size(_stream=None):
        kernels.check(kernels.load().bz_gqa_decode_workspace_size(batch, num_q_heads, num_kv_heads, head_dim,
                                                                   capacity, num_splits, max_seq_len, ctypes.byref(n)),
                      "bz_gqa_decode_workspace_size")
    if device_index >= 0:
        kernels.run_on(torch.device("cuda", device_index), size)
    else:
        size()
    return int(n.value)


def workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, capacity: int,
                    num_splits: int = 0, max_seq_len: int = 0) -> int:
    """Scratch bytes bz_gqa_decode needs (bz_gqa_decode_workspace_size). num_splits=0 needs a current device."""
    # the default split count depends on the device's CU count: the cached size is per device
    dev = torch.cuda.current_device() if num_splits == 0 and torch.cuda.is_available() else -1
    return _workspace_bytes(dev, batch, num_q_heads, num_kv_heads, head_dim, capacity, num_splits, max_seq_len)


def default_splits(batch: int, num_kv_heads: int, head_dim: int, capacity: int, max_seq_len: int = 0) -> int:
    """Split count the library picks when num_splits=0 (needs a current device for its CU count)."""
    n = ctypes.c_int32(0)
    kernels.check(kernels.load().bz_gqa_decode_default_splits(batch, num_kv_heads, head_dim, capacity, max_seq_len,
                                                               ctypes.byref(n)), "bz_gqa_decode_default_splits")
    return int(n.value)


def get_workspace(device: torch.device, batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                  capacity: int, num_splits: int = 0, max_seq_len: int = 0) -> torch.Tensor:
    """The zero-filled scratch of the device's current stream for calls with batch * num_kv_heads groups (batch counts
    rows times query tokens), at least as large as these sizes need.

    A workspace begins with the arrival counters of those groups, which every call leaves at zero, and the rest is
    written before it is read, so one workspace serves every call with the same groups, whatever its split count,
    capacity or length. There is one per (device, stream, groups), because calls in flight on two streams must not
    share counters and partials. A call that needs more room replaces it with a zeroed one at least twice as large;
    the replaced one stays allocated (a captured graph may still use it), so the memory held stays under twice the
    largest need. Call this before capturing a graph that makes fused calls, and pass the result as workspace=:
    nothing is allocated while a stream is being captured (a non-fused call without a workspace then runs on the
    library's static scratch instead)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return kernels.run_on(torch.device("cuda", idx), lambda stream: _stream_workspace(
        idx, stream, batch, num_q_heads, num_kv_heads, head_dim, capacity, num_splits, max_seq_len))


def _stream_workspace(idx: int, stream: int, batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                      capacity: int, num_splits: int, max_seq_len: int) -> torch.Tensor:
    """get_workspace for device idx (current) and the raw handle of its current stream."""
    n = _workspace_bytes(idx if num_splits == 0 else -1, batch, num_q_heads, num_kv_heads, head_dim, capacity,
                         num_splits, max_seq_len)
    key = (idx, stream, batch * num_kv_heads)
    ws = _WS.get(key)
    if ws is not None and ws.numel() >= n:
        kernels.eager().register_workspace(idx, stream, batch * num_kv_heads, ws)
        return ws
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            f"gqa_decode: no workspace of {n} bytes exists for the stream being captured, and nothing is allocated "
            "during a capture: pass workspace= (attention.get_workspace(...), made before the capture)")
    with _WS_LOCK:
        ws = _WS.get(key)
        if ws is None or ws.numel() < n:
            size = n if ws is None else max(n, 2 * ws.numel())
            new = _zeroed_outside_pools(size, idx)
            if new.data_ptr() % 256:
                raise RuntimeError("workspace allocation is not 256-byte aligned")
            if ws is not None:
                _WS_RETIRED.append(ws)
            _WS[key] = ws = new
        kernels.eager().register_workspace(idx, stream, batch * num_kv_heads, ws)  # the native path's lookup
        return ws


def _zeroed_outside_pools(nbytes: int, idx: int) -> torch.Tensor:
    """A zero-filled uint8 tensor of nbytes on device idx, allocated by a helper thread: torch.compile's CUDA-graph
    trees route every allocation of the thread that warms a graph up into that graph's private pool, and a workspace
    cached across calls must not live there (the trees check that the pool holds only the graph's outputs). The zero
    fill runs on a stream of the helper thread and has completed when this returns."""
    box = []

    def make():
        try:
            dev = torch.device("cuda", idx)
            side = torch.cuda.Stream(dev)
            with torch.cuda.stream(side):
                t = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
            side.synchronize()
            box.append(t)
        except BaseException as e:  # re-raised in the calling thread
            box.append(e)

    th = threading.Thread(target=make, name="bz-workspace")
    th.start()
    th.join()
    if isinstance(box[0], BaseException):
        raise box[0]
    return box[0]


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _q_view(q: torch.Tensor) -> tuple[int, int, int, int, int, int, int]:
    """(B, NH, T, D, stride_b, stride_h, stride_t) of a query given as [B, NH, D] or [B, NH, T, D] (the transformers
    layout, query tokens in dim 2; T = 1 for a plain decode step)."""
    if q.dim() == 4:
        return q.size(0), q.size(1), q.size(2), q.size(3), q.stride(0), q.stride(1), q.stride(2)
    _check(q.dim() == 3, f"query must be [B, NH, D] or [B, NH, T, D], got shape {tuple(q.shape)}")
    return q.size(0), q.size(1), 1, q.size(2), q.stride(0), q.stride(1), 0


def _out_view(out: torch.Tensor, B: int, NH: int, T: int, D: int) -> tuple[int, int, int]:
    """(stride_b, stride_h, stride_t) of an output given as [B, T, NH, D] (the reference's layout, T = 1 for
    attn_decode) or [B, NH, T, D]; with T = 1 also [B, NH, D]."""
    _check(out.dtype == torch.bfloat16, "out must be bf16")
    _check(out.stride(-1) == 1, "out's last dimension must be contiguous")
    if out.dim() == 4 and tuple(out.shape) == (B, T, NH, D):
        return out.stride(0), out.stride(2), out.stride(1)
    if out.dim() == 4 and tuple(out.shape) == (B, NH, T, D):
        return out.stride(0), out.stride(1), out.stride(2)
    _check(T == 1 and out.dim() == 3 and tuple(out.shape) == (B, NH, D),
           f"out must be [B, T, NH, D], [B, NH, T, D] or (T = 1) [B, NH, D] with B={B}, T={T}, NH={NH}, D={D}")
    return out.stride(0), out.stride(1), 0


def _mask_view(mask: torch.Tensor, B: int, cap: int) -> tuple[int, int]:
    """(bz_mask_dtype, batch stride) of an additive mask [B or 1, 1, 1, >= cap] / [B or 1, >= cap]."""
    _check(mask.dtype in (torch.bfloat16, torch.float32), "mask dtype must be bf16 or float32")
    _check(mask.stride(-1) == 1 and mask.size(-1) >= cap, "mask's last dim must be contiguous and >= capacity")
    _check(all(s == 1 for s in mask.shape[1:-1]), f"mask must be [B or 1, 1, 1, S], got {tuple(mask.shape)}")
    _check(mask.size(0) in (B, 1), "mask batch dim must be B or 1")
    code = kernels.MASK_BF16 if mask.dtype == torch.bfloat16 else kernels.MASK_F32
    return code, (0 if mask.size(0) == 1 else mask.stride(0))


_ARGS: dict = {}  # layout of a call (shapes, strides, dtypes, devices, scalars) -> (checked argument bytes, out shape)


def _fill_args(q, k_cache, v_cache, scale, out, num_splits, max_seq_len, combine):
    """The bz_gqa_decode_args of a call (pointers of q, k_cache, v_cache and out filled in; ranges, mask and workspace
    left to the caller) and its output tensor (allocated when out is None). The checks depend only on the tensors'
    layout, so a layout seen before reuses its checked arguments and only the pointers are set."""
    key = (q.shape, q.stride(), q.dtype, q.device, k_cache.shape, k_cache.stride(), k_cache.dtype, k_cache.device,
           v_cache.shape, v_cache.stride(), v_cache.dtype, v_cache.device,
           None if out is None else (out.shape, out.stride(), out.dtype, out.device),
           scale, num_splits, max_seq_len, combine)
    hit = _ARGS.get(key)
    if hit is None:
        a, out = _check_args(q, k_cache, v_cache, scale, out, num_splits, max_seq_len, combine)
        if len(_ARGS) >= 512:
            _ARGS.clear()
        _ARGS[key] = (bytes(a), tuple(out.shape))
        return a, out
    a = kernels.GqaDecodeArgs.from_buffer_copy(hit[0])
    if out is None:
        out = torch.empty(hit[1], dtype=torch.bfloat16, device=q.device)
    a.q, a.k_cache, a.v_cache, a.out = q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr()
    return a, out


def _check_args(q, k_cache, v_cache, scale, out, num_splits, max_seq_len, combine):
    _check(q.is_cuda, "query must be a device tensor")
    _check(q.dtype == torch.bfloat16 and k_cache.dtype == torch.bfloat16 and v_cache.dtype == torch.bfloat16,
           "query, k_cache and v_cache must be bf16")
    _check(k_cache.device == q.device and v_cache.device == q.device, "all tensors must be on one device")
    _check(q.stride(-1) == 1, "query's head_dim must be contiguous")
    B, NH, T, D, q_sb, q_sh, q_st = _q_view(q)
    _check(k_cache.dim() == 4 and v_cache.shape == k_cache.shape and v_cache.stride() == k_cache.stride(),
           "k_cache and v_cache must be [B, NKV, capacity, D] with equal shapes and strides")
    _check(k_cache.size(0) == B and k_cache.size(3) == D and k_cache.stride(3) == 1,
           f"k_cache {tuple(k_cache.shape)} does not match query {tuple(q.shape)}")
    NKV, cap = k_cache.size(1), k_cache.size(2)
    if out is None:
        shape = (B, NH, D) if T == 1 else (B, T, NH, D)
        out = torch.empty(shape, dtype=torch.bfloat16, device=q.device)
    _check(out.device == q.device, "out must be on the query's device")
    o_sb, o_sh, o_st = _out_view(out, B, NH, T, D)
    a = kernels.GqaDecodeArgs()
    a.q, a.q_stride_b, a.q_stride_h = q.data_ptr(), q_sb, q_sh
    a.tokens_per_row, a.q_stride_t, a.out_stride_t = T, q_st, o_st
    a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    a.kv_stride_b, a.kv_stride_h, a.kv_stride_s = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.scale = float(scale)
    a.out, a.out_stride_b, a.out_stride_h = out.data_ptr(), o_sb, o_sh
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.capacity = B, NH, NKV, D, cap
    a.num_splits, a.max_seq_len, a.combine = int(num_splits), int(max_seq_len), _combine_code(combine)
    return a, out


def _int32_rows(t: torch.Tensor, B: int, name: str, device) -> torch.Tensor:
    _check(t.dtype == torch.int32 and t.device == device and t.numel() == B and t.is_contiguous(),
           f"{name} must be a contiguous int32 device tensor of {B} elements")
    return t


def _run(a, dev, workspace, entry: str) -> None:
    """Launches bz_gqa_decode or bz_gqa_decode_masked (entry) on the device's current stream.

    Without a workspace, a call made while that stream is being captured into a HIP graph (a torch.cuda.graph, or
    torch.compile's CUDA-graph trees recording) goes to bz_gqa_decode_noalloc: it uses the library's static per-device
    scratch and allocates nothing. The graph then holds that scratch: its replays must not overlap in time with other
    calls on the scratch on the same device. Sizes beyond the scratch (BZ_ERR_SCRATCH) raise under capture. Any other
    call without a workspace takes the cached workspace of its (device, stream)."""
    lib = kernels.load()

    def launch(stream):
        sp = ctypes.c_void_p(stream)
        if workspace is None and torch.cuda.is_current_stream_capturing():
            if entry == "bz_gqa_decode_masked":
                a.seq_lens, a.kv_start = None, None  # the noalloc entry takes the range from the mask
            kernels.check(lib.bz_gqa_decode_noalloc(ctypes.byref(a), sp),
                          "bz_gqa_decode_noalloc (a call captured without workspace=; pass one for these sizes)")
            return
        ws = workspace if workspace is not None else _stream_workspace(
            dev.index, stream, a.batch * max(1, a.tokens_per_row), a.num_q_heads, a.num_kv_heads, a.head_dim,
            a.capacity, a.num_splits, a.max_seq_len)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()
        kernels.check(getattr(lib, entry)(ctypes.byref(a), sp), entry)

    kernels.run_on(dev, launch)


def _default_out(q: torch.Tensor) -> torch.Tensor:
    """The output a call allocates when none is given: [B, NH, D] for one query token, [B, T, NH, D] for T > 1."""
    B, NH = q.size(0), q.size(1)
    if q.dim() == 4 and q.size(2) > 1:
        return torch.empty(B, q.size(2), NH, q.size(3), dtype=torch.bfloat16, device=q.device)
    return torch.empty(B, NH, q.size(-1), dtype=torch.bfloat16, device=q.device)


def gqa_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, seq_lens: torch.Tensor,
               scale: float, out: torch.Tensor | None = None, *, kv_start: torch.Tensor | None = None,
               mask: torch.Tensor | None = None, num_splits: int = 0, max_seq_len: int = 0,
               combine: str | int = "auto", workspace: torch.Tensor | None = None) -> torch.Tensor:
    """GQA decode attention over [kv_start[b], seq_lens[b]) of a bf16 KV cache.

    q: [B, NH, D] or [B, NH, T, D] bf16 (head_dim contiguous); k_cache, v_cache: [B, NKV, capacity, D] bf16;
    seq_lens: [B] int32 (exclusive end); kv_start: [B] int32 or None; mask: optional additive mask
    [B or 1, 1, 1, >= capacity] (bf16 or fp32) applied inside the range (<= -1e30 excludes a position);
    out: [B, NH, D] (default for T = 1), [B, T, NH, D] (default for T > 1) or [B, NH, T, D] bf16. Returns out.
    With T > 1 query tokens, row b's tokens are its last T positions, causal among themselves: token t attends
    [kv_start[b], seq_lens[b] - (T - 1 - t)) (the depth transformer's first step, depth_frame.cu:221-227).
    Under torch.compile the call is the registered operator torch.ops.bz.gqa_decode (one opaque graph node).
    """
    if torch.compiler.is_compiling():
        out = _default_out(q) if out is None else out
        torch.ops.bz.gqa_decode(q, k_cache, v_cache, seq_lens, float(scale), out, kv_start, mask, int(num_splits),
                                int(max_seq_len), _combine_code(combine), workspace)
        return out
    return _gqa_decode(q, k_cache, v_cache, seq_lens, scale, out, kv_start, mask, num_splits, max_seq_len, combine,
                       workspace)


def _gqa_decode(q, k_cache, v_cache, seq_lens, scale, out, kv_start, mask, num_splits, max_seq_len, combine,
                workspace) -> torch.Tensor:
    """gqa_decode's call through the C ABI (the body of the eager path and of torch.ops.bz.gqa_decode): the native
    binding when the stream's workspace exists (or none is needed), else here, which makes it."""
    r = kernels.eager().decode(q, k_cache, v_cache, seq_lens, kv_start, mask, out, scale, num_splits, max_seq_len,
                               combine, workspace, False)
    if r is not None:
        return r
    a, out = _fill_args(q, k_cache, v_cache, scale, out, num_splits, max_seq_len, combine)
    dev = q.device
    a.seq_lens = _int32_rows(seq_lens, a.batch, "seq_lens", dev).data_ptr()
    a.kv_start = _int32_rows(kv_start, a.batch, "kv_start", dev).data_ptr() if kv_start is not None else None
    if mask is not None:
        _check(mask.device == dev, "mask must be on the query's device")
        a.mask_dtype, a.mask_stride_b = _mask_view(mask, a.batch, a.capacity)
        a.mask = mask.data_ptr()
    _run(a, dev, workspace, "bz_gqa_decode")
    return out


def gqa_decode_wave(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, seq_lens: torch.Tensor,
                    scale: float, out: torch.Tensor | None = None, *,
                    kv_start: torch.Tensor | None = None) -> torch.Tensor:
    """gqa_decode computed by one wave per (row, token, q head) (bz_gqa_decode_wave: the device function attend_wave
    launched alone; no split, no workspace). Same shapes and ranges as gqa_decode (no mask); out must be 16-byte
    aligned with strides that are multiples of 8 elements. Faster than gqa_decode only on short rows already cached
    (the real depth shape); it exists to test and time the device function a whole-step depth kernel would call.
    Under torch.compile the call is the registered operator torch.ops.bz.gqa_decode_wave."""
    if torch.compiler.is_compiling():
        out = _default_out(q) if out is None else out
        torch.ops.bz.gqa_decode_wave(q, k_cache, v_cache, seq_lens, float(scale), out, kv_start)
        return out
    return _gqa_decode_wave(q, k_cache, v_cache, seq_lens, scale, out, kv_start)


def _gqa_decode_wave(q, k_cache, v_cache, seq_lens, scale, out, kv_start) -> torch.Tensor:
    """gqa_decode_wave's call through the C ABI."""
    a, out = _fill_args(q, k_cache, v_cache, scale, out, 0, 0, "auto")
    dev = q.device
    a.seq_lens = _int32_rows(seq_lens, a.batch, "seq_lens", dev).data_ptr()
    a.kv_start = _int32_rows(kv_start, a.batch, "kv_start", dev).data_ptr() if kv_start is not None else None
    kernels.run_on(dev, lambda stream: kernels.check(
        kernels.load().bz_gqa_decode_wave(ctypes.byref(a), ctypes.c_void_p(stream)), "bz_gqa_decode_wave"))
    return out


def gqa_decode_masked(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, mask: torch.Tensor,
                      scale: float, out: torch.Tensor | None = None, *, num_splits: int = 0, max_seq_len: int = 0,
                      combine: str | int = "auto", workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Interval-mask form (bz_gqa_decode_masked): each row's range is the first..last position with mask > -1e30,
    derived on the device; the mask is added inside that range. Same shapes as gqa_decode. Under torch.compile the
    call is the registered operator torch.ops.bz.gqa_decode_masked."""
    if torch.compiler.is_compiling():
        out = _default_out(q) if out is None else out
        torch.ops.bz.gqa_decode_masked(q, k_cache, v_cache, mask, float(scale), out, int(num_splits), int(max_seq_len),
                                       _combine_code(combine), workspace)
        return out
    return _gqa_decode_masked(q, k_cache, v_cache, mask, scale, out, num_splits, max_seq_len, combine, workspace)


def _gqa_decode_masked(q, k_cache, v_cache, mask, scale, out, num_splits, max_seq_len, combine,
                       workspace) -> torch.Tensor:
    """gqa_decode_masked's call through the C ABI (the native binding first, as in _gqa_decode)."""
    r = kernels.eager().decode(q, k_cache, v_cache, None, None, mask, out, scale, num_splits, max_seq_len, combine,
                               workspace, True)
    if r is not None:
        return r
    a, out = _fill_args(q, k_cache, v_cache, scale, out, num_splits, max_seq_len, combine)
    dev = q.device
    _check(mask.device == dev, "mask must be on the query's device")
    a.mask_dtype, a.mask_stride_b = _mask_view(mask, a.batch, a.capacity)
    a.mask = mask.data_ptr()
    _run(a, dev, workspace, "bz_gqa_decode_masked")
    return out


def _check_probs(probs: torch.Tensor, a, dev) -> None:
    n = a.batch * a.num_q_heads * a.capacity
    _check(probs.dtype == torch.float32 and probs.device == dev and probs.is_contiguous() and probs.numel() >= n,
           f"probs (dbg) must be a contiguous float32 tensor on the query's device with at least B * NH * capacity = "
           f"{n} elements")


def gqa_decode_probs(q: torch.Tensor, k_cache: torch.Tensor, seq_lens: torch.Tensor | None, scale: float,
                     probs: torch.Tensor | None = None, *, kv_start: torch.Tensor | None = None,
                     mask: torch.Tensor | None = None) -> torch.Tensor:
    """The softmax probabilities of the gqa_decode call with these arguments (bz_gqa_decode_probs): float32
    [B, NH, capacity], each bf16(exp(s - max) / sum) inside the row's range and 0 at excluded positions and outside
    it. seq_lens None: the range comes from the mask, as in gqa_decode_masked. The reference's optional dbg output of
    attn_decode (bb_attn.cu:74, :288-289); a verification path, not a fast one. q: [B, NH, D] (one query token).
    Under torch.compile the call is the registered operator torch.ops.bz.gqa_decode_probs."""
    _check(q.dim() == 3 or (q.dim() == 4 and q.size(2) == 1), "gqa_decode_probs takes one query token per row")
    if probs is None:
        probs = torch.empty(q.size(0), q.size(1), k_cache.size(2), dtype=torch.float32, device=q.device)
    if torch.compiler.is_compiling():
        torch.ops.bz.gqa_decode_probs(q, k_cache, seq_lens, float(scale), probs, kv_start, mask)
        return probs
    return _gqa_decode_probs(q, k_cache, seq_lens, scale, probs, kv_start, mask)


def _gqa_decode_probs(q, k_cache, seq_lens, scale, probs, kv_start, mask) -> torch.Tensor:
    """gqa_decode_probs's call through the C ABI. The probabilities need neither V nor an output: k_cache stands in
    for v_cache and q for out in the argument struct (same shapes and layout checks; neither is read or written)."""
    a, _ = _fill_args(q, k_cache, k_cache, scale, q, 0, 0, "auto")
    dev = q.device
    if seq_lens is not None:
        a.seq_lens = _int32_rows(seq_lens, a.batch, "seq_lens", dev).data_ptr()
        a.kv_start = _int32_rows(kv_start, a.batch, "kv_start", dev).data_ptr() if kv_start is not None else None
    else:
        _check(mask is not None, "gqa_decode_probs needs seq_lens or a mask")
    if mask is not None:
        _check(mask.device == dev, "mask must be on the query's device")
        a.mask_dtype, a.mask_stride_b = _mask_view(mask, a.batch, a.capacity)
        a.mask = mask.data_ptr()
    _check_probs(probs, a, dev)
    kernels.run_on(dev, lambda stream: kernels.check(kernels.load().bz_gqa_decode_probs(
        ctypes.byref(a), ctypes.c_void_p(probs.data_ptr()), ctypes.c_void_p(stream)), "bz_gqa_decode_probs"))
    return probs


def mask_interval(mask: torch.Tensor, capacity: int, batch: int | None = None,
                  seq_lens: torch.Tensor | None = None,
                  kv_start: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(seq_lens, kv_start): per row, the interval [kv_start, seq_lens) of positions < capacity whose mask value is
    > -1e30 (bz_mask_interval), the range gqa_decode_masked derives on the device, computed once for the layers of
    a decode step that share the mask. mask: [B or 1, 1, 1, >= capacity] bf16 / fp32 (or [B or 1, >= capacity]);
    batch defaults to the mask's; seq_lens / kv_start: optional int32 [B] device outputs. Returns them."""
    _check(mask.is_cuda, "mask must be a device tensor")
    B = mask.size(0) if batch is None else int(batch)
    code, stride_b = _mask_view(mask, B, capacity)
    dev = mask.device
    if seq_lens is None:
        seq_lens = torch.empty(B, dtype=torch.int32, device=dev)
    if kv_start is None:
        kv_start = torch.empty(B, dtype=torch.int32, device=dev)
    _int32_rows(seq_lens, B, "seq_lens", dev)
    _int32_rows(kv_start, B, "kv_start", dev)
    kernels.run_on(dev, lambda stream: kernels.check(kernels.load().bz_mask_interval(
        mask.data_ptr(), code, stride_b, B, int(capacity), seq_lens.data_ptr(), kv_start.data_ptr(),
        ctypes.c_void_p(stream)), "bz_mask_interval"))
    return seq_lens, kv_start


def gqa_decode_fused(qkv: torch.Tensor, q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                     cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     cache_pos: torch.Tensor, scale: float, out: torch.Tensor | None = None, *,
                     seq_lens: torch.Tensor | None = None, kv_start: torch.Tensor | None = None,
                     mask: torch.Tensor | None = None, num_splits: int = 0, max_seq_len: int = 0,
                     combine: str | int = "auto", workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Fused decode step (bz_gqa_decode_fused; the reference's attn_decode_fused, bb_attn.cu:433-460).

    qkv: [B, (NH + 2 NKV) * D] bf16 raw q | k | v projections; q_norm_weight, k_norm_weight: [D] bf16; cos, sin:
    [B, D] or [B, 1, D] bf16; cache_pos: int64 device tensor whose first element is the cache slot that receives the
    new k (q_norm/k_norm + RoPE applied) and v of every row. Then attends like gqa_decode over [kv_start, seq_lens),
    or, with seq_lens=None, over the interval of `mask` (required then). head_dim 128. Under torch.compile the call
    is the registered operator torch.ops.bz.gqa_decode_fused (it writes out and the two caches).
    """
    if torch.compiler.is_compiling():
        if out is None:
            NKV, D = k_cache.size(1), k_cache.size(3)
            out = torch.empty(qkv.size(0), qkv.size(1) // D - 2 * NKV, D, dtype=torch.bfloat16, device=qkv.device)
        torch.ops.bz.gqa_decode_fused(qkv, q_norm_weight, k_norm_weight, float(eps), cos, sin, k_cache, v_cache,
                                      cache_pos, float(scale), out, seq_lens, kv_start, mask, int(num_splits),
                                      int(max_seq_len), _combine_code(combine), workspace)
        return out
    return _gqa_decode_fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale,
                             out, seq_lens, kv_start, mask, num_splits, max_seq_len, combine, workspace)


_FUSED: dict = {}  # layout of a fused call -> (checked GqaDecodeFusedArgs bytes, out shape)


def _layout(t):
    return None if t is None else (t.shape, t.stride(), t.dtype, t.device)


def _fused_args(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale, out, seq_lens,
                kv_start, mask, num_splits, max_seq_len, combine):
    """The bz_gqa_decode_fused_args of a call (every pointer but the workspace's filled in) and its output tensor
    (allocated when out is None). The checks depend only on the tensors' layout (shapes, strides, dtypes, devices) and
    the scalars, so a layout seen before reuses its checked arguments and only the pointers are set."""
    key = (qkv.shape, qkv.stride(), qkv.dtype, qkv.device, k_cache.shape, k_cache.stride(), k_cache.dtype,
           k_cache.device, v_cache.shape, v_cache.stride(), v_cache.dtype, v_cache.device, _layout(q_norm_weight),
           _layout(k_norm_weight), _layout(cos), _layout(sin), _layout(cache_pos), _layout(out), _layout(seq_lens),
           _layout(kv_start), _layout(mask), eps, scale, num_splits, max_seq_len, combine)
    hit = _FUSED.get(key)
    if hit is not None:
        f = kernels.GqaDecodeFusedArgs.from_buffer_copy(hit[0])
        if out is None:
            out = torch.empty(hit[1], dtype=torch.bfloat16, device=qkv.device)
        a = f.base  # shares f's memory
        a.q = f.qkv = qkv.data_ptr()
        a.k_cache, a.v_cache, a.out = k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr()
        if seq_lens is not None:
            a.seq_lens = seq_lens.data_ptr()
            a.kv_start = kv_start.data_ptr() if kv_start is not None else None
        if mask is not None:
            a.mask = mask.data_ptr()
        f.q_norm_weight, f.k_norm_weight = q_norm_weight.data_ptr(), k_norm_weight.data_ptr()
        f.cos, f.sin, f.cache_pos = cos.data_ptr(), sin.data_ptr(), cache_pos.data_ptr()
        return f, out
    _check(qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.dtype == torch.bfloat16,
           "qkv must be a bf16 [B, (NH + 2 NKV) * D] tensor with a contiguous last dim")
    _check(k_cache.dim() == 4, "k_cache must be [B, NKV, capacity, D]")
    B, NKV, D = qkv.size(0), k_cache.size(1), k_cache.size(3)
    NH = qkv.size(1) // D - 2 * NKV
    _check(NH > 0 and qkv.size(1) == (NH + 2 * NKV) * D, f"qkv width {qkv.size(1)} is not (NH + 2*{NKV}) * {D}")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        _check(w.dtype == torch.bfloat16 and w.numel() == D and w.is_contiguous() and w.device == qkv.device,
               f"{name} must be a contiguous bf16 [{D}] tensor on the qkv device")
    for name, t in (("cos", cos), ("sin", sin)):
        _check(t.dtype == torch.bfloat16 and t.stride(-1) == 1 and t.size(0) == B and t.size(-1) == D and
               t.numel() == B * D and t.device == qkv.device, f"{name} must be bf16 [B, D] or [B, 1, D]")
    _check(cos.stride(0) == sin.stride(0), "cos and sin must share their batch stride")
    _check(cache_pos.dtype == torch.int64 and cache_pos.numel() >= 1 and cache_pos.device == qkv.device,
           "cache_pos must be an int64 device tensor")
    q_view = qkv[:, :NH * D].view(B, NH, D)
    a, out = _fill_args(q_view, k_cache, v_cache, scale, out, num_splits, max_seq_len, combine)
    dev = qkv.device
    if seq_lens is not None:
        a.seq_lens = _int32_rows(seq_lens, B, "seq_lens", dev).data_ptr()
        a.kv_start = _int32_rows(kv_start, B, "kv_start", dev).data_ptr() if kv_start is not None else None
    else:
        _check(mask is not None, "gqa_decode_fused needs seq_lens or an interval mask")
    if mask is not None:
        _check(mask.device == dev, "mask must be on the qkv device")
        a.mask_dtype, a.mask_stride_b = _mask_view(mask, a.batch, a.capacity)
        a.mask = mask.data_ptr()
    f = kernels.GqaDecodeFusedArgs()
    f.base = a
    f.qkv, f.qkv_stride_b = qkv.data_ptr(), qkv.stride(0)
    f.q_norm_weight, f.k_norm_weight, f.eps = q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), float(eps)
    f.cos, f.sin, f.rope_stride_b = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    f.cache_pos = cache_pos.data_ptr()
    if len(_FUSED) >= 512:
        _FUSED.clear()
    _FUSED[key] = (bytes(f), tuple(out.shape))
    return f, out


def _gqa_decode_fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale, out,
                      seq_lens, kv_start, mask, num_splits, max_seq_len, combine, workspace,
                      probs=None) -> torch.Tensor:
    """gqa_decode_fused's call through the C ABI; with probs (float32 [B, NH, capacity]), then the step's softmax
    probabilities into it (bz_gqa_decode_fused_probs: the reference's dbg output of attn_decode_fused). Without probs
    the native binding runs the call when the stream's workspace exists (or one is passed)."""
    if probs is None:
        r = kernels.eager().fused(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos,
                                  scale, out, seq_lens, kv_start, mask, num_splits, max_seq_len, combine, workspace)
        if r is not None:
            return r
    f, out = _fused_args(qkv, q_norm_weight, k_norm_weight, eps, cos, sin, k_cache, v_cache, cache_pos, scale, out,
                         seq_lens, kv_start, mask, num_splits, max_seq_len, combine)
    a = f.base
    dev = qkv.device
    if probs is not None:
        _check_probs(probs, a, dev)
    lib = kernels.load()

    def launch(stream):
        # _stream_workspace raises rather than allocate while the stream is being captured (the fused entry has no
        # static-scratch form: pass workspace= to capture it)
        ws = workspace if workspace is not None else _stream_workspace(
            dev.index, stream, a.batch * max(1, a.tokens_per_row), a.num_q_heads, a.num_kv_heads, a.head_dim,
            a.capacity, a.num_splits, a.max_seq_len)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()  # a shares f's memory
        sp = ctypes.c_void_p(stream)
        kernels.check(lib.bz_gqa_decode_fused(ctypes.byref(f), sp), "bz_gqa_decode_fused")
        if probs is not None:
            kernels.check(lib.bz_gqa_decode_fused_probs(ctypes.byref(f), ctypes.c_void_p(probs.data_ptr()), sp),
                          "bz_gqa_decode_fused_probs")

    kernels.run_on(dev, launch)
    return out
