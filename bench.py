#!/usr/bin/env python3
"""Benchmark of the GQA decode-attention hot path on one MI355X.

A step is one decode-attention call (bz_gqa_decode through the C ABI) over one batch of synthetic, seeded input
(breeze-tts-2-flash_amd/workloads.py). The headline workload is config 2 (backbone serving: B2, 16 q / 8 KV heads,
head_dim 128, capacity 2048, seq_lens 1024); config 3 (KV 4096) is measured in the same run and reported under
"extra", with the depth frame (config 5) and the ragged batch (config 4).

Timing: W untimed eager calls, then K calls recorded into one HIP graph (torch.cuda.CUDAGraph) between two GPU
wall-clock stamps (a one-thread kernel captured before and after them, libbz_bench_stamp.so; two untimed calls at the
head of the graph), replayed once untimed and once timed: the timed region holds exactly the K calls, without the
graph replay's own fixed cost (about 8 us per replay).
Cold: the calls rotate over enough distinct K/V buffer sets that their valid bytes exceed 16 GB (far more than the
256 MB MALL and than the page translations the GPU holds), whatever K is, and a 1 GiB write (untimed) runs right
before the timed replay, so every timed call streams its K/V from HBM, through cold translations, even when K is
smaller than the set count. value = algorithmic bytes per call / (timed µs
per call), in GB/s. The extras (configs 3 and 4, the fused step, the depth frames, the backbone step) use fixed call
counts of their own, independent of K.

The CPU baseline is the reference's PyTorch CPU attention path (repeat_kv + bf16 matmul + fp32 softmax + matmul,
models/breeze.py:259-286, as restated in oracle/attention.py:eager_bf16) on the same workload, timed on this host.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

METRIC = "GQA decode-attn µs/call + HBM GB/s (% of peak) at B=2, KV=1024/4096"
PEAK_HBM_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000, help="timed calls (K)")
    p.add_argument("--warmup", type=int, default=50, help="untimed eager calls before the timed region (W)")
    p.add_argument("--combine", default="auto", choices=["auto", "last_block", "kernel"])
    p.add_argument("--splits", type=int, default=0, help="0 = library default")
    p.add_argument("--eager", action="store_true", help="launch each call from Python instead of a HIP graph")
    p.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4],
                   help="headline workload (BASELINE config; 2 is the metric's serving shape)")
    p.add_argument("--fused", action="store_true",
                   help="time the fused decode step (bz_gqa_decode_fused) instead of attention alone")
    p.add_argument("--no-extra", action="store_true", help="headline workload only")
    p.add_argument("--backbone-only", action="store_true",
                   help="only the 28-layer backbone decode step and its GEMVs (for profiling)")
    p.add_argument("--backbone-m", type=int, nargs="+", default=[2], choices=[1, 2, 4],
                   help="rows of the --backbone-only step (default 2, the CFG pair)")
    p.add_argument("--depth-only", action="store_true",
                   help="only the depth frames: config 5 (split and wave kernels) and the real depth shape")
    p.add_argument("--protocol-only", action="store_true",
                   help="only the protocol floor: the split kernel's K/V traffic without arithmetic, with and without "
                        "its exchange, configs 2-4, beside the kernel's own cold time")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--per-call", type=int, default=0, metavar="N",
                   help="only the distribution of N single cold calls of --config (a GPU stamp before every call)")
    p.add_argument("--traffic-bytes", type=float, default=None,
                   help="HBM bytes per call (overrides the value read from profiles/)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                   help="only run device-to-device copies of BYTES (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


def _pkg():
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import __graft_entry__
    return __graft_entry__.package()


def fused_inputs(w, dev):
    """Raw q | k | v projections, norm weights and RoPE tables for a fused step at slot seq_len - 1 of workload w
    (seeded; the new token of a decode step whose cache already holds seq_len - 1 positions)."""
    import torch

    B, NH, NKV, D = w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim
    L = int(w.seq_lens[0])
    if any(int(x) != L for x in w.seq_lens):
        raise ValueError("a fused step needs one length for every row")
    gen = torch.Generator().manual_seed(100 + L)
    qkv = (torch.randn(B, (NH + 2 * NKV) * D, generator=gen) * 3).to(torch.bfloat16).to(dev)
    qn = (1 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16).to(dev)
    kn = (1 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16).to(dev)
    inv = 1e6 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.cat([(L - 1) * inv] * 2)
    cos = ang.cos().to(torch.bfloat16).expand(B, D).contiguous().to(dev)
    sin = ang.sin().to(torch.bfloat16).expand(B, D).contiguous().to(dev)
    cache_pos = torch.tensor([L - 1], dtype=torch.int64, device=dev)
    return qkv, qn, kn, cos, sin, cache_pos


# Valid K/V bytes the cold calls rotate over. Far more than MI355X's 256 MB MALL, and more than the GPU's page
# translations cover, so that every timed call is cold in both whatever the call count: with 640 MB of sets, 1000
# calls ran config 3 4% faster than 20 calls (the 20 touched each set once after the flush; the 1000 reused warm
# translations); with 16 GB the two agree within about 1%.
ROTATE_BYTES = 16e9
FLUSH_BYTES = 1 << 30       # untimed write right before each timed replay
EXTRA_CALLS = 1000          # timed calls of each extra workload, whatever --steps is
EXTRA_FRAMES = 200          # timed depth frames
BACKBONE_REPS = 100         # timed backbone steps (and replays of each GEMV's 28-layer graph)
BACKBONE_CHAIN = 5          # steps per replay for the back-to-back backbone figure
BACKBONE_REPS_OTHER_M = 30  # timed backbone steps at M = 1 and 4

_FLUSH = {}


def flush_caches(dev):
    """Write FLUSH_BYTES on the current stream: evicts the L2s and the MALL (more than four times their size), and
    keeps the GPU busy for ~150 µs while the host goes on to submit what follows. (A read of another FLUSH_BYTES after
    the write, so that the caches hold clean lines, measured the same.)"""
    import torch

    buf = _FLUSH.get(dev)
    if buf is None:
        buf = _FLUSH[dev] = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    buf.fill_(1)


class GpuStamps:
    """GPU wall-clock stamps taken by a one-thread kernel (libbz_bench_stamp.so) captured into a graph: two of them
    around the timed calls measure those calls alone on the GPU. Events recorded outside a graph would also hold the
    replay's own fixed cost (about 8 us per replay, 0.4 us per call at 20 calls), and ROCm allows no timing events
    inside a captured graph."""

    _lib = None

    def __init__(self, dev, n=2):
        import torch

        GpuStamps.library()
        self.dev = dev
        self.buf = torch.zeros(n, dtype=torch.int64, device=dev)
        khz = ctypes.c_int(0)
        if GpuStamps._lib.bz_bench_stamp_rate_khz(ctypes.byref(khz)) != 0 or khz.value <= 0:
            raise RuntimeError("bz_bench_stamp_rate_khz failed")
        self.us_per_tick = 1e3 / khz.value

    @staticmethod
    def library():
        from breeze_tts_2_flash_amd import kernels

        if GpuStamps._lib is None:
            lib = ctypes.CDLL(str(kernels.STAMP_PATH))
            lib.bz_bench_stamp.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
            lib.bz_bench_stamp_rate_khz.argtypes = [ctypes.POINTER(ctypes.c_int)]
            lib.bz_bench_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p,
                                                 ctypes.c_void_p]
            GpuStamps._lib = lib
        return GpuStamps._lib

    def stamp(self, i):
        import torch

        stream = torch.cuda.current_stream(self.dev).cuda_stream
        if GpuStamps._lib.bz_bench_stamp(ctypes.c_void_p(self.buf.data_ptr() + 8 * i), ctypes.c_void_p(stream)) != 0:
            raise RuntimeError("bz_bench_stamp failed")

    def us(self, i=0, j=1):
        v = self.buf.cpu().tolist()
        return (v[j] - v[i]) * self.us_per_tick


def capture_timed(fn, dev, lead=None):
    """A HIP graph of [lead()] stamp fn() stamp. Returns (graph, stamps)."""
    import torch

    st = GpuStamps(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        if lead is not None:
            lead()
        st.stamp(0)
        fn()
        st.stamp(1)
    graph.replay()  # untimed: the first replay uploads the graph
    torch.cuda.synchronize()
    return graph, st


def time_captured(timed, dev, flush=True):
    """µs between the stamps of a capture_timed() graph in one replay, after a cache flush (cold data) or not."""
    import torch

    graph, st = timed
    torch.cuda.synchronize()
    if flush:
        flush_caches(dev)
    graph.replay()
    torch.cuda.synchronize()
    return st.us()


def time_calls(pkg, w, dev, steps, warmup, combine, splits, eager, cold, fused=False):
    """µs per call for workload w (one q per call) over `steps` calls; cold rotates distinct K/V buffer sets
    (ROTATE_BYTES of valid K/V whatever `steps` is) and flushes the caches before the timed region. fused: each call
    is a fused decode step (bz_gqa_decode_fused) writing slot seq_len - 1 of its set (the same values every time) and
    attending over it. Returns (µs per call, algorithmic bytes per call, sets, rotated bytes)."""
    import torch
    from breeze_tts_2_flash_amd import workloads

    g = w.to(dev)
    lens = w.seq_lens.tolist()
    nb = workloads.fused_algorithmic_bytes if fused else workloads.algorithmic_bytes
    read_bytes = nb(lens, w.num_q_heads, w.num_kv_heads, w.head_dim)
    nsets = max(16, math.ceil(ROTATE_BYTES / read_bytes)) if cold else 1
    lead = 2 if cold else 0  # untimed calls at the head of the graph, on sets of their own
    nsets += lead
    ks = torch.empty((nsets,) + tuple(g.k.shape), dtype=g.k.dtype, device=dev)
    vs = torch.empty_like(ks)
    ks.copy_(g.k.expand_as(ks))
    vs.copy_(g.v.expand_as(vs))
    out = torch.empty(w.batch, w.num_q_heads, w.head_dim, dtype=torch.bfloat16, device=dev)
    kw = dict(combine=combine, num_splits=splits)
    if fused:
        qkv, qn, kn, cos, sin, cache_pos = fused_inputs(w, dev)
        # the fused entry is captured with a workspace made beforehand (a capture allocates nothing)
        ws = pkg.get_workspace(dev, w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.capacity, splits)

        def run(k, v, o=None):
            return pkg.gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, k, v, cache_pos, g.scale, o, seq_lens=g.seq_lens,
                                        workspace=ws, **kw)
    else:
        def run(k, v, o=None):
            return pkg.gqa_decode(g.q, k, v, g.seq_lens, g.scale, o, **kw)

    def call(i):  # timed call i uses set lead + i mod (nsets - lead); lead calls use sets 0 .. lead - 1
        j = lead + i % (nsets - lead) if i >= 0 else lead + i
        run(ks[j], vs[j], out)

    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    if eager:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if cold:
            flush_caches(dev)
        start.record(stream)
        for i in range(steps):
            call(i)
        end.record(stream)
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1000.0 / steps
    else:
        # GPU stamps around exactly the `steps` calls, after `lead` untimed calls on sets the timed calls do not use
        def lead_calls():
            for i in range(-lead, 0):
                call(i)

        def timed_calls():
            for i in range(steps):
                call(i)
        us = time_captured(capture_timed(timed_calls, dev, lead=lead_calls), dev, flush=cold) / steps
    # the rotated sets hold identical data: the last call's output must equal a fresh call on set 0
    ref = run(ks[0], vs[0])
    torch.cuda.synchronize()
    if not torch.equal(out.view(torch.int16), ref.view(torch.int16)):
        raise RuntimeError("benchmark output differs from a direct call")
    del ks, vs
    torch.cuda.empty_cache()  # the next workload's sets need the memory (up to ~40 GB)
    return us, read_bytes, nsets - lead, (nsets - lead) * read_bytes


BACKBONE = dict(H=2048, nq=2048, nk=1024, inter=6144, layers=28, D=128, cap=2048, len=1024)
STREAM_WGS = (256, 512, 1024)
# weight bytes of the backbone's GEMVs (bf16, hidden 2048, 16 q / 8 KV heads of 128, intermediate 6144)
BACKBONE_GEMV_BYTES = {"gemv_qkv_norm_bytes": 2 * 4096 * 2048, "gemv_o_resid_bytes": 2 * 2048 * 2048,
                       "gemv_gateup_norm_silu_bytes": 2 * 2 * 6144 * 2048, "gemv_down_resid_bytes": 2 * 2048 * 6144}


def per_call_times(pkg, w, dev, calls, fused=False):
    """The distribution of single cold calls of workload w (fused: fused decode steps, as time_calls makes them): one
    HIP graph holding a GPU stamp before every call (and one after the last), rotating over ROTATE_BYTES of K/V sets,
    replayed twice after a cache flush; each interval between stamps is one stamp launch plus one call, and the
    median interval of a graph of stamps alone is subtracted. Returns a dict of µs figures (mean, percentiles, a
    0.25 µs histogram)."""
    import numpy as np
    import torch
    from breeze_tts_2_flash_amd import workloads

    g = w.to(dev)
    read_bytes = workloads.algorithmic_bytes(w.seq_lens.tolist(), w.num_q_heads, w.num_kv_heads, w.head_dim)
    nsets = max(16, math.ceil(ROTATE_BYTES / read_bytes)) + 2
    ks = torch.empty((nsets,) + tuple(g.k.shape), dtype=g.k.dtype, device=dev)
    vs = torch.empty_like(ks)
    ks.copy_(g.k.expand_as(ks))
    vs.copy_(g.v.expand_as(vs))
    out = torch.empty(w.batch, w.num_q_heads, w.head_dim, dtype=torch.bfloat16, device=dev)

    if fused:
        qkv, qn, kn, cos, sin, cache_pos = fused_inputs(w, dev)
        ws = pkg.get_workspace(dev, w.batch, w.num_q_heads, w.num_kv_heads, w.head_dim, w.capacity)

    def call(i):  # sets 0 and 1 for the two lead calls, then 2 .. nsets - 1 in turn
        j = 2 + i % (nsets - 2) if i >= 0 else i + 2
        if fused:
            pkg.gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, ks[j], vs[j], cache_pos, g.scale, out,
                                 seq_lens=g.seq_lens, workspace=ws)
        else:
            pkg.gqa_decode(g.q, ks[j], vs[j], g.seq_lens, g.scale, out)

    def intervals(body, flush):
        st = GpuStamps(dev, n=calls + 1)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            body(-2)
            body(-1)
            for i in range(calls):
                st.stamp(i)
                body(i)
            st.stamp(calls)
        graph.replay()
        torch.cuda.synchronize()
        res = []
        for _ in range(2):
            if flush:
                flush_caches(dev)
            graph.replay()
            torch.cuda.synchronize()
            res.append(np.diff(np.array(st.buf.cpu().tolist(), dtype=np.float64)) * st.us_per_tick)
        return np.concatenate(res)

    stamp_us = float(np.median(intervals(lambda i: None, False)))
    d = intervals(call, True) - stamp_us
    del ks, vs
    torch.cuda.empty_cache()
    lo = math.floor(d.min() * 4) / 4
    hist, edges = np.histogram(d, bins=np.arange(lo, d.max() + 0.25, 0.25))
    pct = {f"p{q}": round(float(np.percentile(d, q)), 3) for q in (1, 10, 50, 90, 99)}
    return {"calls": int(d.size), "stamp_launch_us": round(stamp_us, 3), "mean": round(float(d.mean()), 3), **pct,
            "histogram_0.25us": [[round(float(a), 2), int(c)] for a, c in zip(edges, hist) if c]}


def time_stream_floor(dev, sizes):
    """The floor that one launch and the memory system set for reading a given number of bytes: µs per launch of a
    pure streaming read (libbz_bench_stamp.so's bz_bench_stream_read: 256 threads per workgroup, eight 16-byte
    non-temporal loads per thread in flight, nothing done with the bytes) timed exactly as the cold attention calls
    are (EXTRA_CALLS launches in one HIP graph between GPU stamps, 2 untimed lead launches, rotating over ROTATE_BYTES,
    after a flush), on 256, 512 and 1024 workgroups. sizes: {name: bytes per launch}. Returns
    {name: ({workgroups: µs per launch}, bytes read per launch)}."""
    import torch

    lib = GpuStamps.library()
    buf = torch.empty(int(ROTATE_BYTES), dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    out = {}
    for name, call_bytes in sizes.items():
        res = {}
        nbytes = call_bytes
        for wgs in STREAM_WGS:
            per_wg = call_bytes // wgs // 16 * 16
            nbytes = per_wg * wgs
            regions = buf.numel() // nbytes
            assert regions > EXTRA_CALLS // 4

            def launch(i):
                ptr = buf.data_ptr() + (i % regions) * nbytes
                stream = torch.cuda.current_stream(dev).cuda_stream
                if lib.bz_bench_stream_read(ctypes.c_void_p(ptr), per_wg, wgs, ctypes.c_void_p(sink.data_ptr()),
                                            ctypes.c_void_p(stream)) != 0:
                    raise RuntimeError("bz_bench_stream_read failed")

            def lead():
                for i in (regions - 2, regions - 1):
                    launch(i)

            def timed():
                for i in range(EXTRA_CALLS):
                    launch(i)
            res[wgs] = time_captured(capture_timed(timed, dev, lead=lead), dev) / EXTRA_CALLS
        out[name] = (res, nbytes)
    del buf
    torch.cuda.empty_cache()
    return out


class KvPatternArgs(ctypes.Structure):
    """bz_bench_kv_args of libbz_bench_stamp.so."""
    _fields_ = [("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p), ("kv_stride_b", ctypes.c_int64),
                ("kv_stride_h", ctypes.c_int64), ("kv_stride_s", ctypes.c_int64), ("seq_lens", ctypes.c_void_p),
                ("rows", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("capacity", ctypes.c_int32), ("splits", ctypes.c_int32), ("exchange", ctypes.c_int32),
                ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t), ("out", ctypes.c_void_p),
                ("sink", ctypes.c_void_p)]


def _pattern_chunks(length, splits, D=128):
    """The split kernel's chunk count for a row of `length` positions (min chunk 16 KB of K+V, one split up to
    64 KB), which is what bz_bench_kv_pattern writes for the row when it exchanges."""
    min_chunk, one = 16 * 1024 // (4 * D), 64 * 1024 // (4 * D)
    if length <= 0:
        return 1
    chunk = max(length, min_chunk) if length <= one else max(-(-length // splits), min_chunk)
    return -(-length // chunk)


def time_protocol_floor(pkg, dev, configs=(2, 3, 4)):
    """The floor the split kernel's own traffic and exchange set, per config: µs per launch of bz_bench_kv_pattern
    (the kernel's grid, chunk rule and K/V loads with no arithmetic), without and with the kernel's exchange protocol,
    timed exactly as the cold calls (EXTRA_CALLS launches in one HIP graph between GPU stamps, 2 untimed lead launches,
    rotating over ROTATE_BYTES of K/V sets, after a flush). Each output is checked against the rows' chunk counts
    (every (row, kv head) merged once). Returns {configN: {"splits", "pattern_us", "pattern_exchange_us"}}."""
    import torch
    from breeze_tts_2_flash_amd import workloads

    lib = GpuStamps.library()
    lib.bz_bench_kv_pattern.argtypes = [ctypes.POINTER(KvPatternArgs), ctypes.c_void_p]
    lib.bz_bench_kv_pattern_workspace.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                  ctypes.POINTER(ctypes.c_size_t)]
    res = {}
    for xc in configs:
        w = workloads.make(xc)
        B, NKV, D, cap = w.batch, w.num_kv_heads, w.head_dim, w.capacity
        splits = pkg.default_splits(B, NKV, D, cap, 0)
        lens = w.seq_lens.tolist()
        read_bytes = workloads.algorithmic_bytes(lens, w.num_q_heads, NKV, D)
        nsets = max(16, math.ceil(ROTATE_BYTES / read_bytes)) + 2
        ks = torch.empty((nsets,) + tuple(w.k.shape), dtype=torch.bfloat16, device=dev)
        vs = torch.empty_like(ks)
        ks.copy_(w.k.to(dev).expand_as(ks))
        vs.copy_(w.v.to(dev).expand_as(vs))
        seq = w.seq_lens.to(dev)
        nbytes = ctypes.c_size_t(0)
        if lib.bz_bench_kv_pattern_workspace(B, NKV, splits, ctypes.byref(nbytes)) != 0:
            raise RuntimeError("bz_bench_kv_pattern_workspace failed")
        ws = torch.zeros(nbytes.value, dtype=torch.uint8, device=dev)
        out = torch.zeros(B * NKV * 256, dtype=torch.int16, device=dev)
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        entry = {"splits": splits}
        for exchange in (0, 1):
            a = KvPatternArgs(None, None, ks.stride(1), ks.stride(2), ks.stride(3), seq.data_ptr(), B, NKV, D, cap,
                              splits, exchange, ws.data_ptr(), nbytes.value, out.data_ptr(), sink.data_ptr())

            def launch(j):
                a.k_cache, a.v_cache = ks[j].data_ptr(), vs[j].data_ptr()
                if lib.bz_bench_kv_pattern(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)):
                    raise RuntimeError("bz_bench_kv_pattern failed")

            def lead():
                launch(0)
                launch(1)

            def timed():
                for i in range(EXTRA_CALLS):
                    launch(2 + i % (nsets - 2))
            us = time_captured(capture_timed(timed, dev, lead=lead), dev) / EXTRA_CALLS
            want = torch.tensor([_pattern_chunks(n, splits, D) if exchange else 1 for n in lens for _ in range(NKV)],
                                dtype=torch.float32).repeat_interleave(256).bfloat16().view(torch.int16)
            if not torch.equal(out.cpu(), want):
                raise RuntimeError(f"bz_bench_kv_pattern (config {xc}, exchange {exchange}): wrong chunk counts")
            entry["pattern_exchange_us" if exchange else "pattern_us"] = round(us, 3)
        res[f"config{xc}"] = entry
        del ks, vs
        torch.cuda.empty_cache()
    return res


def make_backbone(dev, M=2):
    """Random-init weights, KV caches and buffers of the reference's backbone at its serving shape (a Qwen3 of hidden
    2048, 16 q / 8 KV heads of 128, intermediate 6144, 28 layers; KV 1024 of 2048 slots) for M rows: 2 is the CFG
    pair, 1 and 4 the other batch sizes the reference's fused step takes (flash/backbone.py:18-22, :58)."""
    import torch

    c = BACKBONE
    H, nq, nk, I, L, D = c["H"], c["nq"], c["nk"], c["inter"], c["layers"], c["D"]
    gen = torch.Generator(device=dev).manual_seed(123)
    bf = torch.bfloat16

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * scale).to(bf)

    layers = []
    for _ in range(L):
        layers.append(dict(ln1=1 + rnd(H, scale=0.1), ln2=1 + rnd(H, scale=0.1), qn=1 + rnd(D, scale=0.1),
                           kn=1 + rnd(D, scale=0.1), wq=rnd(nq, H, scale=H ** -0.5), wk=rnd(nk, H, scale=H ** -0.5),
                           wv=rnd(nk, H, scale=H ** -0.5), wo=rnd(H, nq, scale=nq ** -0.5),
                           wg=rnd(I, H, scale=H ** -0.5), wu=rnd(I, H, scale=H ** -0.5),
                           wd=rnd(H, I, scale=I ** -0.5),
                           kc=rnd(M, nk // D, c["cap"], D), vc=rnd(M, nk // D, c["cap"], D)))
    norm_w = 1 + rnd(H, scale=0.1)
    x0 = rnd(M, H)
    qkv = torch.empty(M, nq + 2 * nk, dtype=bf, device=dev)
    ao = torch.empty(M, nq // D, D, dtype=bf, device=dev)
    h1 = torch.empty(M, H, dtype=bf, device=dev)
    act = torch.empty(M, I, dtype=bf, device=dev)
    xb = [torch.empty(M, H, dtype=bf, device=dev) for _ in range(2)]
    hidden = torch.empty(M, H, dtype=bf, device=dev)
    pos = c["len"] - 1
    inv = 1e6 ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = torch.cat([pos * inv] * 2)
    cos = ang.cos().to(bf).expand(M, D).contiguous().to(dev)
    sin = ang.sin().to(bf).expand(M, D).contiguous().to(dev)
    cache_pos = torch.tensor([pos], dtype=torch.int64, device=dev)
    lens = torch.full((M,), c["len"], dtype=torch.int32, device=dev)
    return dict(M=M, layers=layers, norm_w=norm_w, x0=x0, qkv=qkv, ao=ao, h1=h1, act=act, xb=xb, hidden=hidden,
                cos=cos, sin=sin, cache_pos=cache_pos, lens=lens)


def time_backbone(pkg, dev, reps=BACKBONE_REPS, model=None, M=2):
    """The backbone decode step of make_backbone(dev, M) (or `model`, made earlier by it): per layer gemv_seg (RMSNorm
    + q|k|v) -> gqa_decode_fused -> gemv_resid (o_proj) -> gemv_gateup -> gemv_resid (down), then the final rmsnorm
    (flash/backbone.py:120-129), one HIP graph per step. Also each GEMV alone, rotating over the 28 layers' weights.
    Returns {name: {us, bytes, GB/s}}."""
    import torch

    c = BACKBONE
    H, nq, nk, I, L, D = c["H"], c["nq"], c["nk"], c["inter"], c["layers"], c["D"]
    m = model if model is not None else make_backbone(dev, M)
    M = m["M"]
    layers, norm_w, x0, qkv, ao, h1, act, xb, hidden = (m[k] for k in ("layers", "norm_w", "x0", "qkv", "ao", "h1",
                                                                         "act", "xb", "hidden"))
    cos, sin, cache_pos, lens = m["cos"], m["sin"], m["cache_pos"], m["lens"]
    eps, scale = 1e-6, D ** -0.5
    ws = pkg.get_workspace(dev, M, nq // D, nk // D, D, c["cap"])  # made before the step is captured

    def step():
        x = x0
        for i, ly in enumerate(layers):
            pkg.gemv_seg(x, ly["ln1"], eps, ly["wq"], ly["wk"], ly["wv"], qkv)
            pkg.gqa_decode_fused(qkv, ly["qn"], ly["kn"], eps, cos, sin, ly["kc"], ly["vc"], cache_pos, scale, ao,
                                 seq_lens=lens, workspace=ws)
            pkg.gemv_resid(ao.view(M, nq), ly["wo"], x, h1)
            pkg.gemv_gateup(h1, ly["ln2"], eps, ly["wg"], ly["wu"], act)
            pkg.gemv_resid(act, ly["wd"], h1, xb[i % 2])
            x = xb[i % 2]
        pkg.rmsnorm(x, norm_w, eps, hidden)

    def graph_time(fn, reps, flush=True):
        """Median µs of `reps` replays of fn captured in one graph, each replay timed alone (after a cache flush)."""
        fn()
        torch.cuda.synchronize()
        timed = capture_timed(fn, dev)
        return statistics.median(time_captured(timed, dev, flush=flush) for _ in range(reps))

    out = {}
    layer_bytes = 2 * ((nq + 2 * nk) * H + H * nq + 2 * I * H + H * I) + 2 * 2 * (nk // D) * c["len"] * D * M

    def entry(us):
        return {"us": round(us, 1), "bytes": L * layer_bytes, "GB/s": round(L * layer_bytes / us / 1e3, 1),
                "pct_of_peak_hbm": round(100.0 * L * layer_bytes / us / 1e3 / PEAK_HBM_GBS, 1)}
    out["backbone_step_28_layers"] = entry(graph_time(step, reps))
    # steps back to back and no flush, as a serving loop runs them: the caches hold what the previous steps left
    chain = BACKBONE_CHAIN

    def steps():
        for _ in range(chain):
            step()
    out["backbone_step_28_layers_back_to_back"] = entry(graph_time(steps, max(3, reps // 10), flush=False) / chain)
    # each GEMV alone, over the 28 layers' weights in turn (28 launches per replay)
    cases = {
        "gemv_qkv_norm": (lambda ly: pkg.gemv_seg(x0, ly["ln1"], eps, ly["wq"], ly["wk"], ly["wv"], qkv),
                          2 * (nq + 2 * nk) * H),
        "gemv_o_resid": (lambda ly: pkg.gemv_resid(ao.view(M, nq), ly["wo"], x0, h1), 2 * H * nq),
        "gemv_gateup_norm_silu": (lambda ly: pkg.gemv_gateup(h1, ly["ln2"], eps, ly["wg"], ly["wu"], act),
                                  2 * 2 * I * H),
        "gemv_down_resid": (lambda ly: pkg.gemv_resid(act, ly["wd"], h1, hidden), 2 * H * I),
    }
    for name, (fn, wbytes) in cases.items():
        us = graph_time(lambda: [fn(ly) for ly in layers], reps) / L
        out[name] = {"us": round(us, 3), "weight_bytes": wbytes, "GB/s": round(wbytes / us / 1e3, 1),
                     "pct_of_peak_hbm": round(100.0 * wbytes / us / 1e3 / PEAK_HBM_GBS, 1)}
    return out


def _time_frames(frame, nsteps, dev, frames=EXTRA_FRAMES, warmup=2):
    """µs per frame of `frame` (nsteps launches), `frames` frames recorded back to back in one HIP graph. The depth
    transformer's K/V is written moments before it is read, so it is timed warm (no flush)."""
    import torch

    for _ in range(warmup):
        frame()
    torch.cuda.synchronize()

    def all_frames():
        for _ in range(frames):
            frame()
    return time_captured(capture_timed(all_frames, dev), dev, flush=False) / frames


def time_depth_frame(pkg, dev, wave=False):
    """Config 5: µs per 32-step depth frame (one launch per step, seq_lens 1..32), recorded in one HIP graph; with
    wave=True through bz_gqa_decode_wave (one wave per (row, q head), no split) instead of the split kernel."""
    import torch
    from breeze_tts_2_flash_amd import workloads

    w = workloads.make(5)
    g = w.to(dev)
    nsteps = g.q.shape[0]
    out = torch.empty(w.batch, w.num_q_heads, w.head_dim, dtype=torch.bfloat16, device=dev)

    def frame():
        for s in range(nsteps):
            if wave:
                pkg.gqa_decode_wave(g.q[s], g.k, g.v, g.seq_lens[s], g.scale, out=out)
            else:
                pkg.gqa_decode(g.q[s], g.k, g.v, g.seq_lens[s], g.scale, out=out, max_seq_len=nsteps)

    us_frame = _time_frames(frame, nsteps, dev)
    frame_bytes = sum(workloads.algorithmic_bytes([L, L], w.num_q_heads, w.num_kv_heads, w.head_dim)
                      for L in range(1, nsteps + 1))
    return us_frame, frame_bytes


def time_real_depth_frame(pkg, dev):
    """The reference's depth-transformer attention shape (flash/depth.py:71, :130-131): B2 (the CFG pair), 8 q / 2 KV
    heads of 128, a 17-slot cache, 16 steps attending over 2..17 positions (seed 6, N(0,1)), one launch per step in
    one HIP graph. gqa_decode as called (it takes the wave kernel at this shape) and with the split kernel forced
    (num_splits=1). Returns (µs per frame routed, µs per frame split kernel, algorithmic bytes per frame)."""
    import torch
    from breeze_tts_2_flash_amd import workloads

    B, NH, NKV, D, cap, nsteps = 2, 8, 2, 128, 17, 16
    gen = torch.Generator().manual_seed(6)
    q = torch.randn(nsteps, B, NH, D, generator=gen).bfloat16().to(dev)
    k = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(dev)
    v = torch.randn(B, NKV, cap, D, generator=gen).bfloat16().to(dev)
    lens = [torch.full((B,), s + 2, dtype=torch.int32, device=dev) for s in range(nsteps)]
    out = torch.empty(B, NH, D, dtype=torch.bfloat16, device=dev)
    res = []
    for splits in (0, 1):
        def frame():
            for s in range(nsteps):
                pkg.gqa_decode(q[s], k, v, lens[s], D ** -0.5, out=out, num_splits=splits)
        res.append(_time_frames(frame, nsteps, dev))
    frame_bytes = sum(workloads.algorithmic_bytes([L, L], NH, NKV, D) for L in range(2, nsteps + 2))
    return res[0], res[1], frame_bytes


HOST_CALLS = 500            # calls per host-overhead sample (5 samples, median)


def host_overhead(pkg, dev):
    """Eager host cost per call of the Python entry points on config 1's inputs (B2, 256 positions: every kernel
    takes a few microseconds of GPU time, so the host is the bound): HOST_CALLS back-to-back calls without a
    synchronisation, wall time / calls, median of 5 samples after 50 warmups. 'direct' is the package function (the
    eager path: the native binding's checks and the C ABI call; the GEMVs through ctypes); 'torch_op' the registered
    operator torch.ops.bz.* called eagerly (what a compiled graph calls, plus the dispatcher)."""
    import torch
    from breeze_tts_2_flash_amd import gemv_resid, gqa_decode, gqa_decode_fused, workloads

    w = workloads.make(1).to(dev)
    out = torch.empty(w.batch, w.num_q_heads, w.head_dim, dtype=torch.bfloat16, device=dev)
    qkv, qn, kn, cos, sin, pos = fused_inputs(workloads.make(1), dev)
    kc, vc = w.k.clone(), w.v.clone()
    x = torch.randn(2, 1024, device=dev).bfloat16()
    W = (torch.randn(1024, 1024, device=dev) * 0.03).bfloat16()
    res = torch.randn(2, 1024, device=dev).bfloat16()
    y = torch.empty_like(res)
    cases = {
        "gqa_decode_direct": lambda: gqa_decode(w.q, w.k, w.v, w.seq_lens, w.scale, out),
        "gqa_decode_torch_op": lambda: torch.ops.bz.gqa_decode(w.q, w.k, w.v, w.seq_lens, float(w.scale), out, None,
                                                               None, 0, 0, 0, None),
        "gqa_decode_fused_direct": lambda: gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc, vc, pos, w.scale, out,
                                                            seq_lens=w.seq_lens),
        "gemv_resid_direct": lambda: gemv_resid(x, W, res, y),
        "gemv_resid_torch_op": lambda: torch.ops.bz.gemv_resid(x, W, res, y),
    }
    got = {}
    for name, fn in cases.items():
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        samples = []
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(HOST_CALLS):
                fn()
            samples.append((time.perf_counter() - t0) * 1e6 / HOST_CALLS)
            torch.cuda.synchronize()
        got[name] = round(statistics.median(samples), 2)
    return got


def cpu_baseline(w, calls=200, warmup=20, kind="eager", budget_s=10.0):
    """Median µs per call on the host of the reference's CPU attention for workload w. kind "eager": the eager chain
    (repeat_kv + bf16 matmul + fp32 softmax + matmul, oracle/attention.py:eager_bf16) over the StaticCache capacity with
    the interval mask, as the reference runs decode; kind "sdpa": torch's fp32 scaled_dot_product_attention per row
    over the valid range (oracle/attention.py:sdpa_fp32, the north-star oracle). At most `calls` calls or
    `budget_s` seconds after `warmup`."""
    import torch
    from oracle.attention import eager_bf16, interval_mask, sdpa_fp32

    threads = int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    if kind == "eager":
        q = w.q[:, :, None, :]
        # 0 on each row's [0, seq_len), finfo.min elsewhere: interval_mask's values with a per-row end (the ragged
        # batch's rows differ in length; for equal lengths this is interval_mask([0] * B, seq_len - 1, capacity))
        mask = interval_mask([0] * w.batch, w.capacity - 1, w.capacity)
        pos = torch.arange(w.capacity)
        mask[:, 0, 0, :].masked_fill_(pos[None, :] >= w.seq_lens.long()[:, None], torch.finfo(mask.dtype).min)

        def run():
            eager_bf16(q, w.k, w.v, mask, w.scale)
    else:
        def run():
            sdpa_fp32(w.q, w.k, w.v, w.seq_lens.tolist(), w.scale)
    for _ in range(warmup):
        run()
    ts = []
    t_end = time.perf_counter() + budget_s
    for _ in range(calls):
        t0 = time.perf_counter_ns()
        run()
        ts.append(time.perf_counter_ns() - t0)
        if time.perf_counter() > t_end:
            break
    return statistics.median(ts) / 1000.0, torch.get_num_threads(), len(ts)


WORKLOADS = {
    1: "config 1: reference CPU step, B2, 16q/8kv, D128, K/V 256, seq_lens 256",
    2: "config 2: backbone decode, B2, 16q/8kv, D128, capacity 2048, seq_lens 1024",
    3: "config 3: long split-K, B2, 16q/8kv, D128, capacity 4096, seq_lens 4096, 1% of K x8",
    4: "config 4: ragged server batch, B16 (8 CFG pairs), 16q/8kv, D128, capacity 2048, lengths U[128, 2048]",
}

TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "gqa_split_kernel_config2_traffic.txt")


def traffic_from_profile():
    """HBM bytes per call recorded by the rocprofv3 counter runs summarised in profiles/ (None if absent)."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_call:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def copy_calibration(nbytes, steps):
    """Plain device-to-device copies of nbytes: each dispatch reads and writes exactly nbytes, the reference for
    scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": steps}), flush=True)


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); the "
              "decode-attention path is measured at N=1", file=sys.stderr)
        sys.exit(2)
    import torch

    pkg = _pkg()
    from breeze_tts_2_flash_amd import workloads

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration, args.steps)
        return
    pkg.load()

    if args.backbone_only:
        bb = {f"m{M}": time_backbone(pkg, dev, M=M) for M in args.backbone_m}
        print(json.dumps({"backbone": bb}), flush=True)
        return
    if args.protocol_only:
        floor = time_protocol_floor(pkg, dev)
        for xc in (2, 3, 4):
            floor[f"config{xc}"]["kernel_us"] = round(
                time_calls(pkg, workloads.make(xc), dev, EXTRA_CALLS, args.warmup, "auto", 0, False, cold=True)[0], 3)
        print(json.dumps({"protocol_floor": floor}), flush=True)
        return
    if args.depth_only:
        us_f, _ = time_depth_frame(pkg, dev)
        us_w, _ = time_depth_frame(pkg, dev, wave=True)
        us_r, us_rs, _ = time_real_depth_frame(pkg, dev)
        print(json.dumps({"config5_frame_us": round(us_f, 3), "config5_frame_wave_us": round(us_w, 3),
                          "real_depth_frame_us": round(us_r, 3), "real_depth_frame_split_us": round(us_rs, 3)}),
              flush=True)
        return
    cfg = args.config
    if args.per_call:
        print(json.dumps({"per_call_us": per_call_times(pkg, workloads.make(cfg), dev, args.per_call, args.fused),
                          "config": cfg, "fused": args.fused}), flush=True)
        return
    w2 = workloads.make(cfg)
    splits2 = args.splits or pkg.default_splits(w2.batch, w2.num_kv_heads, w2.head_dim, w2.capacity, 0)
    print(f"[bench] config {cfg} cold, {args.steps} calls, splits={splits2}, combine={args.combine}", file=sys.stderr,
          flush=True)
    us, nbytes, nsets, rotated = time_calls(pkg, w2, dev, args.steps, args.warmup, args.combine, args.splits,
                                            args.eager, cold=True, fused=args.fused)
    gbs = nbytes / us / 1e3
    print(f"[bench] config {cfg} cold: {us:.3f} us/call, {gbs:.1f} GB/s", file=sys.stderr, flush=True)
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(us / 1000.0, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": WORKLOADS[cfg] + (" (fused step: q/k RMSNorm + RoPE + cache write + attention)"
                                                 if args.fused else ""),
                   "us_per_call": round(us, 3), "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 1),
                   "storage": "bf16", "splits": splits2, "combine": args.combine,
                   "timing": "eager launches" if args.eager else "HIP graph replay, GPU wall-clock stamps around the timed calls",
                   "cache": {"mode": "cold", "sets": nsets, "rotated_bytes": rotated, "flush_bytes": FLUSH_BYTES},
                   "algorithmic_bytes_per_call": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": args.traffic_bytes if args.traffic_bytes is not None else
                     (traffic_from_profile() if cfg == 2 and not args.fused else None)},
    }
    extra = {}
    if not args.no_extra:
        us_w, _, _, _ = time_calls(pkg, w2, dev, EXTRA_CALLS, args.warmup, args.combine, args.splits, args.eager,
                                   cold=False, fused=args.fused)
        extra[f"config{cfg}_warm"] = {"us_per_call": round(us_w, 3), "GB/s": round(nbytes / us_w / 1e3, 1),
                                      "calls": EXTRA_CALLS}
        print(f"[bench] config {cfg} warm: {us_w:.3f} us/call", file=sys.stderr, flush=True)
        for xc in (2, 3, 4):
            if xc == cfg:
                continue
            w = workloads.make(xc)
            us_c, nb, ns, rot = time_calls(pkg, w, dev, EXTRA_CALLS, args.warmup, args.combine, args.splits,
                                           args.eager, cold=True)
            extra[f"config{xc}_cold"] = {
                "workload": workloads.NAMES[xc], "us_per_call": round(us_c, 3), "GB/s": round(nb / us_c / 1e3, 1),
                "pct_of_peak_hbm": round(100.0 * nb / us_c / 1e3 / PEAK_HBM_GBS, 1), "bytes": nb, "sets": ns,
                "rotated_bytes": rot, "calls": EXTRA_CALLS}
            print(f"[bench] config {xc} cold: {us_c:.3f} us/call, {nb / us_c / 1e3:.1f} GB/s", file=sys.stderr,
                  flush=True)
            del w
        if not args.fused and w2.head_dim == 128 and len(set(w2.seq_lens.tolist())) == 1:
            us_x, nbx, nsx, rotx = time_calls(pkg, w2, dev, EXTRA_CALLS, args.warmup, args.combine, args.splits,
                                              args.eager, cold=True, fused=True)
            extra[f"config{cfg}_fused_cold"] = {
                "entry": "bz_gqa_decode_fused (q/k RMSNorm + RoPE + cache-slot write + attention)",
                "us_per_call": round(us_x, 3), "GB/s": round(nbx / us_x / 1e3, 1),
                "pct_of_peak_hbm": round(100.0 * nbx / us_x / 1e3 / PEAK_HBM_GBS, 1), "bytes": nbx, "sets": nsx,
                "rotated_bytes": rotx, "calls": EXTRA_CALLS}
            print(f"[bench] config {cfg} fused cold: {us_x:.3f} us/call", file=sys.stderr, flush=True)
        sizes = {f"config{xc}_bytes": workloads.algorithmic_bytes(workloads.make(xc).seq_lens.tolist(), 16, 8, 128)
                 for xc in (2, 3, 4)}
        sizes.update(BACKBONE_GEMV_BYTES)
        floor = {}
        for name, (fl, nbf) in time_stream_floor(dev, sizes).items():
            best = min(fl.values())
            floor[name] = {
                "bytes": nbf, "us_per_launch": {str(k): round(v, 3) for k, v in fl.items()},
                "best_us": round(best, 3), "best_GB/s": round(nbf / best / 1e3, 1),
                "best_pct_of_peak_hbm": round(100.0 * nbf / best / 1e3 / PEAK_HBM_GBS, 1)}
            print(f"[bench] stream floor, {name}: {fl}", file=sys.stderr, flush=True)
        floor["method"] = ("a pure streaming read of the same bytes (no arithmetic, no exchange): the configs' "
                           "algorithmic bytes and the backbone GEMVs' weight bytes, timed like the cold calls; "
                           "keyed by workgroup count")
        extra["stream_floor"] = floor
        proto = time_protocol_floor(pkg, dev)
        for xc in (2, 3, 4):
            kus = us if xc == cfg and not args.fused else extra.get(f"config{xc}_cold", {}).get("us_per_call")
            if kus is not None:
                proto[f"config{xc}"]["kernel_us"] = round(kus, 3)
            print(f"[bench] protocol floor, config {xc}: {proto[f'config{xc}']}", file=sys.stderr, flush=True)
        proto["method"] = ("bz_bench_kv_pattern: the split kernel's grid, chunk rule and K/V loads with no arithmetic "
                           "(pattern_us), then also its exchange protocol on a 1 KB partial per workgroup "
                           "(pattern_exchange_us), timed like the cold calls; kernel_us is the kernel's own cold time "
                           "in this run")
        extra["protocol_floor"] = proto
        us_f, fb = time_depth_frame(pkg, dev)
        extra["config5_depth_frame"] = {"us_per_frame": round(us_f, 3), "us_per_call": round(us_f / 32, 3),
                                        "bytes_per_frame": fb, "GB/s": round(fb / us_f / 1e3, 1),
                                        "frames": EXTRA_FRAMES}
        print(f"[bench] config 5 depth frame: {us_f:.3f} us/frame", file=sys.stderr, flush=True)
        us_w, _ = time_depth_frame(pkg, dev, wave=True)
        extra["config5_depth_frame_wave"] = {"us_per_frame": round(us_w, 3), "us_per_call": round(us_w / 32, 3),
                                             "bytes_per_frame": fb, "GB/s": round(fb / us_w / 1e3, 1),
                                             "frames": EXTRA_FRAMES}
        print(f"[bench] config 5 depth frame, one wave per (row, q head): {us_w:.3f} us/frame", file=sys.stderr,
              flush=True)
        us_r, us_rs, rb = time_real_depth_frame(pkg, dev)
        extra["depth_real_frame"] = {"shape": "B2 8q/2kv D128, 16 steps over 2..17 positions",
                                     "us_per_frame": round(us_r, 3), "us_per_call": round(us_r / 16, 3),
                                     "split_kernel_us_per_frame": round(us_rs, 3), "bytes_per_frame": rb,
                                     "frames": EXTRA_FRAMES}
        print(f"[bench] real depth shape frame: {us_r:.3f} us/frame ({us_rs:.3f} with the split kernel)",
              file=sys.stderr, flush=True)
        bb = time_backbone(pkg, dev)
        bb["timing"] = (f"median of {BACKBONE_REPS} graph replays, each after a {FLUSH_BYTES >> 20} MiB cache flush; "
                        f"back_to_back: {BACKBONE_CHAIN} steps per replay, no flush, median of {max(3, BACKBONE_REPS // 10)}")
        extra["backbone"] = bb
        for k, v in bb.items():
            print(f"[bench] {k}: {v}", file=sys.stderr, flush=True)
        # the reference's other served batch sizes (its fused step takes M in {1, 2, 4}, flash/backbone.py:18-22, :58)
        for M in (1, 4):
            bbm = time_backbone(pkg, dev, reps=BACKBONE_REPS_OTHER_M, M=M)
            bbm["timing"] = (f"as backbone, M = {M}: median of {BACKBONE_REPS_OTHER_M} flushed replays; back_to_back "
                             f"median of {max(3, BACKBONE_REPS_OTHER_M // 10)}")
            extra[f"backbone_m{M}"] = bbm
            print(f"[bench] backbone M={M}: step {bbm['backbone_step_28_layers']['us']} us", file=sys.stderr,
                  flush=True)
        ho = host_overhead(pkg, dev)
        ho["method"] = (f"eager host µs per call: {HOST_CALLS} back-to-back calls without a synchronisation, config 1 "
                        f"inputs (GEMV 2x1024x1024), median of 5 samples")
        extra["host_overhead"] = ho
        print(f"[bench] host overhead: {ho}", file=sys.stderr, flush=True)
        line["extra"] = extra
    if not args.no_cpu:
        us_cpu, cores, n = cpu_baseline(w2, calls=100000, budget_s=10.0)
        line["cpu_baseline"] = {"value": round(nbytes / us_cpu / 1e3, 3), "unit": "GB/s", "cores": cores,
                                "kind": "port", "us_per_call": round(us_cpu, 1),
                                "sample": f"config {cfg} inputs, the reference's eager bf16 chain over the full "
                                          f"{w2.capacity}-slot cache with the interval mask, median of {n} calls "
                                          f"(10 s of CPU time) after 20 warmups"}
        print(f"[bench] cpu baseline: {us_cpu:.1f} us/call on {cores} threads", file=sys.stderr, flush=True)
        # beside it: the reference's own CPU-runnable case (config 1), the eager chain on configs 3 and 4, and the
        # fp32 SDPA oracle on the headline inputs
        cx = {}
        us_c1, _, n1 = cpu_baseline(workloads.make(1), kind="eager", calls=100000, budget_s=3.0)
        cx["config1_eager_us_per_call"], cx["config1_calls"] = round(us_c1, 1), n1
        for xc in (2, 3, 4):
            if xc == cfg:
                continue
            wx = workloads.make(xc)
            us_x, _, nx = cpu_baseline(wx, kind="eager", calls=100000, warmup=5, budget_s=3.0)
            bx = workloads.algorithmic_bytes(wx.seq_lens.tolist(), wx.num_q_heads, wx.num_kv_heads, wx.head_dim)
            cx[f"config{xc}_eager_us_per_call"], cx[f"config{xc}_calls"] = round(us_x, 1), nx
            cx[f"config{xc}_eager_GB/s"] = round(bx / us_x / 1e3, 3)
            print(f"[bench] cpu config {xc} eager: {us_x:.1f} us/call", file=sys.stderr, flush=True)
            del wx
        us_sd, _, nsd = cpu_baseline(w2, kind="sdpa", calls=100000, warmup=5, budget_s=3.0)
        cx[f"config{cfg}_sdpa_fp32_us_per_call"], cx[f"config{cfg}_sdpa_calls"] = round(us_sd, 1), nsd
        cx["budget"] = "3 s of CPU time per extra case (median call after 5-20 warmups)"
        line["cpu_baseline"]["extra"] = cx
        print(f"[bench] cpu config 1 eager: {us_c1:.1f} us/call; config {cfg} sdpa fp32: {us_sd:.1f} us/call",
              file=sys.stderr, flush=True)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
