"""The five decode-attention workloads the benchmark and the parity tests run, with seeded inputs.

Shapes follow the reference's serving setup: backbone 16 q / 8 KV heads, head_dim 128, StaticCache capacity 2048
(third_party/breeze-tts/models/cudagraph/backbone_graph.py:73-75, breeze_infer/api.py:48); CFG pair = batch 2.
Inputs are drawn on the CPU with torch.Generator().manual_seed(seed) in the order q, K, V, then extras; values are
N(0, 1) in fp32 rounded to bf16; scale = head_dim ** -0.5 (the layers' scaling, models/breeze.py:302).

  1  the reference's CPU-runnable step: B2, 16/8, D128, K/V [2, 8, 256, 128], seq_lens 256
  2  backbone serving: B2, 16/8, D128, capacity 2048, seq_lens 1024
  3  long split-K stress: B2, 16/8, D128, capacity 4096, seq_lens 4096, K x8 at a Bernoulli(0.01) set of
     (row, position) before the bf16 cast
  4  ragged server batch: B16 = 8 CFG pairs, capacity 2048, lengths U[128, 2048] shared by each pair, K/V NaN at
     positions >= length
  5  depth frame: B2, 16/8, D64, capacity 32, 32 steps with seq_lens = 1..32 (one q per step)
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class Workload:
    cfg: int
    batch: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    capacity: int
    q: torch.Tensor          # [B, NH, D] bf16, or [steps, B, NH, D] for the depth frame
    k: torch.Tensor          # [B, NKV, capacity, D] bf16
    v: torch.Tensor
    seq_lens: torch.Tensor   # [B] int32, or [steps, B] for the depth frame
    scale: float
    extras: dict = field(default_factory=dict)

    def to(self, device) -> "Workload":
        return Workload(self.cfg, self.batch, self.num_q_heads, self.num_kv_heads, self.head_dim, self.capacity,
                        self.q.to(device), self.k.to(device), self.v.to(device), self.seq_lens.to(device),
                        self.scale, dict(self.extras))


NAMES = {1: "cpu_ref_kv256", 2: "backbone_kv1024_cap2048", 3: "long_kv4096_splitk", 4: "ragged_b16_nan_tails",
         5: "depth_frame_d64_kv1to32"}


def _randn(g: torch.Generator, *shape) -> torch.Tensor:
    return torch.randn(*shape, generator=g, dtype=torch.float32)


def make(cfg: int, scale_factor: int = 1) -> Workload:
    """Seeded inputs of config cfg on the CPU. scale_factor divides the KV capacity/lengths of configs 2-4 (for
    small CPU-checkable variants); 1 gives the BASELINE shapes."""
    g = torch.Generator().manual_seed(cfg)
    NH, NKV = 16, 8
    if cfg == 1:
        B, D, cap = 2, 128, 256
        q = _randn(g, B, NH, D).bfloat16()
        k = _randn(g, B, NKV, cap, D).bfloat16()
        v = _randn(g, B, NKV, cap, D).bfloat16()
        lens = torch.full((B,), cap, dtype=torch.int32)
        return Workload(cfg, B, NH, NKV, D, cap, q, k, v, lens, D ** -0.5)
    if cfg == 2:
        B, D, cap, L = 2, 128, 2048 // scale_factor, 1024 // scale_factor
        q = _randn(g, B, NH, D).bfloat16()
        k = _randn(g, B, NKV, cap, D).bfloat16()
        v = _randn(g, B, NKV, cap, D).bfloat16()
        lens = torch.full((B,), L, dtype=torch.int32)
        return Workload(cfg, B, NH, NKV, D, cap, q, k, v, lens, D ** -0.5)
    if cfg == 3:
        B, D, cap = 2, 128, 4096 // scale_factor
        q = _randn(g, B, NH, D).bfloat16()
        k = _randn(g, B, NKV, cap, D)
        v = _randn(g, B, NKV, cap, D).bfloat16()
        hot = torch.rand(B, cap, generator=g) < 0.01          # (row, position) pairs whose K is scaled x8
        k = torch.where(hot[:, None, :, None], k * 8.0, k).bfloat16()
        lens = torch.full((B,), cap, dtype=torch.int32)
        return Workload(cfg, B, NH, NKV, D, cap, q, k, v, lens, D ** -0.5, {"hot": hot})
    if cfg == 4:
        B, D, cap = 16, 128, 2048 // scale_factor
        q = _randn(g, B, NH, D).bfloat16()
        k = _randn(g, B, NKV, cap, D).bfloat16()
        v = _randn(g, B, NKV, cap, D).bfloat16()
        pair_lens = torch.randint(128 // scale_factor, cap + 1, (B // 2,), generator=g, dtype=torch.int32)
        lens = pair_lens.repeat_interleave(2)
        pos = torch.arange(cap)
        tail = pos[None, :] >= lens[:, None].long()          # [B, cap]
        k[tail[:, None, :, None].expand_as(k)] = float("nan")
        v[tail[:, None, :, None].expand_as(v)] = float("nan")
        return Workload(cfg, B, NH, NKV, D, cap, q, k, v, lens, D ** -0.5)
    if cfg == 5:
        B, D, cap, steps = 2, 64, 32, 32
        q = _randn(g, steps, B, NH, D).bfloat16()
        k = _randn(g, B, NKV, cap, D).bfloat16()
        v = _randn(g, B, NKV, cap, D).bfloat16()
        lens = torch.arange(1, steps + 1, dtype=torch.int32)[:, None].expand(steps, B).contiguous()
        return Workload(cfg, B, NH, NKV, D, cap, q, k, v, lens, D ** -0.5)
    raise ValueError(f"unknown config {cfg}")


def algorithmic_bytes(batch_lens, num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """HBM bytes a decode-attention call must move: K and V of the valid positions, q, out and seq_lens.

    sum_b NKV * len_b * D * 2 B * 2 (K + V) + B * NH * D * 2 (q) + B * NH * D * 2 (out) + 4 * B (seq_lens).
    Masked tails, split partials and merge scratch are implementation overhead and are not counted.
    """
    lens = [int(x) for x in batch_lens]
    B = len(lens)
    kv = sum(num_kv_heads * L * head_dim * 2 * 2 for L in lens)
    return kv + 2 * B * num_q_heads * head_dim * 2 + 4 * B


def fused_algorithmic_bytes(batch_lens, num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    """HBM bytes of a fused decode step (bz_gqa_decode_fused): the attention call's bytes, plus the raw k and v
    projections (B * 2 NKV * D * 2), both norm weights (2 * D * 2), cos and sin (2 * B * D * 2), the new k and v
    written into the cache slot (B * 2 NKV * D * 2) and cache_pos (8). The q read is already in the attention term."""
    B = len(list(batch_lens))
    return (algorithmic_bytes(batch_lens, num_q_heads, num_kv_heads, head_dim) + 2 * B * 2 * num_kv_heads * head_dim * 2
            + 2 * head_dim * 2 + 2 * B * head_dim * 2 + 8)


def flops(batch_lens, num_q_heads: int, head_dim: int) -> int:
    """4 * NH * len * D per row (q . k and p . v, multiply-add = 2 FLOPs)."""
    return sum(4 * num_q_heads * int(L) * head_dim for L in batch_lens)
