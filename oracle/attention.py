"""CPU restatements of the reference's decode attention. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference semantics restated here:
  - repeat_kv head map, third_party/breeze-tts/models/breeze.py:245-256: KV head kvh serves q heads
    kvh*G .. kvh*G+G-1, i.e. q head h reads KV head h // G.
  - eager_attention_forward, models/breeze.py:259-286: softmax(q k^T * scaling + mask) v, mask sliced to the key
    length, softmax in fp32, probabilities cast back to the query dtype.
  - the decode mask, models/cudagraph/backbone_graph.py:239-252: valid KV = [pad_lens[b], position] inclusive,
    everything else finfo(dtype).min; the reference kernel excludes mask values <= -1e30
    (flash/csrc/bb_attn.cu:9-11, :114-115).
"""
from __future__ import annotations

import numpy as np

EXCLUDED = -1e30


def _row_range(b: int, seq_lens, kv_start, capacity: int) -> tuple[int, int]:
    """[start, end) of row b, clamped to 0 <= start <= end <= capacity (the library clamps the same way)."""
    end = min(max(int(seq_lens[b]), 0), capacity)
    start = 0 if kv_start is None else min(max(int(kv_start[b]), 0), end)
    return start, end


def expand_kv_heads(kv: np.ndarray, num_q_heads: int) -> np.ndarray:
    """[NKV, L, D] -> [NH, L, D] with q head h reading KV head h // G (repeat_kv, breeze.py:245-256)."""
    G = num_q_heads // kv.shape[0]
    return kv[np.arange(num_q_heads) // G]


def decode_attention(q, k, v, seq_lens, scale: float, kv_start=None, mask=None) -> np.ndarray:
    """Parity oracle. q [B, NH, D]; k, v [B, NKV, capacity, D]; seq_lens / kv_start [B]; mask [B or 1, >= capacity]
    additive (<= -1e30 excludes). Float64 math; positions outside [start, end) or excluded by the mask are sliced
    away (never multiplied by zero, so NaN there cannot leak). A row with no position gives 0. Returns float64
    [B, NH, D]."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, NH, D = q.shape
    cap = k.shape[2]
    out = np.zeros((B, NH, D), dtype=np.float64)
    for b in range(B):
        start, end = _row_range(b, seq_lens, kv_start, cap)
        if end <= start:
            continue
        kh = expand_kv_heads(k[b, :, start:end], NH)   # [NH, L, D]
        vh = expand_kv_heads(v[b, :, start:end], NH)
        s = np.einsum("hd,hld->hl", q[b], kh) * scale
        keep = np.ones(end - start, dtype=bool)
        if mask is not None:
            m = np.asarray(mask, dtype=np.float64)
            m = m[b if m.shape[0] > 1 else 0, start:end]
            keep = m > EXCLUDED
            s = s + np.where(keep, m, 0.0)
        if not keep.any():
            continue
        s = s[:, keep]
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[b] = np.einsum("hl,hld->hd", p, vh[:, keep])
    return out


def decode_probabilities(q, k, seq_lens, scale: float, kv_start=None, mask=None) -> np.ndarray:
    """The softmax probabilities behind decode_attention: float64 [B, NH, capacity], softmax(q . k * scale + mask) over
    each row's [start, end) with mask-excluded positions dropped, 0 outside the range, at excluded positions and for
    rows with nothing to attend. The reference's optional dbg output of attn_decode (flash/csrc/bb_attn.cu:288-289)
    holds these probabilities rounded to bf16."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    B, NH, D = q.shape
    cap = k.shape[2]
    probs = np.zeros((B, NH, cap), dtype=np.float64)
    for b in range(B):
        start, end = _row_range(b, seq_lens, kv_start, cap)
        if end <= start:
            continue
        kh = expand_kv_heads(k[b, :, start:end], NH)
        s = np.einsum("hd,hld->hl", q[b], kh) * scale
        keep = np.ones(end - start, dtype=bool)
        if mask is not None:
            m = np.asarray(mask, dtype=np.float64)
            m = m[b if m.shape[0] > 1 else 0, start:end]
            keep = m > EXCLUDED
            s = s + np.where(keep, m, 0.0)
        if not keep.any():
            continue
        sk = s[:, keep]
        e = np.exp(sk - sk.max(axis=1, keepdims=True))
        p = np.zeros_like(s)
        p[:, keep] = e / e.sum(axis=1, keepdims=True)
        probs[b, :, start:end] = p
    return probs


def sdpa_fp32(q, k, v, seq_lens, scale: float, kv_start=None):
    """The north-star oracle verbatim: torch scaled_dot_product_attention in fp32 on the CPU with the KV heads
    expanded, sliced per row to [start, end). q [B, NH, D]; k, v [B, NKV, capacity, D] (torch tensors of any
    float dtype). Returns a float32 torch tensor [B, NH, D]."""
    import torch
    import torch.nn.functional as F

    q = q.float().cpu()
    k = k.float().cpu()
    v = v.float().cpu()
    B, NH, D = q.shape
    G = NH // k.shape[1]
    out = torch.zeros(B, NH, D, dtype=torch.float32)
    for b in range(B):
        start, end = _row_range(b, seq_lens, kv_start, k.shape[2])
        if end <= start:
            continue
        kh = k[b, :, start:end].repeat_interleave(G, dim=0)  # == repeat_kv for this row
        vh = v[b, :, start:end].repeat_interleave(G, dim=0)
        o = F.scaled_dot_product_attention(q[b][:, None, :], kh, vh, scale=scale)
        out[b] = o[:, 0, :]
    return out


def decode_attention_tokens(q, k, v, seq_lens, scale: float, kv_start=None, mask=None) -> np.ndarray:
    """T query tokens per row, causal among themselves: the row's tokens are its last T positions and token t
    attends [start, end - (T - 1 - t)) (the depth transformer's first step, flash/csrc/depth_frame.cu:221-227:
    token t of step 0 attends positions 0..t). q [B, NH, T, D]; k, v, seq_lens, kv_start, mask as decode_attention.
    Returns float64 [B, T, NH, D]."""
    q = np.asarray(q, dtype=np.float64)
    B, NH, T, D = q.shape
    cap = np.asarray(k).shape[2]
    out = np.zeros((B, T, NH, D), dtype=np.float64)
    for t in range(T):
        ends = np.zeros(B, dtype=np.int64)
        for b in range(B):
            start, end = _row_range(b, seq_lens, kv_start, cap)
            ends[b] = max(start, end - (T - 1 - t))
        out[:, t] = decode_attention(q[:, :, t], k, v, ends, scale, kv_start=kv_start, mask=mask)
    return out


def repeat_kv(x, n_rep: int):
    """torch [B, NKV, S, D] -> [B, NKV * n_rep, S, D] (models/breeze.py:245-256)."""
    if n_rep == 1:
        return x
    B, NKV, S, D = x.shape
    return x[:, :, None, :, :].expand(B, NKV, n_rep, S, D).reshape(B, NKV * n_rep, S, D)


def eager_bf16(query, key, value, mask, scaling: float):
    """The reference's eager decode attention chain on the CPU (models/breeze.py:259-286): query [B, NH, 1, D],
    key/value [B, NKV, S, D] in bf16, additive mask [B or 1, 1, 1, >= S]. Returns [B, 1, NH, D] bf16. This is the
    CPU baseline's code under test; it is not the parity oracle (it rounds scores and probabilities to bf16)."""
    import torch

    G = query.shape[1] // key.shape[1]
    key_states = repeat_kv(key, G)
    value_states = repeat_kv(value, G)
    attn_weights = torch.matmul(query, key_states.transpose(2, 3)) * scaling
    if mask is not None:
        attn_weights = attn_weights + mask[:, :, :, : key_states.shape[-2]]
    attn_weights = torch.nn.functional.softmax(attn_weights, dim=-1, dtype=torch.float32).to(query.dtype)
    attn_output = torch.matmul(attn_weights, value_states)
    return attn_output.transpose(1, 2).contiguous()


def interval_mask(pad_lens, position: int, capacity: int, dtype=None):
    """The reference's decode mask (backbone_graph.py:239-252): [B, 1, 1, capacity], 0 on [pad_lens[b], position],
    finfo(dtype).min elsewhere. torch tensor (dtype default bf16)."""
    import torch

    dtype = dtype or torch.bfloat16
    pad = torch.as_tensor(pad_lens, dtype=torch.long)
    kv = torch.arange(capacity, dtype=torch.long)
    valid = (kv[None, :] >= pad[:, None]) & (kv[None, :] <= position)
    m = torch.full((pad.numel(), 1, 1, capacity), torch.finfo(dtype).min, dtype=dtype)
    m[:, 0, 0, :].masked_fill_(valid, 0.0)
    return m


def mask_interval(mask) -> tuple[np.ndarray, np.ndarray]:
    """(start, end) int32 per mask row: first and last+1 position with value > -1e30; (0, 0) if none."""
    m = np.asarray(mask, dtype=np.float64)
    m = m.reshape(m.shape[0], m.shape[-1])
    start = np.zeros(m.shape[0], dtype=np.int32)
    end = np.zeros(m.shape[0], dtype=np.int32)
    for b in range(m.shape[0]):
        idx = np.nonzero(m[b] > EXCLUDED)[0]
        if idx.size:
            start[b], end[b] = idx[0], idx[-1] + 1
    return start, end


# ---------------------------------------------------------------------------------------------- fused prologue

def qk_norm_rope(x_bits, w_bits, eps: float, cos_bits, sin_bits):
    """Qwen3 per-head RMSNorm then RoPE, at the eager bf16 rounding points (flash/csrc/bb_attn.cu:78-100, which
    reproduces transformers' Qwen3RMSNorm + apply_rotary_pos_emb, models/breeze.py:211-242):
        h = bf16(x * rsqrt(mean(x^2) + eps))          (x, mean, rsqrt in fp32)
        y = bf16(w * h)
        out = bf16(bf16(y * cos) + bf16(rotate_half(y) * sin)),  rotate_half(y) = [-y[D/2:], y[:D/2]]
    x_bits [..., D], w/cos/sin bits broadcastable to it, all bf16 bit patterns (uint16). Returns uint16 bits."""
    from .bf16 import bf16_to_f32, f32_to_bf16, round_to_bf16

    x = bf16_to_f32(x_bits).astype(np.float32)
    w = bf16_to_f32(w_bits).astype(np.float32)
    cos = bf16_to_f32(cos_bits).astype(np.float32)
    sin = bf16_to_f32(sin_bits).astype(np.float32)
    var = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps), dtype=np.float32)).astype(np.float32)
    h = round_to_bf16((x * r).astype(np.float32))
    y = round_to_bf16((w * h).astype(np.float32))
    half = y.shape[-1] // 2
    rot = np.concatenate([-y[..., half:], y[..., :half]], axis=-1)
    a = round_to_bf16((y * cos).astype(np.float32))
    b = round_to_bf16((rot * sin).astype(np.float32))
    return f32_to_bf16((a + b).astype(np.float32))


def fused_decode(qkv_bits, qn_w_bits, kn_w_bits, eps: float, cos_bits, sin_bits, k_bits, v_bits, cache_pos: int,
                 seq_lens, scale: float, kv_start=None, mask=None):
    """Restatement of attn_decode_fused (bb_attn.cu:433-460, prologue :118-149): split the raw projections
    qkv [B, (NH + 2 NKV) * D] into q | k | v heads, apply q_norm / k_norm + RoPE (qk_norm_rope, cos/sin [B, D]),
    write the new k (normed, roped) and v (raw) into cache slot cache_pos of every row (when 0 <= cache_pos <
    capacity), then attend with decode_attention over the updated cache. Bits are bf16 patterns (uint16).
    Returns (out float64 [B, NH, D], k_bits, v_bits) with the updated caches (copies)."""
    from .bf16 import bf16_to_f32

    B, NKV, cap, D = k_bits.shape
    NH = qkv_bits.shape[1] // D - 2 * NKV
    heads = qkv_bits.reshape(B, NH + 2 * NKV, D)
    cs, sn = cos_bits.reshape(B, 1, D), sin_bits.reshape(B, 1, D)
    q = qk_norm_rope(heads[:, :NH], qn_w_bits, eps, cs, sn)
    k_new = qk_norm_rope(heads[:, NH:NH + NKV], kn_w_bits, eps, cs, sn)
    v_new = heads[:, NH + NKV:]
    k_bits, v_bits = k_bits.copy(), v_bits.copy()
    if 0 <= cache_pos < cap:
        k_bits[:, :, cache_pos] = k_new
        v_bits[:, :, cache_pos] = v_new
    out = decode_attention(bf16_to_f32(q), bf16_to_f32(k_bits), bf16_to_f32(v_bits), seq_lens, scale,
                           kv_start=kv_start, mask=mask)
    return out, k_bits, v_bits


def rope_cos_sin(positions, head_dim: int, base: float = 1_000_000.0):
    """Standard RoPE tables for the given positions (the Qwen3 default rope_theta is 1e6): cos/sin [n, head_dim]
    float32 with inv_freq = base^(-2i/D) repeated over both halves, as transformers' rotary embedding builds them."""
    pos = np.asarray(positions, dtype=np.float64)[:, None]
    inv = base ** (-np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = pos * inv[None, :]
    emb = np.concatenate([ang, ang], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)
