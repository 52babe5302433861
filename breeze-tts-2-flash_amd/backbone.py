"""The backbone decode step on this library: a drop-in for the reference's fused step (flash/backbone.py), which
replaces BackboneGraph._decode_step (third_party/breeze-tts/models/cudagraph/backbone_graph.py:254-286) and is
captured by BackboneGraph.capture (:288-320) into one graph.

Per layer (flash/backbone.py:122-128):
    gemv_seg     RMSNorm + q | k | v projections                      (bz_gemv, plain epilogue)
    attention    q/k RMSNorm + RoPE + KV-cache write + GQA attention  (bz_gqa_decode_fused)
    gemv_resid   o_proj + residual                                    (bz_gemv, residual epilogue)
    gemv_gateup  RMSNorm + gate / up + SiLU * up                      (bz_gemv, silu_mul epilogue)
    gemv_resid   down + residual                                      (bz_gemv, residual epilogue)
then the final RMSNorm (bz_rmsnorm). The embedding, the rotary tables, the fp32 lm_head and CFG stay eager, as in the
reference (:113-134), and are captured with the rest.

How it differs from the reference's step:
  - the attention range comes from the graph's interval mask once per step (bz_mask_interval, one launch) instead of
    the mask being re-read by every layer's attention;
  - the attention workspace is allocated and zero-filled in prepare(), eagerly, so a captured step allocates
    nothing and its replays reuse it (its split counters return to zero at the end of every call);
  - supported graphs: batch 1..4 (the reference: 1, 2, 4), head_dim 128, q heads per KV head 1, 2, 4 or 8 (the
    reference: 2), any cache length.
A graph the kernels cannot take (other dtypes, biases, activations, head sizes, CPU tensors) keeps its original step,
with the reason printed once, as the reference does (flash/backbone.py:49-109). A missing library is an error, not a
fallback: prepare() loads it before looking at the graph.
"""
from __future__ import annotations

import torch

from . import kernels
from .attention import gqa_decode_fused, mask_interval, workspace_bytes
from .gemv import gemv_gateup, gemv_resid, gemv_seg, rmsnorm

ORIG: dict = {}          # the patched class's original methods, by name
_ACTS = ("SiLU", "SiLUActivation")


class Unsupported(Exception):
    """The graph's model is outside what the kernels take; the message says why."""


class LayerWeights:
    """One decoder layer's tensors and constants, as the step passes them to the kernels."""
    __slots__ = ("ln1_w", "ln1_eps", "wq", "wk", "wv", "qn_w", "kn_w", "qk_eps", "scaling", "wo", "ln2_w", "ln2_eps",
                 "wg", "wu", "wd")


def _need(cond: bool, why: str) -> None:
    if not cond:
        raise Unsupported(why)


def _dev_bf16(t, name: str) -> torch.Tensor:
    _need(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.bfloat16 and t.is_contiguous(),
          f"{name} is not a contiguous bf16 device tensor")
    return t


def _layer_weights(layer, i: int) -> LayerWeights:
    at, mlp = layer.self_attn, layer.mlp
    L = LayerWeights()
    L.ln1_w = _dev_bf16(layer.input_layernorm.weight, f"layer {i} input_layernorm")
    L.ln1_eps = float(layer.input_layernorm.variance_epsilon)
    L.ln2_w = _dev_bf16(layer.post_attention_layernorm.weight, f"layer {i} post_attention_layernorm")
    L.ln2_eps = float(layer.post_attention_layernorm.variance_epsilon)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        _need(getattr(getattr(at, name), "bias", None) is None, f"layer {i} {name} has a bias")
    for name in ("gate_proj", "up_proj", "down_proj"):
        _need(getattr(getattr(mlp, name), "bias", None) is None, f"layer {i} {name} has a bias")
    L.wq, L.wk = _dev_bf16(at.q_proj.weight, f"layer {i} q_proj"), _dev_bf16(at.k_proj.weight, f"layer {i} k_proj")
    L.wv, L.wo = _dev_bf16(at.v_proj.weight, f"layer {i} v_proj"), _dev_bf16(at.o_proj.weight, f"layer {i} o_proj")
    L.qn_w, L.kn_w = _dev_bf16(at.q_norm.weight, f"layer {i} q_norm"), _dev_bf16(at.k_norm.weight, f"layer {i} k_norm")
    L.qk_eps = float(at.q_norm.variance_epsilon)
    _need(float(at.k_norm.variance_epsilon) == L.qk_eps, f"layer {i}: q_norm and k_norm eps differ")
    L.scaling = float(at.scaling)
    L.wg = _dev_bf16(mlp.gate_proj.weight, f"layer {i} gate_proj")
    L.wu = _dev_bf16(mlp.up_proj.weight, f"layer {i} up_proj")
    L.wd = _dev_bf16(mlp.down_proj.weight, f"layer {i} down_proj")
    _need(type(getattr(mlp, "act_fn", None)).__name__ in _ACTS, f"layer {i}: the MLP activation is not SiLU")
    _need(at.head_dim == 128, f"layer {i}: head_dim {at.head_dim} (the fused attention takes 128)")
    _need(at.num_key_value_groups in (1, 2, 4, 8), f"layer {i}: {at.num_key_value_groups} q heads per KV head")
    _need(not getattr(at, "sliding_window", None), f"layer {i} uses a sliding window")
    return L


def _collect(graph) -> dict:
    model = graph.model
    layers = list(model.layers)
    _need(len(layers) > 0, "the model has no layers")
    B = int(graph.batch_size)
    _need(1 <= B <= 4, f"batch {B} (the GEMVs take 1..4 rows)")
    Ls = [_layer_weights(layer, i) for i, layer in enumerate(layers)]
    L0 = Ls[0]
    H, I = int(graph.hidden_size), L0.wg.shape[0]
    nq, nk = L0.wq.shape[0], L0.wk.shape[0]
    D = 128
    NH, NKV = nq // D, nk // D
    _need(nq % D == 0 and nk % D == 0 and L0.wv.shape[0] == nk, "q / k / v projection widths are not heads of 128")
    _need(H % 8 == 0 and I % 8 == 0, "hidden and intermediate sizes must be multiples of 8")
    for i, L in enumerate(Ls):
        shapes = (L.wq.shape, L.wk.shape, L.wv.shape, L.wo.shape, L.wg.shape, L.wu.shape, L.wd.shape)
        _need(shapes == ((nq, H), (nk, H), (nk, H), (H, nq), (I, H), (I, H), (H, I)), f"layer {i}: weight shapes")
    norm_w = _dev_bf16(model.norm.weight, "the final norm")
    dev = L0.wq.device
    reason = kernels.device_unsupported(dev.index)
    _need(reason is None, f"device {reason}")
    S = int(graph.max_seq_len)
    cache = graph.static_cache.layers
    _need(len(cache) == len(Ls), "the static cache and the model have different layer counts")
    with torch.cuda.device(dev):
        nbytes = workspace_bytes(B, NH, NKV, D, S)
    return dict(B=B, layers=Ls, norm_w=norm_w, norm_eps=float(model.norm.variance_epsilon), capacity=S,
                qkv=torch.empty(B, nq + 2 * nk, dtype=torch.bfloat16, device=dev),
                ao=torch.empty(B, 1, NH, D, dtype=torch.bfloat16, device=dev),
                h1=torch.empty(B, H, dtype=torch.bfloat16, device=dev),
                act=torch.empty(B, I, dtype=torch.bfloat16, device=dev),
                x=torch.empty(B, H, dtype=torch.bfloat16, device=dev),
                seq_lens=torch.zeros(B, dtype=torch.int32, device=dev),
                kv_start=torch.zeros(B, dtype=torch.int32, device=dev),
                ws=torch.zeros((nbytes + 255) // 256 * 256, dtype=torch.uint8, device=dev))


def prepare(graph) -> dict | None:
    """The step's state for this graph (weights, buffers, workspace), built once per batch size; None when the graph
    is unsupported (the reason is printed once per graph)."""
    st = getattr(graph, "_bz_state", None)
    if st is not None and st["B"] == graph.batch_size:
        return st
    kernels.load()
    try:
        st = _collect(graph)
    except Unsupported as e:
        if getattr(graph, "_bz_unsupported", None) != str(e):
            print(f"[breeze_tts_2_flash_amd] backbone decode step not taken: {e}; using the original step", flush=True)
        graph._bz_unsupported = str(e)
        return None
    graph._bz_state = st
    return st


def _logits_and_cfg(graph) -> None:
    """The eager tail of the step, unchanged: fp32 lm_head on the last hidden state, then classifier-free guidance
    over the cond / uncond halves (backbone_graph.py:269-286)."""
    graph.logits_buf.copy_(graph.lm_head(graph.hidden_buf[:, -1, :].float()))
    if graph.batch_size >= 2:
        cond, uncond = graph.logits_buf[:graph.half], graph.logits_buf[graph.half:]
        graph.cfg_logits_buf.copy_(uncond + graph.guidance_scale * (cond - uncond))
    else:
        graph.cfg_logits_buf.copy_(graph.logits_buf[:graph.half])


def fused_decode_step(graph) -> None:
    """One decode step of a BackboneGraph-like object (the attributes BackboneGraph._decode_step uses) on this
    library's kernels; the original step when prepare() declines the graph."""
    st = prepare(graph)
    if st is None:
        return ORIG["_decode_step"](graph)
    B = st["B"]
    emb = graph.embed_tokens(graph.input_ids_buf)                       # [B, 1, H], eager
    cos, sin = graph.model.rotary_emb(emb, graph.position_ids)          # [B, 1, 128] bf16, eager
    cos, sin = cos.contiguous(), sin.contiguous()
    x = emb.reshape(B, -1)
    mask_interval(graph.attn_mask, st["capacity"], B, st["seq_lens"], st["kv_start"])
    qkv, ao, h1, act, xb = st["qkv"], st["ao"], st["h1"], st["act"], st["x"]
    for L, c in zip(st["layers"], graph.static_cache.layers):
        gemv_seg(x, L.ln1_w, L.ln1_eps, L.wq, L.wk, L.wv, qkv)
        gqa_decode_fused(qkv, L.qn_w, L.kn_w, L.qk_eps, cos, sin, c.keys, c.values, graph.cache_position, L.scaling,
                         ao, seq_lens=st["seq_lens"], kv_start=st["kv_start"], workspace=st["ws"])
        gemv_resid(ao.view(B, -1), L.wo, x, h1)
        gemv_gateup(h1, L.ln2_w, L.ln2_eps, L.wg, L.wu, act)
        gemv_resid(act, L.wd, h1, xb)
        x = xb
    rmsnorm(x, st["norm_w"], st["norm_eps"], graph.hidden_buf.view(B, -1))
    _logits_and_cfg(graph)


def install(graph_cls) -> bool:
    """Replace graph_cls._decode_step (BackboneGraph's) with fused_decode_step; idempotent. Returns True when the step
    is (already) replaced. A visible GPU other than gfx950 declines with the reason printed and the original step
    kept (the reference's pre-flight, flash/support.py:67-84, flash/__init__.py:32-48); with no GPU visible the step is
    patched and every CPU graph keeps its original step through prepare(). The library is loaded first, so a missing
    or stale build fails here (flash/backbone.py:141-148)."""
    import torch

    if torch.cuda.is_available():
        reason = kernels.device_unsupported()
        if reason is not None:
            print(f"[breeze_tts_2_flash_amd] backbone decode step not installed: {reason}", flush=True)
            return False
    kernels.load()
    if "_decode_step" in ORIG:
        return True
    ORIG["_decode_step"] = graph_cls._decode_step
    graph_cls._decode_step = fused_decode_step
    return True


def uninstall(graph_cls) -> None:
    """Restore the original step."""
    if "_decode_step" in ORIG:
        graph_cls._decode_step = ORIG.pop("_decode_step")
