"""A small stand-in for the reference's BackboneGraph (third_party/breeze-tts/models/cudagraph/backbone_graph.py), with
the attributes and the eager decode step that the reference's fused step reads and replaces: a transformers Qwen3Model
backbone, codebook embeddings summed per token, a StaticCache, the interval attention mask built from left padding and
the position (:239-252), an fp32 lm_head and classifier-free guidance over the cond / uncond halves (:254-286), and
capture() into one graph (:288-320). Test infrastructure only."""
from __future__ import annotations

import torch
from torch import nn


class CodebookEmbeddings(nn.Module):
    """One embedding table per codebook, summed: ids [B, 1, C] -> [B, 1, H]."""

    def __init__(self, codebooks: int, vocab: int, hidden: int):
        super().__init__()
        self.tables = nn.ModuleList(nn.Embedding(vocab, hidden) for _ in range(codebooks))

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        out = self.tables[0](ids[..., 0])
        for c in range(1, len(self.tables)):
            out = out + self.tables[c](ids[..., c])
        return out


class MiniBackboneGraph:
    def __init__(self, model, embed: CodebookEmbeddings, lm_head: nn.Linear, batch: int, max_seq_len: int,
                 guidance: float = 3.0):
        from transformers import StaticCache

        dev = next(model.parameters()).device
        self.model, self.embed_tokens, self.lm_head = model, embed, lm_head.float()
        self.device, self.batch_size, self.max_seq_len = dev, batch, max_seq_len
        self.half = batch // 2 if batch > 1 else batch
        self.hidden_size = model.config.hidden_size
        vocab, codebooks = lm_head.out_features, len(embed.tables)
        self.static_cache = StaticCache(config=model.config, max_cache_len=max_seq_len)
        self.cache_position = torch.zeros(1, dtype=torch.long, device=dev)
        self.position_ids = torch.zeros(batch, 1, dtype=torch.long, device=dev)
        self.guidance_scale = torch.tensor(guidance, dtype=torch.float32, device=dev)
        self.input_ids_buf = torch.zeros(batch, 1, codebooks, dtype=torch.long, device=dev)
        self.hidden_buf = torch.zeros(batch, 1, self.hidden_size, dtype=torch.bfloat16, device=dev)
        self.logits_buf = torch.zeros(batch, vocab, dtype=torch.float32, device=dev)
        self.cfg_logits_buf = torch.zeros(self.half, vocab, dtype=torch.float32, device=dev)
        self.attn_mask = torch.zeros(batch, 1, 1, max_seq_len, dtype=torch.bfloat16, device=dev)
        self.graph = None

    def prefill(self, keys, values) -> int:
        """Write per-layer K / V [B, NKV, P, D] (already normed and roped, as a prefill leaves them) at slots 0..P-1."""
        P = keys[0].shape[2]
        pos = torch.arange(P, device=self.device)
        for li, (k, v) in enumerate(zip(keys, values)):
            self.static_cache.update(k, v, li, {"cache_position": pos})
        return P

    def set_step(self, ids: torch.Tensor, pad_lens, cache_pos: int) -> None:
        """Inputs of one decode step: the new token ids, the cache slot and, per row, the RoPE position (cache_pos
        minus the row's left padding) and the interval mask [pad, cache_pos] (backbone_graph.py:239-252, :376-390)."""
        pads = torch.as_tensor(pad_lens, dtype=torch.long, device=self.device)
        self.input_ids_buf.copy_(ids)
        self.cache_position.fill_(cache_pos)
        self.position_ids.copy_((cache_pos - pads).unsqueeze(-1))
        kv = torch.arange(self.max_seq_len, device=self.device)
        valid = (kv[None, :] >= pads[:, None]) & (kv[None, :] <= cache_pos)
        self.attn_mask.fill_(torch.finfo(self.attn_mask.dtype).min)
        self.attn_mask[:, 0, 0, :].masked_fill_(valid, 0.0)
        # this transformers' StaticLayer writes at its own running length rather than at cache_position: point it at
        # the step's slot so the eager step writes where the reference's does
        for layer in self.static_cache.layers:
            if torch.is_tensor(getattr(layer, "cumulative_length", None)):
                layer.cumulative_length.fill_(cache_pos)

    def _decode_step(self) -> None:
        """The eager step: embeddings -> backbone over the static cache -> fp32 lm_head -> CFG."""
        emb = self.embed_tokens(self.input_ids_buf)
        out = self.model(inputs_embeds=emb, attention_mask=self.attn_mask, past_key_values=self.static_cache,
                         position_ids=self.position_ids, cache_position=self.cache_position, use_cache=True)
        self.hidden_buf.copy_(out.last_hidden_state)
        self.logits_buf.copy_(self.lm_head(self.hidden_buf[:, -1, :].float()))
        if self.batch_size >= 2:
            cond, uncond = self.logits_buf[:self.half], self.logits_buf[self.half:]
            self.cfg_logits_buf.copy_(uncond + self.guidance_scale * (cond - uncond))
        else:
            self.cfg_logits_buf.copy_(self.logits_buf[:self.half])

    def capture(self, warmup: int = 2) -> None:
        """Warm up on the current stream, then one eager step and the capture on a side stream."""
        for _ in range(warmup):
            self._decode_step()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._decode_step()
            torch.cuda.synchronize()
            with torch.cuda.graph(self.graph):
                self._decode_step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()


def bits(t: torch.Tensor):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view("uint16")


def build_graph(device, batch: int = 2, layers: int = 2, heads: int = 4, kv_heads: int = 2, hidden: int = 256,
                inter: int = 512, max_seq_len: int = 256, prefill: int = 100, seed: int = 0,
                attn_implementation: str = "eager") -> MiniBackboneGraph:
    """A random-init bf16 Qwen3 backbone (head_dim 128) in a MiniBackboneGraph, its cache prefilled with `prefill`
    random positions."""
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    cfg = Qwen3Config(vocab_size=64, hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=128, rms_norm_eps=1e-6,
                      max_position_embeddings=4096)
    cfg._attn_implementation = attn_implementation
    g = torch.Generator().manual_seed(seed)
    model = Qwen3Model(cfg).eval()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.copy_(1 + 0.1 * torch.randn(p.shape, generator=g))
            elif p.dim() == 2:
                p.copy_(torch.randn(p.shape, generator=g) * p.shape[1] ** -0.5)
    model = model.to(device=device, dtype=torch.bfloat16)
    embed = CodebookEmbeddings(2, 64, hidden)
    with torch.no_grad():
        for t in embed.tables:
            t.weight.copy_(torch.randn(t.weight.shape, generator=g))
    embed = embed.to(device=device, dtype=torch.bfloat16)
    lm_head = nn.Linear(hidden, 48, bias=False)
    with torch.no_grad():
        lm_head.weight.copy_(torch.randn(lm_head.weight.shape, generator=g) * hidden ** -0.5)
    graph = MiniBackboneGraph(model, embed, lm_head.to(device), batch, max_seq_len)
    ks = [torch.randn(batch, kv_heads, prefill, 128, generator=g).to(device, torch.bfloat16) for _ in range(layers)]
    vs = [torch.randn(batch, kv_heads, prefill, 128, generator=g).to(device, torch.bfloat16) for _ in range(layers)]
    graph.prefill(ks, vs)
    return graph


def layer_params(layer) -> dict:
    """oracle.gemv.decoder_layer's parameter dict (bf16 bits) of a transformers Qwen3 decoder layer."""
    at, mlp = layer.self_attn, layer.mlp
    return dict(ln1=bits(layer.input_layernorm.weight), ln2=bits(layer.post_attention_layernorm.weight),
                qn=bits(at.q_norm.weight), kn=bits(at.k_norm.weight), wq=bits(at.q_proj.weight),
                wk=bits(at.k_proj.weight), wv=bits(at.v_proj.weight), wo=bits(at.o_proj.weight),
                wg=bits(mlp.gate_proj.weight), wu=bits(mlp.up_proj.weight), wd=bits(mlp.down_proj.weight),
                eps=float(layer.input_layernorm.variance_epsilon), qk_eps=float(at.q_norm.variance_epsilon),
                scale=float(at.scaling))


def oracle_step(graph: MiniBackboneGraph, pad_lens, cache_pos: int):
    """The decode step of the graph's current inputs through the CPU oracle, on copies of its caches: the final hidden
    state bits [B, H] and the new K / V slot of every layer (bits [B, NKV, D])."""
    import numpy as np

    from oracle.gemv import decoder_layer, rmsnorm

    model, B = graph.model, graph.batch_size
    with torch.no_grad():
        emb = graph.embed_tokens(graph.input_ids_buf)
        cos, sin = model.rotary_emb(emb, graph.position_ids)
    x = bits(emb.reshape(B, -1))
    cos_b, sin_b = bits(cos.reshape(B, -1)), bits(sin.reshape(B, -1))
    seq_lens = np.full(B, cache_pos + 1)
    kv_start = np.asarray(pad_lens)
    slots = []
    for layer, c in zip(model.layers, graph.static_cache.layers):
        x, k2, v2 = decoder_layer(x, layer_params(layer), cos_b, sin_b, bits(c.keys), bits(c.values), cache_pos,
                                  seq_lens, kv_start=kv_start)
        slots.append((k2[:, :, cache_pos], v2[:, :, cache_pos]))
    norm = model.norm
    return rmsnorm(x, bits(norm.weight), float(norm.variance_epsilon)), slots
