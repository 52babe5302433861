"""Pins of the GEMV oracle (oracle.gemv): library routines (transformers' Qwen3RMSNorm, torch's bf16 F.linear and
F.silu on the CPU, which the eager chain of the reference's backbone runs), closed forms, invariants and planted
mistakes. bf16 results may differ from the library by one ulp where a different fp32 summation order moves a value
across a rounding boundary."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.gemv import decoder_layer, gemv, rmsnorm

qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


def _t(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _bf16(rng, *shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def within_ulp(a, b, frac_exact=0.99):
    fa, fb = bf16_to_f32(a).astype(np.float64), bf16_to_f32(b).astype(np.float64)
    ok = np.abs(fa - fb) <= np.abs(fb) * 2.0 ** -7 + 1e-30
    return bool(ok.all() and (a == b).mean() >= frac_exact)


@pytest.mark.parametrize("K", [64, 2048])
def test_rmsnorm_matches_transformers(K):
    rng = np.random.default_rng(K)
    x, w = _bf16(rng, 4, K, scale=3.0), f32_to_bf16((1 + 0.3 * rng.standard_normal(K)).astype(np.float32))
    norm = qwen3.Qwen3RMSNorm(K, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(_t(w).float())
        ref = _bits(norm.to(torch.bfloat16)(_t(x)))
    assert within_ulp(rmsnorm(x, w, 1e-6), ref)


def test_plain_and_segments_match_torch_linear():
    rng = np.random.default_rng(1)
    x = _bf16(rng, 2, 512)
    W = [_bf16(rng, n, 512, scale=0.05) for n in (96, 32, 32)]
    ref = _bits(F.linear(_t(x), _t(np.concatenate(W))))
    assert within_ulp(gemv(x, W), ref)
    # segments are the rows of the concatenation
    parts = np.concatenate([gemv(x, [w]) for w in W], axis=1)
    assert np.array_equal(gemv(x, W), parts)


def test_prologue_residual_and_silu_match_torch():
    rng = np.random.default_rng(2)
    K, N = 256, 128
    x, nw = _bf16(rng, 2, K, scale=2.0), f32_to_bf16((1 + 0.2 * rng.standard_normal(K)).astype(np.float32))
    Wg, Wu, Wo = _bf16(rng, N, K, scale=0.06), _bf16(rng, N, K, scale=0.06), _bf16(rng, N, K, scale=0.06)
    res = _bf16(rng, 2, N)
    norm = qwen3.Qwen3RMSNorm(K, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(_t(nw).float())
        xn = norm.to(torch.bfloat16)(_t(x))
        act = F.silu(F.linear(xn, _t(Wg))) * F.linear(xn, _t(Wu))     # Qwen3MLP: act_fn(gate_proj(x)) * up_proj(x)
        resid = _t(res) + F.linear(_t(x), _t(Wo))                     # residual add after the bf16 linear
    assert within_ulp(gemv(x, [Wg, Wu], nw, 1e-5, epilogue="silu_mul"), _bits(act), 0.98)
    assert within_ulp(gemv(x, [Wo], epilogue="residual", res_bits=res), _bits(resid))


def test_closed_forms():
    rng = np.random.default_rng(3)
    x = _bf16(rng, 2, 64)
    eye = f32_to_bf16(np.eye(64, dtype=np.float32))
    zero = f32_to_bf16(np.zeros((64, 64), np.float32))
    res = _bf16(rng, 2, 64)
    assert np.array_equal(gemv(x, [eye]), x)                                      # identity weights
    assert np.array_equal(gemv(x, [zero], epilogue="residual", res_bits=res), res)  # zero weights: y = res
    assert (bf16_to_f32(gemv(x, [zero, eye], epilogue="silu_mul")) == 0).all()   # silu(0) * up = 0
    big = f32_to_bf16(np.full((2, 64), 40.0, np.float32))                        # silu(g) = g for large g
    assert np.array_equal(gemv(big, [eye, eye], epilogue="silu_mul"),
                          f32_to_bf16(np.full((2, 64), 1600.0, np.float32)))
    # RMSNorm is scale invariant at eps = 0 (a power of two scales every rounding point exactly)
    nw = f32_to_bf16((1 + 0.3 * rng.standard_normal(64)).astype(np.float32))
    assert np.array_equal(rmsnorm(f32_to_bf16(bf16_to_f32(x) * 8), nw, 0.0), rmsnorm(x, nw, 0.0))


def test_planted_mistakes_caught():
    rng = np.random.default_rng(4)
    K, N = 256, 128
    x = _bf16(rng, 2, K)
    W = _bf16(rng, N, K, scale=0.06)
    res = _bf16(rng, 2, N, scale=50.0)
    ref_resid = _bits(_t(res) + F.linear(_t(x), _t(W)))
    good = gemv(x, [W], epilogue="residual", res_bits=res)
    assert within_ulp(good, ref_resid)
    # the residual added to the unrounded fp32 product (no bf16 rounding of the GEMV first)
    acc = bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(W).astype(np.float64).T
    unrounded = f32_to_bf16((bf16_to_f32(res) + acc.astype(np.float32)).astype(np.float32))
    assert not np.array_equal(unrounded, ref_resid)
    # transposed weights
    Ws = _bf16(rng, K, K, scale=0.06)
    assert not within_ulp(gemv(x, [f32_to_bf16(bf16_to_f32(Ws).T.copy())]), _bits(F.linear(_t(x), _t(Ws))), 0.5)
    # silu applied after the product with up
    Wg, Wu = _bf16(rng, N, K, scale=0.06), _bf16(rng, N, K, scale=0.06)
    ref_act = _bits(F.silu(F.linear(_t(x), _t(Wg))) * F.linear(_t(x), _t(Wu)))
    wrong = _bits(F.silu(F.linear(_t(x), _t(Wg)) * F.linear(_t(x), _t(Wu))))
    assert within_ulp(gemv(x, [Wg, Wu], epilogue="silu_mul"), ref_act, 0.98)
    assert not within_ulp(wrong, ref_act, 0.5)
    # eps outside the square root of the RMSNorm
    nw = f32_to_bf16(np.ones(K, np.float32))
    xs = _bf16(rng, 2, K, scale=0.01)
    xf = bf16_to_f32(xs)
    bad = f32_to_bf16(bf16_to_f32(f32_to_bf16(xf / (np.sqrt((xf ** 2).mean(-1, keepdims=True)) + 0.5))))
    assert not within_ulp(bad, rmsnorm(xs, nw, 0.5), 0.5)


def _fp32_attention(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
    """fp32 softmax attention over the whole cache (one query token, no mask), KV heads expanded by h // G, output
    rounded to bf16: the attention the oracle restates (float64 there)."""
    G = query.shape[1] // key.shape[1]
    k = key.float().repeat_interleave(G, dim=1)
    v = value.float().repeat_interleave(G, dim=1)
    p = torch.softmax(query.float() @ k.transpose(-1, -2) * scaling, dim=-1)
    return (p @ v).to(query.dtype).transpose(1, 2).contiguous(), None


def test_decoder_layer_matches_transformers():
    """oracle.gemv.decoder_layer (the reference's per-layer chain, flash/backbone.py:122-128) against transformers'
    Qwen3DecoderLayer in bf16 on the CPU, one decode token per row over a DynamicCache holding 37 earlier positions,
    with the attention computed in fp32 on both sides: the output, the new cache slot's k (normed, roped) and v."""
    from transformers import AttentionInterface, DynamicCache, Qwen3Config

    AttentionInterface.register("oracle_pin_fp32", _fp32_attention)
    H, NH, NKV, D, INTER, B, L = 256, 4, 2, 64, 512, 2, 37
    cfg = Qwen3Config(vocab_size=16, hidden_size=H, intermediate_size=INTER, num_hidden_layers=1,
                      num_attention_heads=NH, num_key_value_heads=NKV, head_dim=D, rms_norm_eps=1e-6,
                      max_position_embeddings=128)
    cfg._attn_implementation = "oracle_pin_fp32"
    torch.manual_seed(5)
    layer = qwen3.Qwen3DecoderLayer(cfg, layer_idx=0).eval()
    with torch.no_grad():
        for name, prm in layer.named_parameters():
            if "norm" in name:
                prm.copy_(1 + 0.1 * torch.randn_like(prm))
            else:
                prm.copy_(torch.randn_like(prm) * prm.shape[1] ** -0.5)
    layer = layer.to(torch.bfloat16)
    rot = qwen3.Qwen3RotaryEmbedding(cfg)
    rng = np.random.default_rng(6)
    k_prev, v_prev = _bf16(rng, B, NKV, L, D), _bf16(rng, B, NKV, L, D)
    x = _bf16(rng, B, H, scale=2.0)
    xt = _t(x)[:, None]
    pos_ids = torch.full((B, 1), L, dtype=torch.long)
    cos, sin = rot(xt, pos_ids)
    cache = DynamicCache()
    cache.update(_t(k_prev), _t(v_prev), 0)
    with torch.no_grad():
        ref = layer(xt, attention_mask=None, position_ids=pos_ids, past_key_values=cache, use_cache=True,
                    position_embeddings=(cos, sin))
    ref = _bits(ref[:, 0])
    k_ref, v_ref = (_bits(t[:, :, L]) for t in (cache.layers[0].keys, cache.layers[0].values))

    sd = {n: _bits(t) for n, t in layer.state_dict().items()}
    p = dict(ln1=sd["input_layernorm.weight"], ln2=sd["post_attention_layernorm.weight"],
             qn=sd["self_attn.q_norm.weight"], kn=sd["self_attn.k_norm.weight"], wq=sd["self_attn.q_proj.weight"],
             wk=sd["self_attn.k_proj.weight"], wv=sd["self_attn.v_proj.weight"], wo=sd["self_attn.o_proj.weight"],
             wg=sd["mlp.gate_proj.weight"], wu=sd["mlp.up_proj.weight"], wd=sd["mlp.down_proj.weight"], eps=1e-6,
             qk_eps=1e-6, scale=D ** -0.5)
    kc = np.zeros((B, NKV, L + 1, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :, :L], vc[:, :, :L] = k_prev, v_prev
    r = bf16_to_f32(ref).astype(np.float64)
    rms = np.sqrt((r ** 2).mean())

    def close(params):
        out, k2, v2 = decoder_layer(x, params, _bits(cos[:, 0]), _bits(sin[:, 0]), kc, vc, L, np.full(B, L + 1))
        g = bf16_to_f32(out).astype(np.float64)
        return bool(np.array_equal(v2[:, :, L], v_ref) and within_ulp(k2[:, :, L], k_ref, 0.98)
                    and (np.abs(g - r) <= 2.0 ** -6 * np.abs(r) + 2.0 ** -6 * rms).all() and (out == ref).mean() >= 0.9)

    assert close(p)
    # planted mistakes: the two layer norms' weights swapped; the MLP's gate and up swapped
    assert not close({**p, "ln1": p["ln2"], "ln2": p["ln1"]})
    assert not close({**p, "wg": p["wu"], "wu": p["wg"]})
