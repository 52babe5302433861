"""GPU: the registered torch operators (torch_ops.py, namespace "bz") under torch.compile. The package functions become
single opaque nodes while dynamo traces them, so fullgraph=True compiles (any graph break would raise), and the
compiled results equal the eager ones bit for bit (the same kernels run). torch.library.opcheck checks the operator
registrations (schema, fake implementations, mutation declarations) against real calls."""
import pytest
import torch

from breeze_tts_2_flash_amd import gemv_resid, gemv_seg, gqa_decode, gqa_decode_fused, hf_attention, workloads
from tests.test_gpu_parity import rand_case

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16)


def test_compiled_attention_fullgraph(device):
    w, st = rand_case(91, 2, 16, 8, 128, 1024, [1000, 777], [0, 5])
    g = w.to(device)
    starts = st.to(device)

    def step(q, k, v, lens, kv_start):
        out = gqa_decode(q, k, v, lens, w.scale, kv_start=kv_start)
        return out.float().sum(-1), out

    torch._dynamo.reset()
    compiled = torch.compile(step, fullgraph=True)
    ref_sum, ref = step(g.q, g.k, g.v, g.seq_lens, starts)
    got_sum, got = compiled(g.q, g.k, g.v, g.seq_lens, starts)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(ref))
    # the reduction is inductor's own kernel in the compiled graph: another summation order, so not bit for bit
    torch.testing.assert_close(got_sum, ref_sum, rtol=1e-5, atol=1e-5)


def test_compiled_decoder_chain_fullgraph(device):
    """q|k|v GEMV -> fused attention (writes the cache slot) -> o_proj + residual, compiled as one graph."""
    B, NH, NKV, D, H, cap = 2, 16, 8, 128, 1024, 512
    gen = torch.Generator(device=device).manual_seed(92)

    def rnd(*shape, s=1.0):
        return (torch.randn(*shape, generator=gen, device=device) * s).bfloat16()

    x = rnd(B, H)
    nw, qn, kn = 1 + rnd(H, s=0.1), 1 + rnd(D, s=0.1), 1 + rnd(D, s=0.1)
    wq, wk, wv, wo = rnd(NH * D, H, s=H ** -0.5), rnd(NKV * D, H, s=H ** -0.5), rnd(NKV * D, H, s=H ** -0.5), \
        rnd(H, NH * D, s=(NH * D) ** -0.5)
    kc0, vc0 = rnd(B, NKV, cap, D), rnd(B, NKV, cap, D)
    cos, sin = rnd(B, D).float().cos().bfloat16(), rnd(B, D).float().sin().bfloat16()
    pos = torch.tensor([300], dtype=torch.int64, device=device)
    lens = torch.full((B,), 301, dtype=torch.int32, device=device)

    def chain(x, kc, vc):
        qkv = torch.empty(B, (NH + 2 * NKV) * D, dtype=torch.bfloat16, device=device)
        gemv_seg(x, nw, 1e-6, wq, wk, wv, qkv)
        ao = gqa_decode_fused(qkv, qn, kn, 1e-6, cos, sin, kc, vc, pos, D ** -0.5, seq_lens=lens)
        y = torch.empty_like(x)
        gemv_resid(ao.reshape(B, NH * D), wo, x, y)
        return y

    torch._dynamo.reset()
    compiled = torch.compile(chain, fullgraph=True)
    kc_e, vc_e = kc0.clone(), vc0.clone()
    kc_c, vc_c = kc0.clone(), vc0.clone()
    ref = chain(x, kc_e, vc_e)
    got = compiled(x, kc_c, vc_c)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(ref))
    assert torch.equal(_bits(kc_c), _bits(kc_e)) and torch.equal(_bits(vc_c), _bits(vc_e))  # the slot write happened


def test_registered_attention_function_compiles_fullgraph(device):
    """transformers' attention entry (hf_attention.mi355_decode_attention) for a q_len == 1 call with the eager mask,
    compiled without a graph break, equal to the eager call."""
    w, _ = rand_case(93, 2, 16, 8, 128, 256, [200, 200])
    g = w.to(device)
    from oracle.attention import interval_mask

    mask = interval_mask([0, 11], 199, 256).to(device)
    q4 = g.q[:, :, None, :]

    class M(torch.nn.Module):
        training = False

    mod = M()

    def attend(q, k, v, m):
        return hf_attention.mi355_decode_attention(mod, q, k, v, m, scaling=w.scale)[0]

    torch._dynamo.reset()
    compiled = torch.compile(attend, fullgraph=True)
    ref = attend(q4, g.k, g.v, mask)
    got = compiled(q4, g.k, g.v, mask)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("op", ["gqa_decode", "gemv_resid"])
def test_opcheck(device, op):
    if op == "gqa_decode":
        w = workloads.make(1)
        g = w.to(device)
        out = torch.empty(2, 16, 128, dtype=torch.bfloat16, device=device)
        args = (g.q, g.k, g.v, g.seq_lens, float(g.scale), out, None, None, 0, 0, 0, None)
        torch.library.opcheck(torch.ops.bz.gqa_decode.default, args)
    else:
        gen = torch.Generator(device=device).manual_seed(94)
        x = torch.randn(2, 512, generator=gen, device=device).bfloat16()
        W = (torch.randn(256, 512, generator=gen, device=device) * 0.05).bfloat16()
        res = torch.randn(2, 256, generator=gen, device=device).bfloat16()
        y = torch.empty(2, 256, dtype=torch.bfloat16, device=device)
        torch.library.opcheck(torch.ops.bz.gemv_resid.default, (x, W, res, y))


def test_compiled_calls_on_two_streams(device):
    """Compiled calls (default mode) issued on two streams at once, without synchronising between them: each stream's
    calls take that stream's own cached workspace, so calls in flight together share no arrival counters or partials,
    and every output equals the eager call bit for bit."""
    cases = [rand_case(95 + i, 2, 16, 8, 128, 2048, [2000 - 300 * i, 1500 + 200 * i], [0, 3 * i]) for i in range(2)]
    gs = [(w.to(device), st.to(device)) for w, st in cases]

    def step(q, k, v, lens, kv_start, out):
        gqa_decode(q, k, v, lens, cases[0][0].scale, out, kv_start=kv_start)
        return out

    refs = [gqa_decode(g.q, g.k, g.v, g.seq_lens, cases[0][0].scale, kv_start=st) for g, st in gs]
    torch._dynamo.reset()
    compiled = torch.compile(step, fullgraph=True)
    outs = [torch.empty_like(r) for r in refs]
    streams = [torch.cuda.Stream(device) for _ in range(2)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream(device))
    for it in range(30):
        for i, (g, st) in enumerate(gs):
            with torch.cuda.stream(streams[i]):
                compiled(g.q, g.k, g.v, g.seq_lens, st, outs[i])
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(_bits(outs[i]), _bits(refs[i])), f"stream {i}"


def test_compiled_attention_cudagraph_trees(device):
    """torch.compile(mode="reduce-overhead"): CUDA-graph trees warm the function up eagerly, record it into a graph,
    then replay it. The warm-up takes a stream workspace allocated outside the trees' memory pool (which must hold
    only the graph's outputs), the recording runs on the library's static scratch, and every call equals the eager
    result bit for bit."""
    w, st = rand_case(96, 2, 16, 8, 128, 2048, [1024, 1024])
    g = w.to(device)

    def step(q, k, v, lens):
        return gqa_decode(q, k, v, lens, w.scale)

    ref = step(g.q, g.k, g.v, g.seq_lens)
    torch._dynamo.reset()
    compiled = torch.compile(step, mode="reduce-overhead", fullgraph=True)
    for i in range(5):
        got = compiled(g.q, g.k, g.v, g.seq_lens).clone()
        torch.cuda.synchronize()
        assert torch.equal(_bits(got), _bits(ref)), f"call {i}"
    torch._dynamo.reset()
