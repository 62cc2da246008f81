"""torch.ops.wgkv.* on the GPU: each operator returns exactly what the direct
library call returns, and a function built from them traces and runs under
torch.compile (aot_eager: fake tensors through the Meta kernels, no code
generation) with the same result."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_ops_equal_direct_calls():
    import wgkv
    from wgkv.gate import GatingPredictor
    print("[torch_ops] equality with direct calls", flush=True)
    g = torch.Generator().manual_seed(0)
    B, S, Hq, Hkv, D, W = 1, 700, 8, 2, 128, 128
    q = torch.randn(B, S, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    gm = (torch.rand(B, Hkv, S, generator=g) < 0.3).to(DEV)
    md = wgkv.generate_sparse_indices(gm, W, B, Hkv, S)
    mo = torch.ops.wgkv.generate_sparse_indices(gm, W)
    R = (S + 63) // 64
    assert torch.equal(md[0], mo[0]) and torch.equal(md[1], mo[1]) and torch.equal(md[2], mo[2])
    for h in range(Hkv):  # only the prefix the kernels read (the last row's column count) carries meaning
        n = int(md[2][0, h, -1])
        assert n > 0 and torch.equal(md[3][0, h, 0, :n], mo[3][0, h, 0, :n])
    a = wgkv.sparse_attn_func(q, k, v, *md, softmax_scale=D ** -0.5)
    b = torch.ops.wgkv.sparse_attn(q, k, v, *mo, D ** -0.5)
    assert torch.equal(a, b)
    kc = torch.randn(64, 16, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(64, 16, D, generator=g).to(torch.bfloat16).to(DEV)
    qd = torch.randn(2, 1, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    sl = torch.tensor([[100, 3], [0, 128]], dtype=torch.int32, device=DEV)
    bt = torch.randperm(64, generator=g)[:32].view(2, Hkv, 8).to(torch.int32).to(DEV)
    assert torch.equal(wgkv.paged_decode_attn(qd, kc, vc, sl, bt, 0.1), torch.ops.wgkv.paged_decode_attn(qd, kc, vc, sl, bt, 0.1))
    gp = GatingPredictor(D, Hkv, ["pre_k", "post_k"], "gelu", 4.0, 1e-3, True, True).to(DEV)
    x1 = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
    x2 = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
    s1, m1 = gp.scores_and_mask(x1, x2, None, 0.5)  # bf16 inputs, 700 tokens: the packed path
    wn = (gp.pre_key_norm.weight.detach(), gp.post_key_norm.weight.detach(), None)
    packed = torch.ops.wgkv.gate_pack_weights(*wn, gp.conv1.weight.detach(), 3, True, Hkv, D, gp.inner_dim)
    assert torch.equal(packed, gp.packed_weights())
    args = (x1, x2, None, *wn, gp.conv1.weight.detach(), gp.conv1.bias.detach(), gp.conv2.weight.detach(),
            gp.conv2.bias.detach(), gp.inner_dim, 0, True, 0.0, 0.5)
    s2, m2 = torch.ops.wgkv.gate_scores_and_mask(*args, w1_packed=packed)
    assert torch.equal(s1, s2) and torch.equal(m1, m2)
    # without packed weights: the fp32 path, as the module function runs it
    s3, m3 = torch.ops.wgkv.gate_scores_and_mask(*args)
    s4, m4 = wgkv.gate.gate_scores_and_mask(*args)
    assert torch.equal(s3, s4) and torch.equal(m3, m4)


def test_compiled_graph_through_the_operators():
    import wgkv  # noqa: F401
    print("[torch_ops] torch.compile aot_eager", flush=True)
    g = torch.Generator().manual_seed(1)
    B, S, Hq, Hkv, D, W = 1, 512, 8, 2, 64, 128
    q = torch.randn(B, S, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, S, Hkv, D, generator=g).to(torch.bfloat16).to(DEV)
    gm = (torch.rand(B, Hkv, S, generator=g) < 0.3).to(DEV)

    def f(q, k, v, gm):
        md = torch.ops.wgkv.generate_sparse_indices(gm, W)
        return torch.ops.wgkv.sparse_attn(q, k, v, *md, D ** -0.5) * 2

    ref = f(q, k, v, gm)
    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    out = cf(q, k, v, gm)
    assert torch.equal(out, ref)
