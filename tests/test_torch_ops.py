"""The dispatcher registration of the path (torch.ops.wgkv.*), host only:
every operator is registered with its schema, and the Meta kernels give the
output shapes of the CUDA kernels (so graphs trace without running them)."""
import pytest
import torch


def test_registered_with_schemas():
    import wgkv  # noqa: F401  (registers the operators)
    names = {"sparse_attn", "paged_decode_attn", "generate_sparse_indices", "gate_scores_and_mask"}
    for n in names:
        op = getattr(torch.ops.wgkv, n)
        schema = str(op.default._schema)
        assert schema.startswith(f"wgkv::{n}("), schema


@pytest.mark.parametrize("S,W", [(300, 128), (64, 64), (4096, 1024)])
def test_meta_shapes(S, W):
    import wgkv  # noqa: F401
    B, Hq, Hkv, D = 1, 8, 2, 128
    meta = dict(device="meta")
    q = torch.empty(B, S, Hq, D, dtype=torch.bfloat16, **meta)
    k = torch.empty(B, S, Hkv, D, dtype=torch.bfloat16, **meta)
    gm = torch.empty(B, Hkv, S, dtype=torch.bool, **meta)
    bc, bo, cc, ci = torch.ops.wgkv.generate_sparse_indices(gm, W)
    R = (S + 63) // 64
    assert bc.shape == (1, 1, R) and bo.shape == (1, 1, R, min(W // 64, R) + 1)
    assert cc.shape == (B, Hkv, R) and ci.shape == (B, Hkv, 1, S) and ci.dtype == torch.int32
    out = torch.ops.wgkv.sparse_attn(q, k, k, bc, bo, cc, ci, D ** -0.5)
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    qd = torch.empty(2, 1, Hq, D, dtype=torch.bfloat16, **meta)
    kc = torch.empty(64, 16, D, dtype=torch.bfloat16, **meta)
    sl = torch.empty(2, Hkv, dtype=torch.int32, **meta)
    bt = torch.empty(2, Hkv, 8, dtype=torch.int32, **meta)
    od = torch.ops.wgkv.paged_decode_attn(qd, kc, kc, sl, bt, D ** -0.5)
    assert od.shape == qd.shape
    inner = 4 * D
    w1 = torch.empty(Hkv * inner, 2 * D, 1, **meta)
    b1 = torch.empty(Hkv * inner, **meta)
    w2 = torch.empty(Hkv, inner, 1, **meta)
    b2 = torch.empty(Hkv, **meta)
    wn = torch.empty(D, **meta)
    x = torch.empty(B, Hkv, S, D, dtype=torch.bfloat16, **meta)
    sc, mk = torch.ops.wgkv.gate_scores_and_mask(x, x, None, wn, wn, None, w1, b1, w2, b2, inner, 0, True, 0.0, 0.1)
    assert sc.shape == (B, Hkv, S) and sc.dtype == torch.float32 and mk.dtype == torch.bool


def test_prefill_swap_point_contract():
    from wgkv import torch_ops
    with pytest.raises(NotImplementedError):
        torch_ops.sparse_attn_func(None, None, None, None, None, None, None, causal=False)
    with pytest.raises(NotImplementedError):
        torch_ops.sparse_attn_func(None, None, None, None, None, None, None, return_softmax_lse=True)
