"""The dispatcher registration of the path (torch.ops.wgkv.*), host only:
every operator is registered with its schema, and the Meta kernels give the
output shapes of the CUDA kernels (so graphs trace without running them)."""
import pytest
import torch


def test_registered_with_schemas():
    import wgkv  # noqa: F401  (registers the operators)
    names = {"sparse_attn", "paged_decode_attn", "generate_sparse_indices", "gate_scores_and_mask",
             "gate_pack_weights"}
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
    pk = torch.ops.wgkv.gate_pack_weights(wn, wn, None, w1, 3, True, Hkv, D, inner)
    sc2, _ = torch.ops.wgkv.gate_scores_and_mask(x, x, None, wn, wn, None, w1, b1, w2, b2, inner, 0, True, 0.0, 0.1,
                                                 w1_packed=pk)
    assert sc2.shape == sc.shape


@pytest.mark.parametrize("H,D,inner,n_in", [(8, 128, 512, 2), (2, 64, 96, 3), (8, 128, 192, 1), (4, 64, 256, 2)])
def test_pack_meta_size_is_the_library_size(H, D, inner, n_in):
    """The Meta kernel of gate_pack_weights allocates what
    wgkv_gate_packed_bytes (a host function of the library) asks for."""
    import wgkv
    w1 = torch.empty(H * inner, n_in * D, 1, device="meta")
    wn = torch.empty(D, device="meta")
    mask = (1 << n_in) - 1
    pk = torch.ops.wgkv.gate_pack_weights(wn, wn, wn, w1, mask, True, H, D, inner)
    assert pk.dtype == torch.uint8 and pk.numel() == wgkv._lib.lib().wgkv_gate_packed_bytes(H, inner, n_in * D, 0)
    pk1 = torch.ops.wgkv.gate_pack_weights(wn, wn, wn, w1, mask, True, H, D, inner, 1)  # bf16 parameters: one plane
    assert pk1.numel() == wgkv._lib.lib().wgkv_gate_packed_bytes(H, inner, n_in * D, 1)
    assert pk1.numel() == pk.numel() // 3 + 2 * 2 * 20 * 128 * 2  # plus the two activation tables
    # shapes the packed layout does not take
    assert wgkv._lib.lib().wgkv_gate_packed_bytes(H, 100, 2 * D, 0) == -1
    assert wgkv._lib.lib().wgkv_gate_packed_bytes(H, inner, 48, 0) == -1


def test_prefill_swap_point_contract():
    from wgkv import torch_ops
    with pytest.raises(NotImplementedError):
        torch_ops.sparse_attn_func(None, None, None, None, None, None, None, causal=False)
    with pytest.raises(NotImplementedError):
        torch_ops.sparse_attn_func(None, None, None, None, None, None, None, return_softmax_lse=True)
