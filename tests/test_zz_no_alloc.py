"""The allocation-free decode entry point (wgkv_paged_decode_attn_noalloc,
static device scratch) against wgkv_paged_decode_attn with a workspace,
through the C ABI: bit-identical outputs on two calls in a row, the second
with a smaller batch and shorter heads (the scratch keeps the first call's
partials, which the second must not see)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ragged_case(B, Hq, Hkv, D, max_len, seed):
    g = torch.Generator().manual_seed(seed)
    P = 16
    sl = torch.randint(1, max_len + 1, (B, Hkv), generator=g, dtype=torch.int32)
    maxb = (max_len + P - 1) // P
    nb = B * Hkv * maxb + 1
    bt = torch.randperm(nb, generator=g)[: B * Hkv * maxb].view(B, Hkv, maxb).to(torch.int32)
    q = torch.randn(B, 1, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    v = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    dev = torch.device("cuda:0")
    return [t.to(dev) for t in (q, k, v, sl, bt)]


def _call_noalloc(q, k, v, sl, bt, scale):
    from wgkv import _lib
    B, _, Hq, D = q.shape
    Hkv = sl.shape[1]
    out = torch.empty_like(q)
    q3, o3 = q[:, 0], out[:, 0]
    st = _lib.lib().wgkv_paged_decode_attn_noalloc(
        q3.data_ptr(), q3.stride(0), q3.stride(1),
        k.data_ptr(), v.data_ptr(), k.shape[0], k.shape[1],
        sl.data_ptr(), sl.stride(0),
        bt.data_ptr(), bt.stride(0), bt.stride(1), bt.shape[2],
        o3.data_ptr(), o3.stride(0), o3.stride(1),
        B, Hq, Hkv, D, float(scale), _lib.stream_handle(q.device))
    _lib.check(st, "wgkv_paged_decode_attn_noalloc")
    return out


@pytest.mark.parametrize("G", [4, 8])
def test_noalloc_matches_workspace_entry_point(G):
    import wgkv
    from oracle import attention
    cases = [(4, 8 * G, 8, 128, 20000, 1), (1, 2 * G, 2, 64, 3000, 2)]  # the second call is smaller
    for B, Hq, Hkv, D, max_len, seed in cases:
        q, k, v, sl, bt = _ragged_case(B, Hq, Hkv, D, max_len, seed + 10 * G)
        print(f"[no-alloc] G={G} B={B} Hkv={Hkv} D={D} max_len={max_len}", flush=True)
        a = _call_noalloc(q, k, v, sl, bt, D ** -0.5)
        b = wgkv.paged_decode_attn(q, k, v, sl, bt, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        ref = attention.paged_decode(q.cpu(), k.cpu(), v.cpu(), sl.cpu(), bt.cpu(), D ** -0.5)
        err = (a.float().cpu() - ref).abs()
        assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3


def test_noalloc_rejects_too_many_heads():
    from wgkv import _lib
    q, k, v, sl, bt = _ragged_case(1, 8, 2, 128, 64, 3)
    st = _lib.lib().wgkv_paged_decode_attn_noalloc(
        q.data_ptr(), 0, 128, k.data_ptr(), v.data_ptr(), k.shape[0], 16, sl.data_ptr(), 2,
        bt.data_ptr(), 0, bt.shape[2], bt.shape[2], q.data_ptr(), 0, 128,
        1025, 8, 2, 128, 0.1, _lib.stream_handle(q.device))
    assert st == _lib.ERR_UNSUPPORTED
