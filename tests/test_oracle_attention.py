"""Attention oracles pinned by float64 loops, closed forms and invariances."""
import pytest
import torch

from oracle import attention, meta


def paged_case(B, Hq, Hkv, D, page, max_len, num_blocks, seed, pad=-1):
    """Random paged cache like utils/test_flash_attn_with_kvcache.py:93-116."""
    g = torch.Generator().manual_seed(seed)
    maxb = (max_len + page - 1) // page
    seqlens = torch.randint(1, max_len + 1, (B, Hkv), generator=g, dtype=torch.int32)
    table = torch.full((B, Hkv, maxb), pad, dtype=torch.int32)
    avail = torch.randperm(num_blocks, generator=g)
    off = 0
    for b in range(B):
        for h in range(Hkv):
            n = (int(seqlens[b, h]) + page - 1) // page
            table[b, h, :n] = avail[off:off + n].to(torch.int32)
            off += n
    q = torch.randn(B, 1, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(num_blocks, page, D, generator=g).to(torch.bfloat16)
    v = torch.randn(num_blocks, page, D, generator=g).to(torch.bfloat16)
    return q, k, v, seqlens, table


@pytest.mark.parametrize("heads", [(4, 4), (8, 2), (8, 4)])
@pytest.mark.parametrize("page", [16, 32])
def test_decode_matches_float64_loop(heads, page):
    Hq, Hkv = heads
    q, k, v, sl, bt = paged_case(2, Hq, Hkv, 16, page, 70, 64, seed=Hq + page)
    ref = attention.paged_decode(q, k, v, sl, bt, 0.25, dtype=torch.float64)
    loop = attention.paged_decode_loop(q, k, v, sl, bt, 0.25)
    assert torch.allclose(ref, loop, atol=1e-10)


def test_decode_closed_forms():
    q, k, v, sl, bt = paged_case(1, 4, 2, 32, 16, 40, 16, seed=3)
    # identical keys -> uniform softmax -> mean of V rows
    k[:] = k[0, 0]
    out = attention.paged_decode(q, k, v, sl, bt, 0.1, dtype=torch.float64)
    for h in range(2):
        T = int(sl[0, h])
        rows = v[bt[0, h, :(T + 15) // 16].long()].reshape(-1, 32)[:T].double()
        assert torch.allclose(out[0, 0, 2 * h], rows.mean(0), atol=1e-12)
    # a single token -> that token's V row
    sl[:] = 1
    out = attention.paged_decode(q, k, v, sl, bt, 0.1, dtype=torch.float64)
    assert torch.allclose(out[0, 0, 0], v[bt[0, 0, 0]][0].double())
    # empty head -> zeros
    sl[0, 1] = 0
    out = attention.paged_decode(q, k, v, sl, bt, 0.1)
    assert torch.count_nonzero(out[0, 0, 2:]) == 0


def test_decode_page_permutation_invariance():
    q, k, v, sl, bt = paged_case(2, 8, 2, 64, 16, 300, 128, seed=9)
    perm = torch.randperm(128, generator=torch.Generator().manual_seed(1))
    inv = torch.argsort(perm)
    k2, v2 = k[perm], v[perm]
    bt2 = torch.where(bt >= 0, inv[bt.clamp(min=0).long()].to(torch.int32), bt)
    a = attention.paged_decode(q, k, v, sl, bt, 0.125)
    b = attention.paged_decode(q, k2, v2, sl, bt2, 0.125)
    assert torch.equal(a, b)


@pytest.mark.parametrize("S,W,G", [(70, 64, 2), (130, 64, 1), (200, 128, 3)])
def test_masked_prefill_matches_rowloop(S, W, G):
    g = torch.Generator().manual_seed(S)
    H = 2
    q = torch.randn(1, H * G, S, 16, generator=g).to(torch.bfloat16)
    k = torch.randn(1, H, S, 16, generator=g).to(torch.bfloat16)
    v = torch.randn(1, H, S, 16, generator=g).to(torch.bfloat16)
    gm = (torch.rand(1, H, S, generator=g) < 0.2).numpy()
    mask = meta.ideal_mask(gm, W, G)
    a = attention.masked_prefill(q, k, v, mask)
    b = attention.masked_prefill_rowloop(q, k, v, mask)
    assert torch.allclose(a, b, atol=1e-10)


def test_masked_prefill_full_mask_is_causal_sdpa():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 4, 50, 8, generator=g)
    k = torch.randn(1, 2, 50, 8, generator=g)
    v = torch.randn(1, 2, 50, 8, generator=g)
    gm = torch.ones(1, 2, 50, dtype=torch.bool).numpy()
    mask = meta.ideal_mask(gm, 64, 2)
    a = attention.masked_prefill(q, k, v, mask)
    b = torch.nn.functional.scaled_dot_product_attention(
        q.double(), k.double().repeat_interleave(2, 1), v.double().repeat_interleave(2, 1), is_causal=True)
    assert torch.allclose(a, b, atol=1e-10)


@pytest.mark.parametrize("S,W,G", [(70, 64, 2), (200, 128, 1), (300, 64, 3)])
def test_sparse_prefill_rows_matches_dense_mask(S, W, G):
    g = torch.Generator().manual_seed(S + W)
    H = 2
    q = torch.randn(1, H * G, S, 16, generator=g).to(torch.bfloat16)
    k = torch.randn(1, H, S, 16, generator=g).to(torch.bfloat16)
    v = torch.randn(1, H, S, 16, generator=g).to(torch.bfloat16)
    gm = (torch.rand(1, H, S, generator=g) < 0.2)
    rows = [0, 1, 63, 64, S // 2, S - 1]
    a = attention.sparse_prefill_rows(q, k, v, gm, W, rows)
    full = attention.masked_prefill(q, k, v, meta.ideal_mask(gm.numpy(), W, G))
    assert torch.allclose(a, full[:, :, rows], atol=1e-12)
