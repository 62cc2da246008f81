"""Pinning of the QUEST oracle (oracle/quest.py) by properties that do not
restate its formula: the score bounds every q.k in the page, budgets at the
extremes, a planted page, and the partial page's place."""
import torch

from oracle import quest
from oracle.dualcache import DualCacheOracle


def filled_cache(L=1, H=2, D=32, W=32, S=700, seed=0, frac=0.5):
    g = torch.Generator().manual_seed(seed)
    c = DualCacheOracle(L, H, D, W, H * (S + W), S + W, block_size=16)
    k = torch.randn(H, S, D, generator=g)
    v = torch.randn(H, S, D, generator=g)
    m = torch.rand(H, S, generator=g) < frac
    c.prefill(0, k, v, m)
    return c, g


def test_score_bounds_every_key_of_the_page():
    c, g = filled_cache()
    for h in range(2):
        kmin, kmax = quest.page_bounds(c, 0, h)
        n = int(c.global_lengths[0, h])
        ids = c.block_table[0, h, 2:2 + kmin.shape[0]].long()
        rows = c.block_pool_k.view(-1, 16, 32)[ids].reshape(-1, 32)[:n].double()
        for _ in range(5):
            q = torch.randn(1, 32, generator=g)
            s = quest.page_scores(q, kmin, kmax)
            dots = rows @ q[0].double()
            for p in range(kmin.shape[0]):
                assert dots[p * 16:(p + 1) * 16].max() <= s[p] + 1e-9


def test_budget_extremes_and_partial_page():
    c, g = filled_cache()
    q = torch.randn(4, 32, generator=g)
    n = [int(x) for x in c.global_lengths[0]]
    # a budget covering every token selects every page, in order
    sl, bl = quest.select(c, 0, q, 20, 10 ** 6, 2)
    for h in range(2):
        pages = (n[h] + 15) // 16
        assert sl[h] == 20 + n[h]
        assert bl[h] == [int(x) for x in c.block_table[0, h, :2]] + [int(x) for x in c.block_table[0, h, 2:2 + pages]]
    # a budget inside the local window selects no global page
    sl, bl = quest.select(c, 0, q, 20, 16, 2)
    assert sl == [20, 20] and all(len(b) == 2 for b in bl)
    # a tight budget keeps the partial page last and counts only its valid rows
    sl, bl = quest.select(c, 0, q, 20, 20 + 5 * 16, 2)
    for h in range(2):
        rem = n[h] % 16
        if rem:
            assert bl[h][-1] == int(c.block_table[0, h, 2 + n[h] // 16])
            assert sl[h] == 20 + 4 * 16 + rem
        else:
            assert sl[h] == 20 + 5 * 16


def test_planted_page_is_selected():
    c, g = filled_cache(S=900)
    q = torch.randn(4, 32, generator=g)
    h, p = 1, 7
    row0 = int(c.block_table[0, h, 2 + p]) * 16
    c.block_pool_k[row0 + 3] = 50.0 * q[h * 2 + 1]  # one key aligned with a query of head 1
    sl, bl = quest.select(c, 0, q, 32, 32 + 3 * 16, 2)
    assert int(c.block_table[0, h, 2 + p]) in bl[h]
