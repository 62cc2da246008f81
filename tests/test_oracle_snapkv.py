"""Pinning of the SnapKV oracle by properties (no restatement of its formula):
dropped count and order preservation, the dropped scores are the lowest,
ratio 1 releases every page, a planted key every query attends to is kept,
and promotion reuses released pages from the end of the list."""
import torch

from oracle import snapkv
from oracle.dualcache import DualCacheOracle


def global_keys(c, l, h):
    n = int(c.global_lengths[l, h])
    ids = c.block_table[l, h, 2:2 + (n + 15) // 16].long()
    return c.block_pool_k.view(-1, 16, c.D)[ids].reshape(-1, c.D)[:n]


def setup(L=2, H=2, G=2, D=32, W=32, S=600, seed=0):
    g = torch.Generator().manual_seed(seed)
    c = DualCacheOracle(L, H, D, W, L * H * (S + 200), S + 200, block_size=16)
    for l in range(L):
        c.prefill(l, torch.randn(H, S, D, generator=g), torch.randn(H, S, D, generator=g),
                  torch.rand(H, S, generator=g) < 0.5)
    w = snapkv.QueryWindow(L, 16, H * G, D)
    for l in range(L):
        w.record(l, torch.randn(H * G, S, D, generator=g))
    return c, w, g


def test_counts_order_and_lowest_scores():
    c, w, g = setup()
    before = {(l, h): global_keys(c, l, h).clone() for l in range(2) for h in range(2)}
    scores = {}
    for l in range(2):
        qw = w.buf[l].view(16, 2, 2, 32).permute(1, 2, 0, 3)
        for h in range(2):
            scores[(l, h)] = snapkv.head_scores(qw[h], before[(l, h)], 32 ** -0.5, 5)
    dropped = snapkv.evict(c, w, 2, 32 ** -0.5, 0.3, 5)
    for (l, h), k_before in before.items():
        n = k_before.shape[0]
        ev = dropped[(l, h)]
        assert len(ev) == int(n * 0.3)
        kept = [i for i in range(n) if i not in set(ev)]
        k_after = global_keys(c, l, h)
        assert torch.equal(k_after, k_before[kept])            # kept tokens, in order
        s = scores[(l, h)]
        assert s[ev].max() <= s[kept].min()                     # the lowest were dropped
        assert int(c.global_lengths[l, h]) == len(kept)


def test_ratio_one_releases_all_pages_and_promotion_reuses_them():
    c, w, g = setup(L=1, H=2)
    pages_before = [(int(c.global_lengths[0, h]) + 15) // 16 for h in range(2)]
    snapkv.evict(c, w, 2, 32 ** -0.5, 1.0, 5)
    assert c.global_lengths.sum() == 0
    assert len(c.free_block_ids) == sum(pages_before)
    free = list(c.free_block_ids)
    # promote one token of every head: the new pages come from the end of the list
    c.local_length = c.W
    c.local_is_global[:, :, c.local_ptr] = True
    c.migrate()
    assert [int(c.block_table[0, h, 2]) for h in range(2)] == free[-2:]
    assert c.free_block_ids == free[:-2]


def test_planted_key_is_kept():
    c, w, g = setup(L=1, H=1, G=2, S=800)
    n = int(c.global_lengths[0, 0])
    target = 123
    page = int(c.block_table[0, 0, 2 + target // 16])
    # every window query aligned with the planted key
    w.buf[0] = w.buf[0][:1].expand_as(w.buf[0]).clone()
    c.block_pool_k[page * 16 + target % 16] = 20.0 * w.buf[0, 0, 0]
    before = global_keys(c, 0, 0).clone()
    dropped = snapkv.evict(c, w, 2, 32 ** -0.5, 0.9, 5)
    assert target not in dropped[(0, 0)]
    kept = [i for i in range(n) if i not in set(dropped[(0, 0)])]
    assert torch.equal(global_keys(c, 0, 0)[kept.index(target)], before[target])
