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


# ---- against the reference's own snapkv_evict (tests/golden/snapkv_golden.*) ----
import json  # noqa: E402
import os  # noqa: E402
import types  # noqa: E402

import numpy as np  # noqa: E402
import pytest  # noqa: E402

import scenarios  # noqa: E402

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def snapkv_gold():
    with open(os.path.join(GOLD, "snapkv_golden.json")) as f:
        meta = json.load(f)
    return np.load(os.path.join(GOLD, "snapkv_golden.npz")), meta


def golden_heads(z, name):
    """{(l, h): (pooled scores (n,) f64, dropped positions (sorted list))} in call order."""
    heads = [tuple(int(x) for x in r) for r in z[f"{name}.heads"]]
    out, at_s, at_e = {}, 0, 0
    sc = scenarios.SNAPKV_SCENARIOS[name]
    for l, h in heads:
        n = sc["lengths"][l][h]
        ne = int(n * sc["ratio"])
        out[(l, h)] = (torch.from_numpy(z[f"{name}.scores"][at_s:at_s + n]).double(),
                       [int(x) for x in z[f"{name}.evicted"][at_e:at_e + ne]])
        at_s += n
        at_e += ne
    return out


def assert_tie_equivalent(scores_ref, dropped_ref, dropped, rel_tol=0.0, label="", slack=None):
    """``dropped`` is a valid choice for the reference's scores: the same
    count, every position scoring below the reference's cut (its largest
    dropped score) dropped, none above it -- up to rel_tol of the cut plus,
    with ``slack`` (absolute, per position), the slack of the position and
    of the cut's position."""
    assert len(dropped) == len(dropped_ref), label
    if not dropped_ref:
        return
    ci = dropped_ref[int(torch.argmax(scores_ref[dropped_ref]))]
    cut = float(scores_ref[ci])
    tol = torch.full_like(scores_ref, rel_tol * abs(cut))
    if slack is not None:
        tol = tol + slack + float(slack[ci])
    d = set(dropped)
    below = set(torch.nonzero(scores_ref < cut - tol).flatten().tolist())
    above = set(torch.nonzero(scores_ref > cut + tol).flatten().tolist())
    assert below <= d, (label, sorted(below - d)[:10])
    assert not (above & d), (label, sorted(above & d)[:10])


def bf16_logit_slack(qw, keys, scale, kernel_size):
    """Per key position (n,): how far (absolute) a pooled score computed with
    bf16 logits may move when the logit sums are accumulated in another
    float32 order.  A logit sum q.k (float64) within 2**-20 * sum |q_d k_d|
    of a bf16 rounding boundary (16 float32 ulps of the magnitude, beyond
    any float32 accumulation error of D <= 128 terms) may round to the
    other bf16 neighbour; that moves the logit x by at most two bf16 steps
    of x, its probability p by p * dx and the row's softmax normaliser by
    the sum of those moves, which moves every probability of the row by that
    relative amount (to first order, each doubled here).  A key's score (a
    mean over the window of the max over the group) moves by at most the
    window mean of the max over the group of its probabilities' moves, and a
    pooled score by the largest move in its pooling window.  qw (G, win, D),
    keys (n, D); zero where no logit of the head is near a boundary."""
    from oracle import gate as ogate
    G, win, D = qw.shape
    q, k = qw.double().reshape(-1, D), keys.double()
    acc = q @ k.T
    mag = q.abs() @ k.abs().T
    _, e = torch.frexp(acc)
    dist = ogate.bf16_midpoint_distance(acc) * torch.ldexp(torch.ones_like(acc), e - 24)
    amb = dist < mag * 2.0 ** -20
    x = snapkv.logits(qw.float(), keys.float(), scale, True).double().reshape(-1, k.shape[0])
    p = torch.softmax(x, dim=-1)
    _, ex = torch.frexp(x)
    dx = 2.0 * torch.ldexp(torch.ones_like(x), ex - 8)
    own = torch.where(amb, 2.0 * p * dx, torch.zeros_like(p))       # the flipped entries themselves
    norm = 2.0 * own.sum(-1, keepdim=True)                           # relative move of each row's normaliser
    move = (own + p * norm).view(G, win, -1)
    slack = move.amax(0).sum(0) / win
    r = kernel_size // 2
    if r:
        slack = torch.nn.functional.max_pool1d(slack.view(1, 1, -1), 2 * r + 1, 1, r).view(-1)
    return slack


def oracle_cache(st, sc):
    P = 16
    return types.SimpleNamespace(
        P=P, D=sc["D"], L=sc["L"], H=sc["H"], local_blocks_per_head=sc["W"] // P,
        block_pool_k=st["pool_k"].float().clone(), block_pool_v=st["pool_v"].float().clone(),
        block_table=st["block_table"].clone(), global_lengths=st["global_lengths"].clone(),
        free_block_ids=list(st["free_ids"]), total_blocks=st["total_blocks"])


def oracle_window(st, sc):
    return types.SimpleNamespace(buf=st["qbuf"].float(), window=sc["win"])


def kept_checksum(c, sc):
    lb = sc["W"] // 16
    dt = torch.bfloat16 if sc["dtype"] == "bf16" else torch.float32
    kk = scenarios.logical_tokens(c.block_pool_k.to(dt), c.block_table, c.global_lengths, lb)
    vv = scenarios.logical_tokens(c.block_pool_v.to(dt), c.block_table, c.global_lengths, lb)
    return scenarios.checksum(*[kk[k] for k in sorted(kk)], *[vv[k] for k in sorted(vv)])


@pytest.mark.parametrize("name", list(scenarios.SNAPKV_SCENARIOS))
def test_oracle_matches_reference_snapkv(name):
    z, meta = snapkv_gold()
    sc = scenarios.SNAPKV_SCENARIOS[name]
    st = scenarios.snapkv_state(sc)
    assert scenarios.checksum(st["pool_k"], st["pool_v"], st["qbuf"], st["block_table"]) == meta[name]["inputs_sha256"]
    gold = golden_heads(z, name)
    bf = sc["dtype"] == "bf16"
    scale = sc["D"] ** -0.5
    # the oracle's own choice: same scores, a tie-equivalent drop set, the same tables
    c = oracle_cache(st, sc)
    dropped = snapkv.evict(c, oracle_window(st, sc), sc["G"], scale, sc["ratio"], sc["ksz"], logits_bf16=bf)
    assert sorted(dropped) == sorted(gold)
    qw_all = oracle_window(st, sc).buf
    before = oracle_cache(st, sc)
    for (l, h), (s_ref, ev_ref) in gold.items():
        n = s_ref.numel()
        keys = scenarios.logical_tokens(before.block_pool_k, before.block_table, before.global_lengths,
                                        sc["W"] // 16)[(l, h)]
        qw = qw_all[l].view(sc["win"], sc["H"], sc["G"], sc["D"]).permute(1, 2, 0, 3)[h]
        s = snapkv.head_scores(qw, keys, scale, sc["ksz"], logits_bf16=bf).double()
        assert s.numel() == n
        assert torch.allclose(s, s_ref, rtol=1e-6, atol=0), (name, l, h, (s - s_ref).abs().max().item())
        assert_tie_equivalent(s_ref, ev_ref, dropped[(l, h)], 1e-6, f"{name} {l} {h}")
    assert np.array_equal(c.global_lengths.numpy(), z[f"{name}.global_lengths"])
    assert np.array_equal(c.block_table.numpy(), z[f"{name}.block_table"])
    assert c.free_block_ids == z[f"{name}.free_ids"].tolist()
    # replaying the reference's own choice among equal scores gives its kept contents exactly
    c2 = oracle_cache(st, sc)
    snapkv.evict(c2, oracle_window(st, sc), sc["G"], scale, sc["ratio"], sc["ksz"], logits_bf16=bf,
                 choose=lambda l, h, s, ne: gold[(l, h)][1])
    assert kept_checksum(c2, sc) == meta[name]["kept_sha256"]
