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


# ---- against the reference's own quest_select_blocks (tests/golden/quest_golden.*) ----
import json  # noqa: E402
import os  # noqa: E402
import types  # noqa: E402

import numpy as np  # noqa: E402
import pytest  # noqa: E402

import scenarios  # noqa: E402

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def quest_gold():
    with open(os.path.join(GOLD, "quest_golden.json")) as f:
        meta = json.load(f)
    return np.load(os.path.join(GOLD, "quest_golden.npz")), meta


def ranked_heads(sc, local, budget):
    """Heads whose full pages the reference ranks with topk at this step
    (0 < full capacity < full pages), with (full pages, capacity)."""
    P = 16
    out = []
    budget_blocks = (max(budget - local, 0) + P - 1) // P
    for h, n in enumerate(sc["lengths"]):
        full, rem = divmod(n, P)
        cap = min(budget_blocks, full + (1 if rem else 0))
        k = cap - (1 if rem else 0)
        if 0 < k < full:
            out.append((h, full, k))
    return out


def golden_rankings(z, name, i, sc, local, budget):
    """{head: (page scores (full,) f64, chosen page positions)} of step i."""
    sc_all = z[f"{name}.{i}.ranked_scores"]
    ch_all = z[f"{name}.{i}.ranked_choice"]
    out, a, b = {}, 0, 0
    for h, full, k in ranked_heads(sc, local, budget):
        out[h] = (torch.from_numpy(sc_all[a:a + full]).double(), sorted(int(x) for x in ch_all[b:b + k]))
        a += full
        b += k
    assert a == sc_all.shape[0] and b == ch_all.shape[0]
    return out


def assert_same_choice_up_to_ties(scores, chosen_ref, chosen, tol, label=""):
    """``chosen`` is a valid top-k for the reference's scores: the same count,
    every page scoring above the reference's cut (its smallest chosen score)
    chosen and none below it, up to ``tol``."""
    assert len(chosen) == len(chosen_ref), label
    cut = float(scores[chosen_ref].min())
    c = set(chosen)
    above = set(torch.nonzero(scores > cut + tol).flatten().tolist())
    below = set(torch.nonzero(scores < cut - tol).flatten().tolist())
    assert above <= c, (label, sorted(above - c))
    assert not (below & c), (label, sorted(below & c))


def bf16_step(x):
    _, e = torch.frexp(torch.tensor(float(x), dtype=torch.float64))
    return float(torch.ldexp(torch.tensor(1.0, dtype=torch.float64), e - 8))


def check_selection_against_golden(z, name, i, sc, st, sel_len, sel_rows, scores_of_head=None):
    """sel_len (H,) ints and sel_rows (H lists of page ids, local pages first,
    kept full pages, partial page last) against step i of the golden."""
    local, budget = sc["steps"][i]
    P, lb = 16, sc["W"] // 16
    g_len = z[f"{name}.{i}.seqlens"][0].tolist()
    g_bt = z[f"{name}.{i}.block_table"][0]
    assert list(sel_len) == g_len, (name, i)
    rank = golden_rankings(z, name, i, sc, local, budget)
    local_blocks = (local + P - 1) // P
    for h, n in enumerate(sc["lengths"]):
        table = st["block_table"][0, h]
        full, rem = divmod(n, P)
        row = sel_rows[h]
        ref_row = [int(x) for x in g_bt[h][:len(row)]]
        assert row[:local_blocks] == ref_row[:local_blocks], (name, i, h)
        budget_blocks = (max(budget - local, 0) + P - 1) // P
        cap = min(budget_blocks, full + (1 if rem else 0))
        if cap > 0 and rem:
            assert row[-1] == ref_row[-1] == int(table[lb + full]), (name, i, h)  # the partial page, last
        ours = set(row[local_blocks:len(row) - (1 if cap > 0 and rem else 0)])
        refs = set(ref_row[local_blocks:len(ref_row) - (1 if cap > 0 and rem else 0)])
        if h not in rank:
            assert ours == refs, (name, i, h)
            continue
        s_ref, ch_ref = rank[h]
        pos = {int(table[lb + p]): p for p in range(full)}
        chosen = sorted(pos[pg] for pg in ours)
        assert sorted(pos[pg] for pg in refs) == ch_ref
        cut = float(s_ref[ch_ref].min())
        tol = bf16_step(cut) if sc["dtype"] == "bf16" else 1e-5 * abs(cut)
        assert_same_choice_up_to_ties(s_ref, ch_ref, chosen, tol, f"{name} step {i} head {h}")
        if scores_of_head is not None:
            s = scores_of_head(h, full)
            assert torch.allclose(s, s_ref, rtol=0, atol=tol), (name, i, h)


@pytest.mark.parametrize("name", list(scenarios.QUEST_SCENARIOS))
def test_oracle_matches_reference_quest(name):
    z, meta = quest_gold()
    sc = scenarios.QUEST_SCENARIOS[name]
    st = scenarios.quest_state(sc)
    assert scenarios.checksum(st["pool_k"], st["key_min"], st["key_max"], st["block_table"], *st["qs"]) == \
        meta[name]["inputs_sha256"]
    cache = types.SimpleNamespace(block_table=st["block_table"], global_lengths=st["global_lengths"],
                                  block_pool_k=st["pool_k"].float(), block_size=16, local_window_size=sc["W"])
    bf = sc["dtype"] == "bf16"
    G = sc["G"]
    for i, (local, budget) in enumerate(sc["steps"]):
        q = st["qs"][i].float()
        lens, blocks = quest.select(cache, 0, q, local, budget, G, scores_bf16=bf)

        def scores_of_head(h, full):
            kmin, kmax = quest.page_bounds(cache, 0, h)
            return quest.page_scores(q[h * G:(h + 1) * G], kmin[:full], kmax[:full], bf)

        check_selection_against_golden(z, name, i, sc, st, lens, blocks, scores_of_head)
