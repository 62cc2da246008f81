"""QUEST page selection on the CPU (test infrastructure only -- see
``oracle/__init__.py``).

Restates quest_select_blocks (src/modeling_layers.py:452-576) over an
``oracle.dualcache`` (or any object with the same block_table /
global_lengths / block_pool_k / P attributes), with the page key bounds
recomputed from the logical cache: for page p of a head, the elementwise
min / max over its valid key rows -- what the reference writes at prefill
(:1333-1347) and accumulates at promotion (:744-761).

Scores are float64, or (``scores_bf16``) rounded as the reference's bf16
torch ops round them: each product q_d * bound_d to bf16, the sum to bf16.
Differences kept on purpose, as in the GPU kernels: equal scores at the cut
keep the lowest page index (the reference's topk leaves their order
unspecified); kept full pages are listed in page order (the reference lists
them in score order -- attention does not depend on it).

Pinned by the reference's own selections (tests/golden/quest_golden.npz,
written by its quest_select_blocks in bf16 and fp32: page scores, chosen
pages, lengths, tables) and, in tests/test_oracle_quest.py, by the QUEST
bound property (a page's score bounds q.k for every key in it), the budget
limits (a budget covering every token selects every page; a budget within
the local window selects no global page), a planted page that must win, and
the partial page's place.
"""
import torch


def page_bounds(cache, layer, head):
    """(kmin, kmax) float32 (pages, D) of the head's logical global pages."""
    P = cache.P if hasattr(cache, "P") else cache.block_size
    lb = cache.local_blocks_per_head if hasattr(cache, "local_blocks_per_head") else cache.local_window_size // P
    n = int(cache.global_lengths[layer, head])
    pages = (n + P - 1) // P
    ids = cache.block_table[layer, head, lb:lb + pages].long()
    D = cache.block_pool_k.shape[1]
    rows = cache.block_pool_k.view(-1, P, D)[ids].float()  # (pages, P, D)
    valid = (torch.arange(pages * P).view(pages, P) < n)[:, :, None]
    kmin = torch.where(valid, rows, torch.full_like(rows, float("inf"))).amin(dim=1)
    kmax = torch.where(valid, rows, torch.full_like(rows, float("-inf"))).amax(dim=1)
    return kmin, kmax


def page_scores(q_group, kmin, kmax, scores_bf16=False):
    """max over the group's query heads of sum_d q_d * (q_d >= 0 ? max_d : min_d)."""
    q = q_group.double()[:, None, :]                       # (G, 1, D)
    sel = torch.where(q >= 0, kmax.double()[None], kmin.double()[None])
    if scores_bf16:
        prod = (q * sel).to(torch.bfloat16).double()
        return prod.sum(-1).to(torch.bfloat16).double().amax(dim=0)
    return (q * sel).sum(-1).amax(dim=0)                   # (pages,)


def select(cache, layer, q, local_tokens, budget, num_kv_groups, scores_bf16=False):
    """q (Hq, D).  Returns (seqlens list[int] (H), blocks list[list[int]] (H))."""
    P = cache.P if hasattr(cache, "P") else cache.block_size
    lb = cache.local_blocks_per_head if hasattr(cache, "local_blocks_per_head") else cache.local_window_size // P
    H = cache.global_lengths.shape[1]
    G = num_kv_groups
    local_blocks = (local_tokens + P - 1) // P
    budget_blocks = (max(budget - local_tokens, 0) + P - 1) // P
    seqlens, blocks = [], []
    for h in range(H):
        bt = cache.block_table[layer, h]
        n = int(cache.global_lengths[layer, h])
        full, rem = divmod(n, P)
        gblocks = full + (1 if rem else 0)
        capacity = min(budget_blocks, gblocks)
        k = capacity - (1 if rem else 0)
        sel = []
        if k > 0:
            if k >= full:
                sel = list(range(full))
            else:
                kmin, kmax = page_bounds(cache, layer, h)
                s = page_scores(q[h * G:(h + 1) * G], kmin[:full], kmax[:full], scores_bf16)
                order = sorted(range(full), key=lambda p: (-float(s[p]), p))
                sel = sorted(order[:k])
        ids = [int(bt[i]) for i in range(local_blocks)] + [int(bt[lb + p]) for p in sel]
        if capacity > 0 and rem:
            ids.append(int(bt[lb + full]))
        blocks.append(ids)
        seqlens.append(local_tokens + len(sel) * P + (rem if capacity > 0 and rem else 0))
    return seqlens, blocks
