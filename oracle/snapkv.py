"""SnapKV eviction on the CPU (test infrastructure only -- see
``oracle/__init__.py``).

Restates snapkv_record_queries / snapkv_evict (src/modeling_layers.py:
579-671) over an ``oracle.dualcache.DualCacheOracle``: per (layer, KV head)
the global tokens are scored by the window queries' attention (softmax over
the head's global keys, max over the grouped query heads, mean over the
window, max-pooled with stride 1), the int(len * ratio) lowest are dropped,
the kept tokens are packed in order into the head's first pages, and the
released pages are appended to ``free_block_ids`` (reused first by
promotion, ``DualCacheOracle.migrate``).

The logits are fp32 products, or (``logits_bf16``) rounded as the
reference's bf16 matmul and scalar multiply round them,
bf16(bf16(q.k) * scale); equal scores are dropped lower position first (the
reference's topk leaves their order unspecified).  Pinned by the reference's
own outputs (tests/golden/snapkv_golden.npz, written by its snapkv_evict in
bf16 and in fp32: pooled scores, dropped positions, lengths, tables, free
list and kept contents) and, in tests/test_oracle_snapkv.py, by properties:
the dropped count, order preservation, every kept score >= every dropped
score, ratio 1 releasing every page, and a planted key every window query
attends to.
"""
import torch
import torch.nn.functional as F


class QueryWindow:
    """The last ``window`` queries per layer (:579-592)."""

    def __init__(self, L, window, Hq, D):
        self.buf = torch.zeros(L, window, Hq, D)
        self.length = 0
        self.ptr = 0
        self.window = window
        self.L = L

    def record(self, layer, q):
        """q (Hq, S, D) of one layer's call."""
        S = q.shape[1]
        if S > 1:
            take = min(self.window, S)
            self.buf[layer, :take] = q[:, -take:, :].transpose(0, 1).float()
            if layer == self.L - 1:
                self.length = take
                self.ptr = take % self.window
        else:
            self.buf[layer, self.ptr] = q[:, 0, :].float()
            if layer == self.L - 1:
                self.length = min(self.window, self.length + 1)
                self.ptr = (self.ptr + 1) % self.window


def logits(qw, keys, scale, logits_bf16=False):
    """(G, window, n) float32 logits q.k * scale; with logits_bf16 the product
    sum is rounded to bf16, then the scaled value (the reference's bf16
    torch.matmul(...) * self.scaling, src/modeling_layers.py:616-617)."""
    if logits_bf16:
        acc = (qw.double() @ keys.double().T).to(torch.bfloat16).float()
        return (acc * torch.tensor(scale, dtype=torch.float32)).to(torch.bfloat16).float()
    return (qw.float() @ keys.float().T) * scale


def head_scores(qw, keys, scale, kernel_size, logits_bf16=False):
    """qw (G, window, D), keys (n, D) -> pooled scores (n,) float32."""
    attn = torch.softmax(logits(qw, keys, scale, logits_bf16), dim=-1)
    s = attn.amax(dim=0).mean(dim=0).view(1, 1, -1)
    return F.max_pool1d(s, kernel_size=kernel_size, stride=1, padding=kernel_size // 2).view(-1)


def evict(cache, window, num_kv_groups, scale, ratio, kernel_size, logits_bf16=False, choose=None):
    """Evict on every (layer, head) of ``cache``; returns the dropped positions
    per (layer, head) (logical global indices before the eviction).
    ``choose(l, h, scores, n_evict)`` (optional) names the dropped positions
    instead of the lowest-score rule (to replay another implementation's
    choice among equal scores)."""
    if not hasattr(cache, "free_block_ids"):
        cache.free_block_ids = []
    P, D, lb = cache.P, cache.D, cache.local_blocks_per_head
    kc = cache.block_pool_k.view(-1, P, D)
    G = num_kv_groups
    dropped = {}
    for l in range(cache.L):
        qw = window.buf[l].view(window.window, cache.H, G, D).permute(1, 2, 0, 3)
        for h in range(cache.H):
            n = int(cache.global_lengths[l, h])
            n_evict = int(n * ratio)
            if n_evict == 0:
                continue
            pages = (n + P - 1) // P
            ids = cache.block_table[l, h, lb:lb + pages].long()
            keys = kc[ids].reshape(-1, D)[:n]
            s = head_scores(qw[h], keys, scale, kernel_size, logits_bf16)
            if choose is not None:
                ev = torch.as_tensor(choose(l, h, s, n_evict), dtype=torch.int64)
            else:
                ev = torch.sort(s, stable=True).indices[:n_evict]
            keep = torch.ones(n, dtype=torch.bool)
            keep[ev] = False
            kept_idx = torch.nonzero(keep).flatten()
            linear = (ids[:, None] * P + torch.arange(P)[None, :]).reshape(-1)[:n]
            kept = kept_idx.numel()
            if kept:
                kk = cache.block_pool_k[linear[kept_idx]].clone()
                vv = cache.block_pool_v[linear[kept_idx]].clone()
                cache.block_pool_k[linear[:kept]] = kk
                cache.block_pool_v[linear[:kept]] = vv
            new_pages = (kept + P - 1) // P
            if new_pages < pages:
                cache.free_block_ids.extend(int(x) for x in cache.block_table[l, h, lb + new_pages:lb + pages])
                cache.block_table[l, h, lb + new_pages:lb + pages] = cache.total_blocks - 1
            cache.global_lengths[l, h] = kept
            dropped[(l, h)] = sorted(int(x) for x in ev)
    return dropped
