"""Synthetic decode workloads at the shapes the benchmarks are quoted on.

* ``decode_beta``   -- batch B, per-KV-head admitted count
  ``round(f * (ctx - W))`` with ``f ~ Beta(2, 8)`` (mean 20 %), plus the
  full local window W; Llama-3.1-8B head shapes.
* ``decode_ragged`` -- per (sequence, head) fraction ``f ~ U[lo, hi]``
  independently, same token count rule.

The physical pages of all heads are a random permutation of the pool (as the
reference's decode benchmark does, utils/benchmark_decode.py:72-77); K/V and
q are N(0,1) bf16.  Everything is generated on ``device`` from a seeded
generator.
"""
from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class DecodeWorkload:
    q: torch.Tensor            # (B, 1, Hq, D) bf16
    k_cache: torch.Tensor      # (num_pages, page, D) bf16
    v_cache: torch.Tensor
    cache_seqlens: torch.Tensor  # (B, Hkv) int32
    block_table: torch.Tensor    # (B, Hkv, max_pages) int32, -1 past the end
    softmax_scale: float
    name: str

    @property
    def total_tokens(self):
        return int(self.cache_seqlens.sum().item())

    def algorithmic_bytes(self):
        """K+V rows read, page-table entries read, q read and out written."""
        B, _, Hq, D = self.q.shape
        page = self.k_cache.shape[1]
        sl = self.cache_seqlens.to(torch.int64)
        kv = int(sl.sum().item()) * D * 2 * 2
        table = int(((sl + page - 1) // page).sum().item()) * 4
        return kv + table + 2 * B * Hq * D * 2 + 4 * sl.numel()


def _build(seqlens, Hq, D, page, device, seed, name):
    B, Hkv = seqlens.shape
    pages = (seqlens + page - 1) // page
    total = int(pages.sum())
    max_pages = int(pages.max())
    g = torch.Generator(device="cpu").manual_seed(seed)
    perm = torch.randperm(total, generator=g).to(torch.int32)
    table = torch.full((B, Hkv, max_pages), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        for h in range(Hkv):
            n = int(pages[b, h])
            table[b, h, :n] = perm[off:off + n]
            off += n
    gd = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(total, page, D, generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn(total, page, D, generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    q = torch.randn(B, 1, Hq, D, generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    return DecodeWorkload(q, k, v, torch.as_tensor(seqlens, dtype=torch.int32).to(device),
                          table.to(device), D ** -0.5, name)


def decode_beta(ctx=32768, batch=1, Hq=32, Hkv=8, D=128, window=1024, page=16, device="cuda", seed=0):
    rng = np.random.default_rng(seed)
    f = rng.beta(2.0, 8.0, size=(batch, Hkv))
    seqlens = window + np.rint(f * (ctx - window)).astype(np.int64)
    return _build(seqlens, Hq, D, page, device, seed, f"decode_beta_b{batch}_{ctx // 1024}k")


def decode_ragged(ctx=131072, batch=8, Hq=32, Hkv=8, D=128, window=1024, page=16,
                  lo=0.02, hi=0.60, device="cuda", seed=0):
    rng = np.random.default_rng(seed)
    f = rng.uniform(lo, hi, size=(batch, Hkv))
    seqlens = window + np.rint(f * (ctx - window)).astype(np.int64)
    return _build(seqlens, Hq, D, page, device, seed, f"decode_ragged_b{batch}_{ctx // 1024}k")
