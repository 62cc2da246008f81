"""Attention oracles (torch on the CPU, float32 / float64).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

* ``paged_decode``   -- per (sequence, KV head) gather of the paged cache and
  a dense softmax, restating ``flash_attn_with_kvcache_ref`` of
  utils/test_flash_attn_with_kvcache.py:16-71 (the semantics of the
  reference's decode kernels, src/modeling_layers.py:834-1000, and of its
  ``decode_kernel_handle`` contract, :1439-1447).  Computed in float32 (or
  float64) from the bf16 inputs: the fp32 result the build is compared with.
* ``paged_decode_loop`` -- the same definition written as a scalar float64
  loop over tokens; used only to pin ``paged_decode``.
* ``masked_prefill`` -- SDPA under an explicit boolean mask, GQA by
  ``h_kv = h_q // G`` (utils/test_sparse_attn.py:60-66, :51).
"""
import math

import torch


def _gather_head(k_cache, v_cache, block_table_row, seqlen):
    page = k_cache.shape[1]
    n_pages = (seqlen + page - 1) // page
    ids = block_table_row[:n_pages].long()
    k = k_cache[ids].reshape(-1, k_cache.shape[2])[:seqlen]
    v = v_cache[ids].reshape(-1, v_cache.shape[2])[:seqlen]
    return k, v


def paged_decode(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale,
                 dtype=torch.float32):
    """Reference paged decode.

    q (B,1,Hq,D); k_cache/v_cache (NB,page,D); cache_seqlens (B,Hkv) int32;
    block_table (B,Hkv,maxB) int32 -> (B,1,Hq,D) in ``dtype``.  A head with
    ``seqlen == 0`` yields zeros, as the reference reduce kernel does
    (src/modeling_layers.py:998-999).
    """
    B, _, Hq, D = q.shape
    Hkv = cache_seqlens.shape[1]
    G = Hq // Hkv
    out = torch.zeros(B, 1, Hq, D, dtype=dtype)
    for b in range(B):
        for h in range(Hkv):
            T = int(cache_seqlens[b, h])
            if T == 0:
                continue
            k, v = _gather_head(k_cache, v_cache, block_table[b, h], T)
            k = k.to(dtype)
            v = v.to(dtype)
            qh = q[b, 0, h * G:(h + 1) * G].to(dtype)
            s = (qh @ k.T) * softmax_scale
            p = torch.softmax(s, dim=-1)
            out[b, 0, h * G:(h + 1) * G] = p @ v
    return out


def paged_decode_loop(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale):
    """Scalar float64 restatement of the same definition (tiny inputs only)."""
    B, _, Hq, D = q.shape
    Hkv = cache_seqlens.shape[1]
    G = Hq // Hkv
    page = k_cache.shape[1]
    qd = q.double().tolist()
    kd = k_cache.double()
    vd = v_cache.double()
    out = torch.zeros(B, 1, Hq, D, dtype=torch.float64)
    for b in range(B):
        for hq in range(Hq):
            h = hq // G
            T = int(cache_seqlens[b, h])
            if T == 0:
                continue
            logits = []
            rows = []
            for t in range(T):
                pid = int(block_table[b, h, t // page])
                krow = kd[pid, t % page].tolist()
                rows.append(vd[pid, t % page])
                logits.append(sum(a * c for a, c in zip(qd[b][0][hq], krow)) * softmax_scale)
            m = max(logits)
            w = [math.exp(x - m) for x in logits]
            z = sum(w)
            acc = torch.zeros(D, dtype=torch.float64)
            for wi, r in zip(w, rows):
                acc += (wi / z) * r
            out[b, 0, hq] = acc
    return out


def masked_prefill(q, k, v, mask, softmax_scale=None, dtype=torch.float64):
    """SDPA under ``mask`` with GQA.

    q (B,Hq,S,D), k/v (B,Hkv,S,D), mask (B,Hq,S,S) bool -> (B,Hq,S,D).
    Rows whose mask is empty cannot occur under a causal band (the diagonal is
    always visible, utils/test_sparse_attn.py:78-88).
    """
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    kk = k.to(dtype).repeat_interleave(G, dim=1)
    vv = v.to(dtype).repeat_interleave(G, dim=1)
    s = torch.matmul(q.to(dtype), kk.transpose(-1, -2).contiguous()) * softmax_scale
    s = s.masked_fill(~torch.as_tensor(mask), float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vv)


def masked_prefill_rowloop(q, k, v, mask, softmax_scale=None):
    """Row-by-row float64 restatement of ``masked_prefill`` (tiny inputs)."""
    B, Hq, S, D = q.shape
    G = Hq // k.shape[1]
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    out = torch.zeros(B, Hq, S, D, dtype=torch.float64)
    for b in range(B):
        for hq in range(Hq):
            kk = k[b, hq // G].double()
            vv = v[b, hq // G].double()
            for i in range(S):
                cols = torch.nonzero(torch.as_tensor(mask[b, hq, i])).flatten()
                s = (kk[cols] @ q[b, hq, i].double()) * softmax_scale
                p = torch.exp(s - s.max())
                out[b, hq, i] = (p / p.sum()) @ vv[cols]
    return out


def sparse_prefill_rows(q, k, v, g_mask, local_window_size, rows, softmax_scale=None, bs=64):
    """Selected query rows of the sparse prefill, straight from the ideal mask
    of utils/test_sparse_attn.py:78-88: row i of block r = i // bs sees keys
    j <= i with g_mask[j] or j >= r*bs - W + 1.  q (B,Hq,S,D), k/v (B,Hkv,S,D),
    g_mask (B,Hkv,S) bool; returns (B, Hq, len(rows), D) float64."""
    B, Hq, S, D = q.shape
    G = Hq // k.shape[1]
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    gm = torch.as_tensor(g_mask)
    out = torch.zeros(B, Hq, len(rows), D, dtype=torch.float64)
    for ri, i in enumerate(rows):
        start = max(0, (i // bs) * bs - local_window_size + 1)
        for b in range(B):
            for hq in range(Hq):
                h = hq // G
                vis = gm[b, h, :i + 1].clone()
                vis[start:i + 1] = True
                cols = torch.nonzero(vis).flatten()
                s = (k[b, h, cols].double() @ q[b, hq, i].double()) * softmax_scale
                p = torch.softmax(s, dim=0)
                out[b, hq, ri] = p @ v[b, h, cols].double()
    return out
