"""Sparse-prefill metadata oracle (numpy, integer arithmetic).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restates the vertical-slash index builder of the reference:

* band blocks  ``block_count`` / ``block_offset``  -- src/modeling_layers.py:321-349
* admitted columns ``column_count`` / ``column_index`` -- src/modeling_layers.py:352-381
* brute force  ``generate_sparse_indices_ref``     -- src/modeling_layers.py:274-318
* mask rebuilt from metadata                        -- utils/test_sparse_attn.py:35-58
* ideal mask causal & (admitted | band)             -- utils/test_sparse_attn.py:78-88

Shapes follow the reference: ``block_count (1,1,R)``, ``block_offset
(1,1,R,P+1)``, ``column_count (B,Hkv,R)``, ``column_index (B,Hkv,1,N)`` with
``R = ceil(S/bs)`` and ``P = min(W//bs, R)``.  Only the valid prefixes
(``block_offset[..., :block_count]``, ``column_index[..., :column_count]``)
are part of the contract (utils/test_sparse_indices.py:30-48).
"""
import numpy as np


def num_row_blocks(seq_len, bs=64):
    return (seq_len + bs - 1) // bs


def band_blocks(local_window_size, seq_len, bs=64):
    """Fast band builder, src/modeling_layers.py:321-349.

    Rows ``r < P`` (prologue) see blocks starting at 0, bs, ..., r*bs; later
    rows see ``P+1`` blocks starting at ``1 + (r-P+c)*bs`` -- i.e. at exactly
    ``r*bs - W + 1`` when ``W == P*bs``.  The count of the last row is
    recomputed from the true range (:342-347).
    """
    R = num_row_blocks(seq_len, bs)
    P = min(local_window_size // bs, R)
    block_count = np.zeros((1, 1, R), dtype=np.int32)
    block_offset = np.zeros((1, 1, R, P + 1), dtype=np.int32)
    block_count[0, 0, :P] = np.arange(1, P + 1)
    block_count[0, 0, P:] = P + 1
    for r in range(P):
        block_offset[0, 0, r, :P] = np.arange(P) * bs
    rows = np.arange(R - P)[:, None]
    cols = np.arange(P + 1)[None, :]
    block_offset[0, 0, P:] = 1 + (rows + cols) * bs
    start_last = (R - 1) * bs
    first = max(0, start_last - local_window_size + 1)
    block_count[0, 0, -1] = len(range(first, seq_len, bs))
    return block_count, block_offset


def admitted_columns(g_mask, local_window_size, bs=64):
    """Fast column builder, src/modeling_layers.py:352-381.

    ``column_count[b,h,r]`` = number of admitted positions ``< r*bs - W + 1``
    (0 for prologue rows).  The reference gets it from per-block sums whose
    blocks start at position 1 (position 0 is its own first block), then a
    cumulative sum (:364-373).  ``column_index[b,h,0,:]`` lists all admitted
    positions ascending (the ``torch.nonzero`` order, :376-379), cut to the
    largest per-head count below ``1 + bs*((S-1)//bs)`` (:369, :378): later
    positions lie in every row's band, so they are never needed as columns.
    """
    g_mask = np.asarray(g_mask, dtype=bool)
    B, H, S = g_mask.shape
    R = num_row_blocks(S, bs)
    P = min(local_window_size // bs, R)
    n_chunks = (S - 1) // bs
    trimmed = g_mask[:, :, 1:1 + n_chunks * bs].reshape(B, H, n_chunks, bs).sum(axis=3)
    sums = np.concatenate([g_mask[:, :, :1].astype(np.int64), trimmed], axis=2)
    cum = np.cumsum(sums, axis=2)
    max_global = int(cum[:, :, -1].max()) if cum.size else 0
    column_count = np.zeros((B, H, R), dtype=np.int32)
    column_count[:, :, P:] = cum[:, :, :R - P]
    column_index = np.zeros((B, H, 1, max_global), dtype=np.int32)
    for b in range(B):
        for h in range(H):
            idx = np.nonzero(g_mask[b, h])[0][:max_global]
            column_index[b, h, 0, :len(idx)] = idx
    return column_count, column_index


def generate_sparse_indices(g_mask, local_window_size, bs=64):
    """src/modeling_layers.py:384-409 (``W % bs == 0`` is required, :394)."""
    if local_window_size % bs != 0:
        raise AssertionError("local_window_size must be a multiple of the block size")
    S = np.asarray(g_mask).shape[2]
    block_count, block_offset = band_blocks(local_window_size, S, bs)
    column_count, column_index = admitted_columns(g_mask, local_window_size, bs)
    return block_count, block_offset, column_count, column_index


def sparse_indices_bruteforce(g_mask, local_window_size, bs_m=64, bs_n=64):
    """Brute-force builder, src/modeling_layers.py:274-318.

    For each row block ``i``: band blocks start at every ``bs_n`` step of
    ``[max(0, i*bs_m - W + 1), min(i*bs_m + bs_m, S))``; the admitted
    columns counted are those strictly below that start.
    """
    g_mask = np.asarray(g_mask, dtype=bool)
    B, H, S = g_mask.shape
    R = (S + bs_m - 1) // bs_m
    width = (local_window_size + bs_m - 1 + bs_n - 1) // bs_n
    max_global = int(g_mask.sum(axis=2).max()) if g_mask.size else 0
    block_count = np.zeros((1, 1, R), dtype=np.int32)
    block_offset = np.zeros((1, 1, R, width), dtype=np.int32)
    column_count = np.zeros((B, H, R), dtype=np.int32)
    column_index = np.zeros((B, H, 1, max_global), dtype=np.int32)
    for i in range(R):
        start_row = i * bs_m
        lo = max(0, start_row - local_window_size + 1)
        hi = min(start_row + bs_m, S)
        offs = list(range(lo, hi, bs_n))
        block_count[0, 0, i] = len(offs)
        block_offset[0, 0, i, :len(offs)] = offs
    for b in range(B):
        for h in range(H):
            idx = [p for p in range(S) if g_mask[b, h, p]]
            column_index[b, h, 0, :len(idx)] = idx
            for i in range(R):
                lo = max(0, i * bs_m - local_window_size + 1)
                column_count[b, h, i] = sum(1 for p in idx if p < lo)
    return block_count, block_offset, column_count, column_index


def mask_from_metadata(block_count, block_offset, column_count, column_index,
                       num_kv_groups, seq_len, bs=64):
    """Dense boolean mask implied by the metadata, causal applied.

    utils/test_sparse_attn.py:35-58: rows of block ``i`` see every column of
    each listed band block (clipped to ``S``) and every listed admitted column;
    then ``& tril``.  Returned per query head: ``(B, Hq, S, S)``.
    """
    B, H, R = column_count.shape
    Hq = H * num_kv_groups
    mask = np.zeros((B, Hq, seq_len, seq_len), dtype=bool)
    for b in range(B):
        for hq in range(Hq):
            h = hq // num_kv_groups
            for i in range(R):
                r0, r1 = i * bs, min(i * bs + bs, seq_len)
                for off in block_offset[0, 0, i, :block_count[0, 0, i]]:
                    mask[b, hq, r0:r1, off:min(off + bs, seq_len)] = True
                cc = column_count[b, h, i]
                if cc > 0:
                    mask[b, hq, r0:r1, column_index[b, h, 0, :cc]] = True
    return mask & np.tril(np.ones((seq_len, seq_len), dtype=bool))


def ideal_mask(g_mask, local_window_size, num_kv_groups, bs=64):
    """utils/test_sparse_attn.py:78-88: causal & (admitted | band).

    The band of row block ``i`` is ``[i*bs - W + 1, end_row)`` -- block
    granular, so a row can see up to ``W + bs - 1`` tokens back.
    """
    g_mask = np.asarray(g_mask, dtype=bool)
    B, H, S = g_mask.shape
    m = np.repeat(np.broadcast_to(g_mask[:, :, None, :], (B, H, S, S)), num_kv_groups, axis=1).copy()
    R = num_row_blocks(S, bs)
    for i in range(R):
        r0, r1 = i * bs, min(i * bs + bs, S)
        c0 = max(0, r0 - local_window_size + 1)
        m[:, :, r0:r1, c0:r1] = True
    return m & np.tril(np.ones((S, S), dtype=bool))
