"""Dual-cache state-machine oracle (torch CPU tensors; integer bookkeeping).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restates, for batch 1 (the reference asserts ``batch_size == 1`` in
inference, src/modeling_layers.py:1614):

* pool / page-table initialisation  -- prefill_wrapper :1196-1288
* local ring write at prefill       -- :1290-1300
* global scatter at prefill         -- :1302-1331 (bump allocation in head order)
* decode ring write + flag          -- decode_wrapper :1390-1413
* lazy promotion when the ring is full -- migrate_local_kv_to_global :674-763
  (bump allocation in row-major (layer, head) order, ``torch.nonzero``)
* deferred re-gating of a full window -- refresh_local_is_global :1169-1180
* decode metadata                    -- :1429-1436

Capacity is checked for the whole call before anything is written (the
reference asserts per head, mid-way; the condition that raises is the same).
Attribute names are the reference's, so fixtures written by the reference can
be compared attribute by attribute.
"""
import torch


class CapacityError(AssertionError):
    pass


class DualCacheOracle:
    def __init__(self, num_layers, num_kv_heads, head_dim, local_window_size,
                 max_total_tokens, max_tokens_per_head, block_size=16,
                 g_defer=False, dtype=torch.bfloat16):
        if local_window_size % block_size:
            raise AssertionError("local_window_size % block_size != 0")  # :1467
        L, H, W, P = num_layers, num_kv_heads, local_window_size, block_size
        self.L, self.H, self.D, self.W, self.P = L, H, head_dim, W, P
        self.local_blocks_per_head = W // P
        self.max_tokens_per_head = max_tokens_per_head
        self.total_blocks = (max_total_tokens + P - 1) // P
        max_blocks_per_head = (max_tokens_per_head + P - 1) // P
        self.block_table = torch.full((L, H, max_blocks_per_head), self.total_blocks - 1, dtype=torch.int32)
        n_local = L * H * self.local_blocks_per_head
        self.block_table[:, :, :self.local_blocks_per_head] = torch.arange(n_local, dtype=torch.int32).view(L, H, -1)
        self.block_pool_k = torch.zeros(self.total_blocks * P, head_dim, dtype=dtype)
        self.block_pool_v = torch.zeros(self.total_blocks * P, head_dim, dtype=dtype)
        self.local_is_global = torch.zeros(L, H, W, dtype=torch.bool)
        self.global_lengths = torch.zeros(L, H, dtype=torch.int32)
        self.local_region_starts = (torch.arange(L, dtype=torch.int32)[:, None] * H
                                    + torch.arange(H, dtype=torch.int32)[None, :]) * W
        self.local_ptr = 0
        self.local_length = 0
        self.next_free_block = n_local
        self.g_defer = g_defer
        self.local_pre_key = torch.zeros(L, H, W, head_dim, dtype=dtype) if g_defer else None

    # ---------------------------------------------------------------- prefill
    def prefill(self, layer, key, value, g_mask, pre_key=None):
        """key/value (H,S,D), g_mask (H,S) bool.  Mirrors :1290-1331."""
        H, S, _ = key.shape
        W, P = self.W, self.P
        n_loc = min(S, W)
        n_early = S - W
        counts = []
        for h in range(H):
            counts.append(int(g_mask[h, :n_early].sum()) if n_early > 0 else 0)
        nxt = self.next_free_block
        for h in range(H):
            if counts[h] == 0:
                continue
            if n_loc + counts[h] > self.max_tokens_per_head:
                raise CapacityError(f"layer {layer} head {h}: exceeds max_tokens_per_head")
            pages = (counts[h] + P - 1) // P
            if nxt + pages > self.total_blocks:
                raise CapacityError(f"layer {layer} head {h}: exceeds total_blocks")
            nxt += pages
        # 1. local ring: slot i <- token S-n_loc+i
        for h in range(H):
            base = int(self.local_region_starts[layer, h])
            self.block_pool_k[base:base + n_loc] = key[h, S - n_loc:]
            self.block_pool_v[base:base + n_loc] = value[h, S - n_loc:]
            self.local_is_global[layer, h, :n_loc] = g_mask[h, S - n_loc:]
            if self.g_defer:
                self.local_pre_key[layer, h, :n_loc] = pre_key[h, S - n_loc:]
        self.local_length = n_loc
        # 2. global: admitted tokens of [0, S-W), ascending, fresh contiguous pages
        for h in range(H):
            if counts[h] == 0:
                continue
            idx = torch.nonzero(g_mask[h, :n_early]).flatten()
            pages = (counts[h] + P - 1) // P
            first = self.next_free_block
            lb = self.local_blocks_per_head
            self.block_table[layer, h, lb:lb + pages] = torch.arange(first, first + pages, dtype=torch.int32)
            self.block_pool_k[first * P:first * P + counts[h]] = key[h, idx]
            self.block_pool_v[first * P:first * P + counts[h]] = value[h, idx]
            self.global_lengths[layer, h] = counts[h]
            self.next_free_block += pages

    # ----------------------------------------------------------------- decode
    def migrate(self):
        """Promote ring slot ``local_ptr`` of every flagged (layer, head).  :674-763."""
        W, P, lb = self.W, self.P, self.local_blocks_per_head
        slot = self.local_ptr
        items = [(l, h) for l in range(self.L) for h in range(self.H) if bool(self.local_is_global[l, h, slot])]
        if not items:
            return
        new_pages = 0
        for l, h in items:
            gl = int(self.global_lengths[l, h])
            if W + gl + 1 > self.max_tokens_per_head:
                raise CapacityError("Tokens exceed max_tokens_per_head")
            if gl % P == 0:
                new_pages += 1
        free = getattr(self, "free_block_ids", None)  # SnapKV: released pages, reused first (:694-712)
        from_free = min(new_pages, len(free)) if free is not None else 0
        if self.next_free_block + new_pages - from_free > self.total_blocks:
            raise CapacityError("Allocation exceeds total_blocks")
        reuse = free[len(free) - from_free:] if from_free else []
        if from_free:
            del free[len(free) - from_free:]
        nxt = self.next_free_block
        for l, h in items:
            gl = int(self.global_lengths[l, h])
            logical = lb + gl // P
            if gl % P == 0:
                if reuse:
                    self.block_table[l, h, logical] = reuse.pop(0)
                else:
                    self.block_table[l, h, logical] = nxt
                    nxt += 1
            src = int(self.local_region_starts[l, h]) + slot
            dst = int(self.block_table[l, h, logical]) * P + gl % P
            self.block_pool_k[dst] = self.block_pool_k[src]
            self.block_pool_v[dst] = self.block_pool_v[src]
            self.global_lengths[l, h] = gl + 1
        self.next_free_block = nxt

    def decode(self, layer, key, value, g_mask=None, pre_key=None, regate=None):
        """One token: key/value (H,D), g_mask (H,) bool or None (deferred).

        ``regate(layer, pre_key_window, k_window, v_window) -> (H,W) bool`` is
        called when the deferred window is full (slot W-1 written).
        Returns ``(cache_seqlens (H,), block_table (H,maxB))`` for attention.
        """
        W = self.W
        if layer == 0 and self.local_length == W:
            self.migrate()
        if self.local_length < W:
            slot, cur = self.local_length, self.local_length + 1
        else:
            slot, cur = self.local_ptr, W
        rows = self.local_region_starts[layer].long() + slot
        self.block_pool_k[rows] = key
        self.block_pool_v[rows] = value
        if g_mask is None:
            self.local_pre_key[layer, :, slot] = pre_key
            if slot == W - 1:
                self.refresh(layer, regate)
        else:
            self.local_is_global[layer, :, slot] = g_mask
        if layer == self.L - 1:
            if self.local_length < W:
                self.local_length = cur
            else:
                self.local_ptr = (self.local_ptr + 1) % W
        seqlens = (cur + self.global_lengths[layer]).to(torch.int32)
        return seqlens, self.block_table[layer].clone()

    def refresh(self, layer, regate):
        """:1169-1180 -- re-gate the whole local window of ``layer`` at once."""
        s = int(self.local_region_starts[layer, 0])
        span = self.H * self.W
        k = self.block_pool_k[s:s + span].view(self.H, self.W, self.D)
        v = self.block_pool_v[s:s + span].view(self.H, self.W, self.D)
        self.local_is_global[layer] = regate(layer, self.local_pre_key[layer], k, v)

    # ------------------------------------------------------------ inspection
    def logical_cache(self, layer, head, cur_len):
        """(K, V) rows a decode step at ``layer`` would attend to, in page order."""
        T = cur_len + int(self.global_lengths[layer, head])
        n_pages = (T + self.P - 1) // self.P
        ids = self.block_table[layer, head, :n_pages].long()
        k = self.block_pool_k.view(self.total_blocks, self.P, self.D)[ids].reshape(-1, self.D)[:T]
        v = self.block_pool_v.view(self.total_blocks, self.P, self.D)[ids].reshape(-1, self.D)[:T]
        return k, v
