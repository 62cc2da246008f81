"""The dual cache: one paged pool shared by the local ring and the per-head
global caches of every (layer, KV head).

Attribute names, dtypes and shapes are those the reference's prefill_wrapper
sets on its cache object (src/modeling_layers.py:1196-1288), so harnesses
that read them (scripts/profiling.py:150-184) work unchanged:

* ``block_table``  int32 (L, Hkv, ceil(max_tokens_per_head/16)), sentinel total_blocks-1
* ``block_pool_k`` / ``block_pool_v``  (total_blocks*16, D) in the K/V dtype
* ``local_is_global`` bool (L, Hkv, W); ``global_lengths`` int32 (L, Hkv)
* ``local_region_starts`` int32 (L, Hkv) = (l*Hkv + h) * W
* ``local_ptr``, ``local_length`` host ints; ``total_blocks`` host int
* ``local_pre_key`` (L, Hkv, W, D) when gating is deferred

The bump pointer lives on the device (``next_free_block_dev``) so that no
decode step synchronises with the host; ``next_free_block`` reads it back.
``status`` is a device int32 set to a non-zero code by a kernel that found
the cache full (and then wrote nothing).
"""
import torch

from . import _lib


class DualCache:
    """Cache object for gating_mode 3; pass it as ``past_key_value``."""

    def __init__(self):
        self.gated_kv_initialized = False

    # -- set up at layer-0 prefill, as the reference does (:1196-1288) -----
    def initialize(self, config, head_dim, dtype, device):
        if self.gated_kv_initialized:
            raise AssertionError("dual cache is already initialised")  # reference :1197
        L = config.num_hidden_layers
        H = config.num_key_value_heads
        W = config.local_window_size
        P = config.block_size
        if W % P:
            raise AssertionError("local_window_size % block_size != 0")
        lb = W // P
        self.num_layers, self.num_kv_heads, self.head_dim = L, H, head_dim
        self.local_window_size, self.block_size = W, P
        self.max_tokens_per_head = config.max_tokens_per_head
        self.total_blocks = (config.max_total_tokens + P - 1) // P
        max_blocks_per_head = (config.max_tokens_per_head + P - 1) // P
        n_local = L * H * lb
        if n_local >= self.total_blocks:
            raise AssertionError("max_total_tokens cannot hold the local windows")
        i32 = dict(dtype=torch.int32, device=device)
        self.block_table = torch.full((L, H, max_blocks_per_head), self.total_blocks - 1, **i32)
        self.block_table[:, :, :lb] = torch.arange(n_local, **i32).view(L, H, lb)
        self.block_pool_k = torch.empty(self.total_blocks * P, head_dim, dtype=dtype, device=device)
        self.block_pool_v = torch.empty(self.total_blocks * P, head_dim, dtype=dtype, device=device)
        self.local_is_global = torch.zeros(L, H, W, dtype=torch.bool, device=device)
        self.global_lengths = torch.zeros(L, H, **i32)
        self.local_region_starts = ((torch.arange(L, **i32)[:, None] * H + torch.arange(H, **i32)[None, :]) * W)
        self.local_pre_key = (torch.empty(L, H, W, head_dim, dtype=dtype, device=device)
                              if getattr(config, "g_defer", False) else None)
        if getattr(config, "snapkv_enabled", False):  # reference :1249-1261
            if getattr(config, "use_quest", False):
                raise AssertionError("SnapKV and QUEST are exclusive")
            if not (config.snapkv_max_cached_tokens > 0 and 0.0 < config.snapkv_evict_ratio <= 1.0
                    and config.snapkv_kernel_size % 2 == 1):
                raise AssertionError("invalid SnapKV settings")
            self.snapkv_query_buffer = torch.empty(L, config.snapkv_window_size, config.num_attention_heads,
                                                   head_dim, dtype=dtype, device=device)
            self.snapkv_query_length = 0
            self.snapkv_query_ptr = 0
            # [evicted on the last call, evictions so far] -- decided on the device
            self.snapkv_state = torch.zeros(2, **i32)
            # the released pages, in release order, and their count -- on the device,
            # where the promotion kernel takes pages from the end of the list
            self.free_block_ids_dev = torch.zeros(self.total_blocks, **i32)
            self.free_count_dev = torch.zeros(1, **i32)
        if getattr(config, "use_quest", False):  # page key bounds (reference :1232-1240)
            self.quest_block_key_min = torch.empty(self.total_blocks, head_dim, dtype=dtype, device=device)
            self.quest_block_key_max = torch.empty(self.total_blocks, head_dim, dtype=dtype, device=device)
        self.local_ptr = 0
        self.local_length = 0
        self.prefill_length = 0  # prompt tokens in the cache (all layers); chunks continue from here
        self.decode_started = False
        # (local_ptr, local_length, slot of the last ring write) on the device
        # for graph-captured decode steps
        self.ring_state = torch.zeros(3, **i32)
        self.device_ring = False
        # deferred gating: when set, decode steps leave the window re-gate to
        # the caller (layers.refresh_windows after a step that wrote slot W-1)
        self.refresh_by_caller = False
        # the layer whose decode-step ring write its q/k/v projection's launch
        # has already done (decode_wrapper then skips the append), else None
        self.ring_written_by = None
        self.next_free_block_dev = torch.full((1,), n_local, **i32)
        self.status = torch.zeros(1, **i32)
        # random_sparsity ablation: decode-step draws per layer so far (device
        # counters of the counter-based generator) and its seed
        self.random_draws = torch.zeros(L, **i32)
        self.random_seed = int(getattr(config, "random_seed", 0))
        self.cache_seqlens = torch.zeros(L, 1, H, **i32)   # decode lengths, one row per layer
        self.gated_kv_initialized = True

    def use_device_ring(self, on=True):
        """Switch decode steps to the device copy of the ring pointers (for
        HIP-graph capture of a whole decode step); the copy is loaded from the
        host pointers here.  The host pointers keep being advanced by the
        Python decode path; a caller replaying a captured step advances them
        with ``advance_host_ring``."""
        if on:
            self.ring_state.copy_(torch.tensor([self.local_ptr, self.local_length, -1], dtype=torch.int32))
        self.device_ring = on

    def advance_host_ring(self):
        """The host-side pointer update decode_wrapper makes after the last
        layer (src/modeling_layers.py:1409-1413)."""
        if self.local_length < self.local_window_size:
            self.local_length += 1
        else:
            self.local_ptr = (self.local_ptr + 1) % self.local_window_size

    @property
    def free_block_ids(self):
        """SnapKV's released-page list (a host copy; the device list is
        ``free_block_ids_dev[:free_count_dev]``)."""
        n = int(self.free_count_dev.item())
        return self.free_block_ids_dev[:n].tolist()

    @property
    def snapkv_evict_count(self):
        """Evictions so far (the reference's snapkv_evict_count, :1506); a
        host read of the device counter."""
        return int(self.snapkv_state[1].item())

    @property
    def next_free_block(self):
        return int(self.next_free_block_dev.item())

    def raise_if_failed(self, where):
        code = int(self.status.item())
        if code:
            self.status.zero_()
            raise _lib.WGKVCapacityError(code, where)

    def k_cache(self):
        return self.block_pool_k.view(self.total_blocks, self.block_size, self.head_dim)

    def v_cache(self):
        return self.block_pool_v.view(self.total_blocks, self.block_size, self.head_dim)
