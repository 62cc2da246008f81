"""torch-facing wrappers of the HIP kernels (device memory and streams only).

Each wrapper validates shapes/dtypes on the host, passes raw pointers and
strides to the C ABI and raises on a non-zero status.  Scratch memory is a
per-device workspace tensor allocated once and reused by every call on the
device: calls issued on one stream run in turn, but calls on different
streams of one device that may run at the same time would share (and
corrupt) the workspace and must not be made -- the C ABI's rule for its
workspace arguments.  A workspace that is replaced by a larger one is kept
alive (not returned to the caching allocator), because a captured HIP graph
may still hold its address.
"""
import torch

from . import _lib

_workspaces = {}
_decode_workspaces = {}
_retired = []  # replaced workspaces, kept for graphs captured with their addresses


def _dev_key(device):
    dev = torch.device(device)
    return dev, (dev.index if dev.index is not None else torch.cuda.current_device())


def workspace(device, nbytes):
    """Uninitialised per-device scratch of at least ``nbytes`` bytes."""
    dev, key = _dev_key(device)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _retired.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _workspaces[key] = ws
    return ws


def decode_workspace(device):
    """The decode attention's per-device workspace (arrival counters and split
    partials), sized for the largest head_dim so that it never grows and a
    captured graph's address stays valid.  Zero-filled once: every call
    leaves its arrival counters zero again."""
    dev, key = _dev_key(device)
    ws = _decode_workspaces.get(key)
    if ws is None:
        nbytes = int(_lib.lib().wgkv_paged_decode_workspace_bytes(1, 1, 128))
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        _decode_workspaces[key] = ws
    return ws


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _require_cuda(*tensors):
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("wgkv kernels take device tensors (no CPU fallback)")


# ---------------------------------------------------------------------------
# kernel (2): ragged paged decode attention
# ---------------------------------------------------------------------------
def _validate_decode(q, k_cache, v_cache, cache_seqlens, block_table):
    """Shape contract of src/modeling_layers.py:818-831, generalised to batch > 1."""
    if q.dim() != 4 or q.shape[1] != 1:
        raise AssertionError("q must be (batch, 1, num_query_heads, head_size)")
    B, _, Hq, D = q.shape
    if cache_seqlens.dim() != 2 or cache_seqlens.shape[0] != B:
        raise AssertionError("cache_seqlens must be (batch, num_kv_heads)")
    Hkv = cache_seqlens.shape[1]
    if Hq % Hkv:
        raise AssertionError("num_query_heads must be a multiple of num_kv_heads")
    if block_table.dim() != 3 or block_table.shape[:2] != (B, Hkv):
        raise AssertionError("block_table must be (batch, num_kv_heads, max_blocks)")
    if k_cache.dim() != 3 or k_cache.shape != v_cache.shape or k_cache.shape[2] != D:
        raise AssertionError("k_cache/v_cache must be (num_blocks, block_size, head_size)")
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("This kernel only supports BF16 inputs for q, k_cache, and v_cache.")
    if cache_seqlens.dtype != torch.int32 or block_table.dtype != torch.int32:
        raise TypeError("cache_seqlens and block_table must be int32")
    return B, Hq, Hkv, D


def paged_decode_attn(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, out=None):
    """Decode attention over paged per-head caches; returns (B, 1, Hq, D) bf16."""
    B, Hq, Hkv, D = _validate_decode(q, k_cache, v_cache, cache_seqlens, block_table)
    _require_cuda(q, k_cache, v_cache, cache_seqlens, block_table)
    q3 = q[:, 0]
    if q3.stride(2) != 1:
        q3 = q3.contiguous()
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache/v_cache must be contiguous")
    sl = cache_seqlens if cache_seqlens.stride(1) == 1 else cache_seqlens.contiguous()
    bt = block_table if block_table.stride(2) == 1 else block_table.contiguous()
    if out is None:
        out = torch.empty(B, 1, Hq, D, dtype=torch.bfloat16, device=q.device)
    o3 = out[:, 0]
    L = _lib.lib()
    ws = decode_workspace(q.device)
    st = L.wgkv_paged_decode_attn(
        _ptr(q3), q3.stride(0), q3.stride(1),
        _ptr(k_cache), _ptr(v_cache), k_cache.shape[0], k_cache.shape[1],
        _ptr(sl), sl.stride(0),
        _ptr(bt), bt.stride(0), bt.stride(1), bt.shape[2],
        _ptr(o3), o3.stride(0), o3.stride(1),
        B, Hq, Hkv, D,
        float(softmax_scale),
        _ptr(ws), ws.numel(),
        _lib.stream_handle(q.device))
    _lib.check(st, "wgkv_paged_decode_attn")
    return out


def paged_decode_attn_handle(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, **_unused):
    """Handle form used by ``decode_kernel_handle`` (src/modeling_layers.py:1439-1447).

    Validation and output allocation happen now; the returned closure only
    enqueues the kernels, so it can be re-run (or timed) on its own.
    """
    B, Hq, Hkv, D = _validate_decode(q, k_cache, v_cache, cache_seqlens, block_table)
    out = torch.empty(B, 1, Hq, D, dtype=torch.bfloat16, device=q.device)

    def handle():
        return paged_decode_attn(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, out=out)

    return handle


# Names of the reference's decode entry points (src/modeling_layers.py:766-815,
# :1007-1140): all resolve to the HIP kernel.
flash_attn_with_kvcache_wrapper = paged_decode_attn
flash_attn_with_kvcache_wrapper_handle = paged_decode_attn_handle
flash_attn_with_kvcache_wrapper_triton_handle = paged_decode_attn_handle


def flash_attn_with_kvcache_wrapper_triton(*args, **kwargs):
    return paged_decode_attn_handle(*args, **kwargs)()


# ---------------------------------------------------------------------------
# kernel (4), prefill half: vertical-slash metadata
# ---------------------------------------------------------------------------
def generate_sparse_indices(g_mask, local_window_size, batch_size, num_kv_heads, seq_len, device=None,
                            block_size=64, exact_width=False):
    """Device-built metadata with the signature of src/modeling_layers.py:385-409.

    Returns ``(block_count (1,1,R), block_offset (1,1,R,P+1), column_count
    (B,Hkv,R), column_index (B,Hkv,1,N))``.  ``N`` is ``seq_len`` (an upper
    bound, no host sync) unless ``exact_width`` is set, in which case the
    per-head totals are read back and ``N`` is the reference's
    ``max_global_size``.  Only the valid prefixes carry meaning, as in the
    reference's own test (utils/test_sparse_indices.py:30-48).
    """
    if local_window_size % block_size != 0:
        raise AssertionError("local_window_size must be a multiple of block_size")
    if g_mask.shape != (batch_size, num_kv_heads, seq_len):
        raise AssertionError("g_mask must be (batch, num_kv_heads, seq_len)")
    _require_cuda(g_mask)
    dev = g_mask.device
    m = g_mask if g_mask.dtype == torch.uint8 else g_mask.to(torch.bool).view(torch.uint8)
    if m.stride(2) != 1:
        m = m.contiguous()
    R = (seq_len + block_size - 1) // block_size
    P = min(local_window_size // block_size, R)
    i32 = dict(dtype=torch.int32, device=dev)
    block_count = torch.empty(1, 1, R, **i32)
    block_offset = torch.empty(1, 1, R, P + 1, **i32)
    column_count = torch.empty(batch_size, num_kv_heads, R, **i32)
    column_index = torch.empty(batch_size, num_kv_heads, 1, seq_len, **i32)
    column_total = torch.empty(batch_size, num_kv_heads, **i32)
    st = _lib.lib().wgkv_build_prefill_meta(
        _ptr(m), m.stride(0), m.stride(1),
        batch_size, num_kv_heads, seq_len, local_window_size, block_size,
        _ptr(block_count), _ptr(block_offset),
        _ptr(column_count), _ptr(column_index), seq_len, _ptr(column_total),
        _lib.stream_handle(dev))
    _lib.check(st, "wgkv_build_prefill_meta")
    if exact_width:
        width = int(column_total.max().item())
        column_index = column_index[..., :width]
    return block_count, block_offset, column_count, column_index


# ---------------------------------------------------------------------------
# kernel (1), cache half: prefill admission and the decode-step append
# ---------------------------------------------------------------------------
def _u8(mask):
    return mask if mask.dtype == torch.uint8 else mask.to(torch.bool).view(torch.uint8)


def prefill_admit(cache, layer, key, value, g_mask, pre_key=None):
    """Admission of one layer's prompt into ``cache`` (batch 1).

    key/value/pre_key (H, S, D) bf16 views (d contiguous), g_mask (H, S).
    Capacity failures are recorded in ``cache.status`` (read by the caller).
    """
    H, S, D = key.shape
    _require_cuda(key, value, g_mask)
    m = _u8(g_mask)
    if m.stride(1) != 1:
        m = m.contiguous()
    L = _lib.lib()
    ws = workspace(key.device, L.wgkv_prefill_admit_workspace_bytes(H, S))
    lpk = cache.local_pre_key if (pre_key is not None and cache.local_pre_key is not None) else None
    st = L.wgkv_prefill_admit(
        _ptr(key), _ptr(value), key.stride(0), key.stride(1),
        _ptr(pre_key) if lpk is not None else None,
        pre_key.stride(0) if lpk is not None else 0, pre_key.stride(1) if lpk is not None else 0,
        _ptr(m), m.stride(0),
        layer, cache.num_layers, H, S, D,
        cache.local_window_size, cache.block_size, cache.max_tokens_per_head, cache.total_blocks,
        _ptr(cache.block_pool_k), _ptr(cache.block_pool_v), _ptr(cache.block_table), cache.block_table.shape[2],
        _ptr(cache.global_lengths), _ptr(cache.local_is_global.view(torch.uint8)), _ptr(lpk),
        _ptr(cache.next_free_block_dev), _ptr(cache.status),
        _ptr(ws), ws.numel(), _lib.stream_handle(key.device))
    _lib.check(st, "wgkv_prefill_admit")


def decode_append(cache, layer, key=None, value=None, g_mask=None, pre_key=None, migrate=False, write=True,
                  cache_seqlens=None, advance=False):
    """Decode-step cache update of ``cache``: optional lazy promotion (all
    layers) and the ring write of ``layer``'s token.  key/value/pre_key (H, D).

    With ``cache.device_ring`` the ring pointers are read from (and, with
    ``advance``, advanced in) ``cache.ring_state`` on the device, so the step
    can be captured in a HIP graph; promotion then runs only if the ring is
    full, decided on the device."""
    H = cache.num_kv_heads
    D = cache.head_dim
    L = _lib.lib()
    m = None
    if write and g_mask is not None:
        m = _u8(g_mask).reshape(H).contiguous()
    head = (_ptr(key) if write else None, _ptr(value) if write else None, key.stride(0) if write else 0,
            _ptr(pre_key) if (write and pre_key is not None) else None,
            pre_key.stride(0) if (write and pre_key is not None) else 0,
            _ptr(m),
            layer, cache.num_layers, H, D,
            cache.local_window_size, cache.block_size, cache.max_tokens_per_head, cache.total_blocks)
    tail = (_ptr(cache.block_pool_k), _ptr(cache.block_pool_v), _ptr(cache.block_table), cache.block_table.shape[2],
            _ptr(cache.global_lengths), _ptr(cache.local_is_global.view(torch.uint8)), _ptr(cache.local_pre_key),
            _ptr(cache.next_free_block_dev), _ptr(cache_seqlens), _ptr(cache.status),
            _ptr(getattr(cache, "quest_block_key_min", None)), _ptr(getattr(cache, "quest_block_key_max", None)),
            _ptr(getattr(cache, "free_block_ids_dev", None)), _ptr(getattr(cache, "free_count_dev", None)),
            _lib.stream_handle(cache.block_pool_k.device))
    if getattr(cache, "device_ring", False):
        st = L.wgkv_decode_append_ring(*head, _ptr(cache.ring_state), int(advance), int(migrate), int(write), *tail)
        _lib.check(st, "wgkv_decode_append_ring")
    else:
        st = L.wgkv_decode_append(*head, cache.local_ptr, cache.local_length, int(migrate), int(write), *tail)
        _lib.check(st, "wgkv_decode_append")


def random_admission(flags, random_sparsity, seed, draw_counter, active=None):
    """wgkv_random_admission: flags (H, n) bool device tensor (n contiguous)
    <- r >= bf16(random_sparsity) for counter-based draws r in [0, 1)
    (get_random_g_scores, src/modeling_layers.py:1160-1166, made on the
    device); ``draw_counter`` is a device int32 (one element) the call
    advances; ``active`` = (device int32 tensor, value): the launch does
    nothing unless the tensor's first element equals value."""
    if flags.dim() != 2 or flags.dtype != torch.bool or flags.stride(1) != 1:
        raise AssertionError("flags must be a (H, n) bool tensor with n contiguous")
    if draw_counter.dtype != torch.int32 or not draw_counter.is_cuda:
        raise TypeError("draw_counter must be a device int32 tensor")
    _require_cuda(flags)
    H, n = flags.shape
    st = _lib.lib().wgkv_random_admission(
        _ptr(flags.view(torch.uint8)), flags.stride(0), H, n, float(random_sparsity), int(seed) & (2 ** 64 - 1),
        _ptr(draw_counter), _ptr(active[0]) if active is not None else None,
        int(active[1]) if active is not None else 0, _lib.stream_handle(flags.device))
    _lib.check(st, "wgkv_random_admission")


# ---------------------------------------------------------------------------
# kernel (3): sparse (vertical-slash) causal prefill attention
# ---------------------------------------------------------------------------
def sparse_attn_func(q, k, v, block_count, block_offset, column_count, column_index,
                     softmax_scale=None, causal=True, return_softmax_lse=False, out=None):
    """The contract of the reference's sparse_attn_func
    (src/modeling_layers.py:1366-1374): q (B,S,Hq,D), k/v (B,S,Hkv,D) bf16 ->
    (B,S,Hq,D) bf16; metadata from generate_sparse_indices (block 64)."""
    if not causal:
        raise NotImplementedError("only causal sparse prefill is on the path")
    if return_softmax_lse:
        raise NotImplementedError("return_softmax_lse is not used by the path")
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    if k.shape != (B, S, Hkv, D) or v.shape != k.shape:
        raise AssertionError("k/v must be (batch, seq, num_kv_heads, head_dim)")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("sparse prefill takes bf16 q/k/v")
    if k.stride() != v.stride():
        raise ValueError("k and v must share strides")
    _require_cuda(q, k, v, block_count, block_offset, column_count, column_index)
    if q.stride(3) != 1 or k.stride(3) != 1:
        raise ValueError("head_dim must be contiguous")
    R = (S + 63) // 64
    if block_count.numel() != R or column_count.shape != (B, Hkv, R):
        raise AssertionError("metadata does not match (batch, heads, seq) with block 64")
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    bc = block_count.reshape(R).contiguous()
    bo = block_offset.reshape(R, -1).contiguous()
    cc = column_count.contiguous()
    ci = column_index
    if ci.stride(-1) != 1:
        ci = ci.contiguous()
    if out is None:
        out = torch.empty(B, S, Hq, D, dtype=torch.bfloat16, device=q.device)
    st = _lib.lib().wgkv_sparse_prefill_attn(
        _ptr(q), q.stride(0), q.stride(1), q.stride(2),
        _ptr(k), _ptr(v), k.stride(0), k.stride(1), k.stride(2),
        _ptr(out), out.stride(0), out.stride(1), out.stride(2),
        _ptr(bc), _ptr(bo), bo.shape[1],
        _ptr(cc), _ptr(ci), ci.stride(0), ci.stride(1),
        B, S, Hq, Hkv, D, 64, float(softmax_scale), _lib.stream_handle(q.device))
    _lib.check(st, "wgkv_sparse_prefill_attn")
    return out


# ---------------------------------------------------------------------------
# chunked gated prefill: kernels (1) and (3) for a prompt fed in pieces
# ---------------------------------------------------------------------------
class ChunkStep:
    """One layer of one prompt chunk [chunk_start, chunk_start + C) (batch 1),
    in its three device steps: ``admit()`` (admission into the cache and the
    chunk's column counts), ``attend()`` (the chunk's sparse attention) and
    ``ring()`` (the ring rewrite), in that order.  ``chunk_prefill`` runs all
    three.

    q (C, Hq, D), key/value (C, Hkv, D) bf16 views (d contiguous; typically
    ``x[0].transpose(0, 1)`` of the layer's (1, H, C, D) states), g_mask
    (Hkv, C), pre_key like key (deferred gating).  Capacity failures are
    recorded in ``cache.status`` and the chunk's cache writes are skipped.
    """

    def __init__(self, cache, layer, q, key, value, g_mask, chunk_start, softmax_scale=None, pre_key=None,
                 out=None):
        C, Hq, D = q.shape
        Hkv = key.shape[1]
        if key.shape != (C, Hkv, D) or value.shape != key.shape:
            raise AssertionError("key/value must be (chunk_len, num_kv_heads, head_dim)")
        if q.dtype != torch.bfloat16 or key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
            raise TypeError("chunked prefill takes bf16 q/k/v")
        if key.stride() != value.stride():
            raise ValueError("key and value must share strides")
        if g_mask.shape != (Hkv, C):
            raise AssertionError("g_mask must be (num_kv_heads, chunk_len)")
        _require_cuda(q, key, value, g_mask)
        if q.stride(2) != 1 or key.stride(2) != 1:
            raise ValueError("head_dim must be contiguous")
        m = _u8(g_mask)
        if m.stride(1) != 1:
            m = m.contiguous()
        self.cache, self.layer, self.q, self.key, self.value, self.mask = cache, layer, q, key, value, m
        self.c0, self.C, self.Hq, self.Hkv, self.D = chunk_start, C, Hq, Hkv, D
        self.scale = D ** -0.5 if softmax_scale is None else softmax_scale
        self.lib = _lib.lib()
        W = cache.local_window_size
        self.ws = workspace(key.device, self.lib.wgkv_chunk_admit_workspace_bytes(Hkv, C, W))
        self.column_count = torch.empty(Hkv, (C + 63) // 64, dtype=torch.int32, device=key.device)
        self.lpk = cache.local_pre_key if (pre_key is not None and cache.local_pre_key is not None) else None
        self.pre_key = pre_key
        self.out = out if out is not None else torch.empty(C, Hq, D, dtype=torch.bfloat16, device=q.device)
        self.stream = _lib.stream_handle(key.device)

    def _update(self, stage):
        c, k, pk, lpk = self.cache, self.key, self.pre_key, self.lpk
        st = self.lib.wgkv_chunk_cache_update(
            stage,
            _ptr(k), _ptr(self.value), k.stride(1), k.stride(0),
            _ptr(pk) if lpk is not None else None,
            pk.stride(1) if lpk is not None else 0, pk.stride(0) if lpk is not None else 0,
            _ptr(self.mask), self.mask.stride(0),
            self.layer, c.num_layers, self.Hkv, self.c0, self.C, self.D,
            c.local_window_size, c.block_size, c.max_tokens_per_head, c.total_blocks,
            _ptr(c.block_pool_k), _ptr(c.block_pool_v), _ptr(c.block_table), c.block_table.shape[2],
            _ptr(c.global_lengths), _ptr(c.local_is_global.view(torch.uint8)), _ptr(lpk),
            _ptr(c.next_free_block_dev), _ptr(c.status), _ptr(self.column_count),
            _ptr(self.ws), self.ws.numel(), self.stream)
        _lib.check(st, f"wgkv_chunk_cache_update(stage {stage})")

    def admit(self):
        self._update(0)

    def attend(self):
        c, q, k, o = self.cache, self.q, self.key, self.out
        st = self.lib.wgkv_chunk_prefill_attn(
            _ptr(q), q.stride(0), q.stride(1),
            _ptr(k), _ptr(self.value), k.stride(0), k.stride(1),
            _ptr(o), o.stride(0), o.stride(1),
            _ptr(c.block_pool_k), _ptr(c.block_pool_v),
            _ptr(c.block_table), c.block_table.shape[2],
            _ptr(self.column_count),
            self.layer, self.c0, self.C, self.Hq, self.Hkv, self.D, c.local_window_size, c.block_size,
            float(self.scale), self.stream)
        _lib.check(st, "wgkv_chunk_prefill_attn")
        return o

    def ring(self):
        self._update(1)


def chunk_prefill(cache, layer, q, key, value, g_mask, chunk_start, softmax_scale=None, pre_key=None, out=None):
    """Admission, sparse attention and ring rewrite of one layer of one prompt
    chunk (see ChunkStep).  Returns the chunk's (C, Hq, D) bf16 output."""
    step = ChunkStep(cache, layer, q, key, value, g_mask, chunk_start, softmax_scale, pre_key, out)
    step.admit()
    out = step.attend()
    step.ring()
    return out


def chunk_attend(step):
    """The attention kernel of an admitted chunk (``ChunkStep.attend``): the
    default ``chunk_prefill_kernel`` swap point of the layer."""
    return step.attend()


# ---------------------------------------------------------------------------
# QUEST page selection (the reference's comparison baseline) over kernel (2)
# ---------------------------------------------------------------------------
def quest_update_bounds(cache, layer, from_lengths=None):
    """Recompute the page key bounds of ``layer``'s global pages from
    ``from_lengths`` (H,) (the global lengths before an admission; None: from
    the first page)."""
    st = _lib.lib().wgkv_quest_update_bounds(
        _ptr(cache.block_pool_k), _ptr(cache.block_table), cache.block_table.shape[2],
        _ptr(cache.global_lengths), _ptr(from_lengths),
        layer, cache.num_layers, cache.num_kv_heads, cache.local_window_size, cache.block_size,
        cache.head_dim, _ptr(cache.quest_block_key_min), _ptr(cache.quest_block_key_max),
        _lib.stream_handle(cache.block_pool_k.device))
    _lib.check(st, "wgkv_quest_update_bounds")


def quest_select(cache, layer, q, local_tokens, token_budget, scores_bf16=True):
    """quest_select_blocks (src/modeling_layers.py:452-576) for one decode
    step of ``layer``: q (Hq, D) bf16.  Page scores are rounded as the
    reference's bf16 ops round them (``scores_bf16``; False: fp32).  Returns
    (cache_seqlens (1, H), block_table (1, H, cap)) for paged_decode_attn."""
    H, D = cache.num_kv_heads, cache.head_dim
    P = cache.block_size
    cap = (local_tokens + P - 1) // P + (max(token_budget - local_tokens, 0) + P - 1) // P + 1
    dev = q.device
    key = ("quest_sel", H, cap)
    bufs = cache.__dict__.setdefault("_quest_bufs", {})
    if key not in bufs:  # stable buffers (a captured decode step reuses them)
        bufs[key] = (torch.zeros(1, H, cap, dtype=torch.int32, device=dev), torch.zeros(1, H, dtype=torch.int32, device=dev))
    sel_bt, sel_len = bufs[key]
    L = _lib.lib()
    ws = workspace(dev, L.wgkv_quest_select_workspace_bytes(H, cache.block_table.shape[2]))
    st = L.wgkv_quest_select(
        _ptr(q), q.stride(0),
        _ptr(cache.block_table), cache.block_table.shape[2], _ptr(cache.global_lengths),
        _ptr(cache.quest_block_key_min), _ptr(cache.quest_block_key_max),
        layer, cache.num_layers, q.shape[0], H, D,
        cache.local_window_size, P, int(local_tokens), int(token_budget), int(bool(scores_bf16)),
        _ptr(sel_bt), cap, _ptr(sel_len),
        _ptr(ws), ws.numel(), _lib.stream_handle(dev))
    _lib.check(st, "wgkv_quest_select")
    return sel_len, sel_bt


def snapkv_evict(cache, num_kv_groups, softmax_scale, window, kernel_size, evict_ratio, max_cached_tokens=-1,
                 logits_bf16=True, scores_out=None):
    """wgkv_snapkv_evict over every (layer, KV head) of ``cache``
    (snapkv_evict, src/modeling_layers.py:595-671): scores, lowest-score
    selection, in-place packing and page release on the device, run only if
    the sum of the global lengths exceeds ``max_cached_tokens`` (decided on
    the device; -1 always runs).  ``cache.snapkv_state`` (int32 (2)) holds
    [ran on this call, evictions so far].  ``logits_bf16`` rounds the logits
    as the reference's bf16 matmul does.  ``scores_out`` (optional, f32
    (L*H, max_tokens_per_head)) receives the pooled scores of the evicted
    heads."""
    L, H, D, P = cache.num_layers, cache.num_kv_heads, cache.head_dim, cache.block_size
    mtph = cache.max_tokens_per_head
    qbuf = cache.snapkv_query_buffer
    _require_cuda(qbuf, cache.block_pool_k)
    if qbuf.dtype != torch.bfloat16 or not qbuf.is_contiguous():
        raise TypeError("the SnapKV query window must be contiguous bf16")
    if tuple(qbuf.shape) != (L, window, H * num_kv_groups, D):
        raise AssertionError("query window shape does not match the cache")
    dev = qbuf.device
    lib = _lib.lib()
    nbytes = int(lib.wgkv_snapkv_workspace_bytes(L, H, num_kv_groups, window, mtph))
    if nbytes <= 0:
        raise ValueError("unsupported SnapKV shape")
    ws = cache.__dict__.get("_snapkv_ws")
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        cache.__dict__["_snapkv_ws"] = ws
    if scores_out is not None and (scores_out.dtype != torch.float32 or scores_out.numel() < L * H * mtph
                                   or not scores_out.is_contiguous()):
        raise ValueError("scores_out must be contiguous f32 with L*H*max_tokens_per_head elements")
    st = lib.wgkv_snapkv_evict(
        _ptr(cache.block_pool_k), _ptr(cache.block_pool_v), _ptr(cache.block_table), _ptr(cache.global_lengths),
        _ptr(cache.free_block_ids_dev), _ptr(cache.free_count_dev), _ptr(qbuf),
        L, H, int(num_kv_groups), D, P,
        cache.local_window_size // P, cache.block_table.shape[2], cache.total_blocks, mtph,
        int(window), int(kernel_size), float(evict_ratio), float(softmax_scale), int(max_cached_tokens),
        int(bool(logits_bf16)), _ptr(cache.snapkv_state), _ptr(scores_out),
        _ptr(ws), ws.numel(), _lib.stream_handle(dev))
    _lib.check(st, "wgkv_snapkv_evict")
