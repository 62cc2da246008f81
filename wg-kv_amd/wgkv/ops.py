"""torch-facing wrappers of the HIP kernels (device memory and streams only).

Each wrapper validates shapes/dtypes on the host, passes raw pointers and
strides to the C ABI and raises on a non-zero status.  Scratch memory is a
per-device workspace tensor allocated once and reused; calls on one device
are ordered by the stream, so sharing it is safe.
"""
import torch

from . import _lib

_workspaces = {}


def workspace(device, nbytes):
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _workspaces[key] = ws
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
    nbytes = L.wgkv_paged_decode_workspace_bytes(B, Hkv, D)
    ws = workspace(q.device, nbytes)
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
