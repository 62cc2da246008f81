"""MI355X-native write-gated dual-cache KV path (WG-KV hot path).

Host side of the path: the reference's layer/cache API on top of the HIP
C-ABI library ``libwgkv.so`` (include/wgkv.h).  Device work always goes
through that library; there is no CPU fallback.
"""
from . import _lib, ops, torch_ops  # noqa: F401  (torch_ops registers torch.ops.wgkv.*)
from .ops import (  # noqa: F401
    flash_attn_with_kvcache_wrapper,
    flash_attn_with_kvcache_wrapper_handle,
    flash_attn_with_kvcache_wrapper_triton,
    flash_attn_with_kvcache_wrapper_triton_handle,
    generate_sparse_indices,
    paged_decode_attn,
    paged_decode_attn_handle,
    sparse_attn_func,
)

__all__ = [
    "sparse_attn_func",
    "generate_sparse_indices",
    "paged_decode_attn",
    "paged_decode_attn_handle",
    "flash_attn_with_kvcache_wrapper",
    "flash_attn_with_kvcache_wrapper_handle",
    "flash_attn_with_kvcache_wrapper_triton",
    "flash_attn_with_kvcache_wrapper_triton_handle",
]
