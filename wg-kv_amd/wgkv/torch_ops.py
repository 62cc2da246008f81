"""The path's functional entry points as torch dispatcher operators.

``torch.ops.wgkv.*`` wraps the C-ABI library for callers that go through
the dispatcher (tracing, ``torch.compile``, other frameworks' op
registries).  Each operator has a CUDA (HIP) kernel -- the library call --
and a Meta kernel that only computes output shapes, so graphs can be traced
without running the path.  The layer's default swap points (``prefill_kernel``,
``decode_kernel_handle``) call these operators.

Operators (schemas below):
  sparse_attn             -- sparse_attn_func, the prefill kernel the
                             reference calls at src/modeling_layers.py:1366-1374
  paged_decode_attn       -- flash_attn_with_kvcache as wrapped at :766-800
  generate_sparse_indices -- :384-409 (column_index width = seq_len)
  gate_scores_and_mask    -- GatingPredictor.forward (:170-205) plus the
                             admission of :1465, on fp32 parameters (with
                             the optional packed first layer)
  gate_pack_weights       -- the packed first layer of the bf16
                             matrix-core gate path (no reference counterpart)
"""
import torch

from . import ops as _ops
from .gate import gate_scores_and_mask as _gate_scores_and_mask
from .gate import pack_weights as _pack_weights

_INPUT_NAMES = ("pre_k", "post_k", "v")

_LIB = torch.library.Library("wgkv", "DEF")
_LIB.define("sparse_attn(Tensor q, Tensor k, Tensor v, Tensor block_count, Tensor block_offset, "
            "Tensor column_count, Tensor column_index, float softmax_scale) -> Tensor")
_LIB.define("paged_decode_attn(Tensor q, Tensor k_cache, Tensor v_cache, Tensor cache_seqlens, "
            "Tensor block_table, float softmax_scale) -> Tensor")
_LIB.define("generate_sparse_indices(Tensor g_mask, int local_window_size, int block_size=64) "
            "-> (Tensor, Tensor, Tensor, Tensor)")
_LIB.define("gate_scores_and_mask(Tensor? pre_key, Tensor? post_key, Tensor? value, Tensor? w_pre, "
            "Tensor? w_post, Tensor? w_v, Tensor w1, Tensor b1, Tensor w2, Tensor b2, int inner, int act, "
            "bool rms, float clamp_min, float threshold, Tensor? w1_packed=None, int precision=0) -> (Tensor, Tensor)")
_LIB.define("gate_pack_weights(Tensor? w_pre, Tensor? w_post, Tensor? w_v, Tensor w1, int inputs_mask, bool rms, "
            "int num_kv_heads, int head_dim, int inner, int precision=0) -> Tensor")


# ---- CUDA (HIP) kernels: the library calls ----------------------------------
def _sparse_attn(q, k, v, block_count, block_offset, column_count, column_index, softmax_scale):
    return _ops.sparse_attn_func(q, k, v, block_count, block_offset, column_count, column_index,
                                 softmax_scale=softmax_scale)


def _paged_decode_attn(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale):
    return _ops.paged_decode_attn(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale)


def _generate_sparse_indices(g_mask, local_window_size, block_size=64):
    B, H, S = g_mask.shape
    return _ops.generate_sparse_indices(g_mask, local_window_size, B, H, S, block_size=block_size)


def _gate(pre_key, post_key, value, w_pre, w_post, w_v, w1, b1, w2, b2, inner, act, rms, clamp_min, threshold,
          w1_packed=None, precision=0):
    return _gate_scores_and_mask(pre_key, post_key, value, w_pre, w_post, w_v, w1, b1, w2, b2, inner, act, rms,
                                 clamp_min, threshold, w1_packed=w1_packed, precision=precision)


def _gate_pack(w_pre, w_post, w_v, w1, inputs_mask, rms, num_kv_heads, head_dim, inner, precision=0):
    names = [n for i, n in enumerate(_INPUT_NAMES) if inputs_mask >> i & 1]
    return _pack_weights(w_pre, w_post, w_v, w1, names, rms, num_kv_heads, head_dim, inner, precision=precision)


_LIB.impl("sparse_attn", _sparse_attn, "CUDA")
_LIB.impl("paged_decode_attn", _paged_decode_attn, "CUDA")
_LIB.impl("generate_sparse_indices", _generate_sparse_indices, "CUDA")
_LIB.impl("gate_scores_and_mask", _gate, "CUDA")
_LIB.impl("gate_pack_weights", _gate_pack, "CUDA")


# ---- Meta kernels: output shapes only ----------------------------------------
def _sparse_attn_meta(q, k, v, block_count, block_offset, column_count, column_index, softmax_scale):
    return q.new_empty(q.shape)


def _paged_decode_attn_meta(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale):
    return q.new_empty(q.shape)


def _generate_sparse_indices_meta(g_mask, local_window_size, block_size=64):
    B, H, S = g_mask.shape
    R = (S + block_size - 1) // block_size
    P = min(local_window_size // block_size, R)
    i32 = dict(dtype=torch.int32, device=g_mask.device)
    return (torch.empty(1, 1, R, **i32), torch.empty(1, 1, R, P + 1, **i32),
            torch.empty(B, H, R, **i32), torch.empty(B, H, 1, S, **i32))


def _gate_meta(pre_key, post_key, value, w_pre, w_post, w_v, w1, b1, w2, b2, inner, act, rms, clamp_min, threshold,
               w1_packed=None, precision=0):
    ref = next(t for t in (post_key, pre_key, value) if t is not None)
    B, H, S, _ = ref.shape
    return (torch.empty(B, H, S, dtype=torch.float32, device=ref.device),
            torch.empty(B, H, S, dtype=torch.bool, device=ref.device))


_LIB.impl("sparse_attn", _sparse_attn_meta, "Meta")
_LIB.impl("paged_decode_attn", _paged_decode_attn_meta, "Meta")
_LIB.impl("generate_sparse_indices", _generate_sparse_indices_meta, "Meta")
def _gate_pack_meta(w_pre, w_post, w_v, w1, inputs_mask, rms, num_kv_heads, head_dim, inner, precision=0):
    n_in = bin(inputs_mask & 7).count("1")
    planes = 1 if precision else 3
    tables = 2 * 2 * 20 * 128 * 2 if precision else 0  # bf16 parameters: GELU and SiLU tables after the plane
    return torch.empty(num_kv_heads * inner * n_in * head_dim * planes * 2 + tables, dtype=torch.uint8,
                       device=w1.device)


_LIB.impl("gate_scores_and_mask", _gate_meta, "Meta")
_LIB.impl("gate_pack_weights", _gate_pack_meta, "Meta")


# ---- the layer's swap points through the dispatcher ---------------------------
def sparse_attn_func(q, k, v, block_count, block_offset, column_count, column_index,
                     softmax_scale=None, causal=True, return_softmax_lse=False):
    """``prefill_kernel`` with the reference's signature (:1366-1374),
    dispatched as ``torch.ops.wgkv.sparse_attn``."""
    if not causal:
        raise NotImplementedError("only causal sparse prefill is on the path")
    if return_softmax_lse:
        raise NotImplementedError("return_softmax_lse is not used by the path")
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** -0.5
    return torch.ops.wgkv.sparse_attn(q, k, v, block_count, block_offset, column_count, column_index,
                                      float(softmax_scale))


def paged_decode_attn_handle(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, **_unused):
    """``decode_kernel_handle`` (:766-777): returns a callable that runs
    ``torch.ops.wgkv.paged_decode_attn`` when invoked."""
    def handle():
        return torch.ops.wgkv.paged_decode_attn(q, k_cache, v_cache, cache_seqlens, block_table,
                                                float(softmax_scale))
    return handle
