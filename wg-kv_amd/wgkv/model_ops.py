"""Fused bf16 decoder building blocks for the end-to-end harness
(csrc/model_ops.hip): RMSNorm with the residual add before it, rotary
embedding of q and k, the SwiGLU product, and the one-row products of a
decode step (``linear``, ``swiglu_linear``, the ``Linear`` module).  Each
replaces a chain of small torch kernels of the reference model
(src/modeling_llama.py:61-76, :115-146, :149-161, :366, :399) or a
hipBLASLt call with one launch and rounds to bf16 where the torch
composition does.  ``usable`` says when a call qualifies (bf16 CUDA tensors
of supported shapes); callers keep the torch ops otherwise."""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .ops import _ptr


def _as_rows(t):
    """t as (rows, hidden) with a contiguous last dim (a view when possible)."""
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def usable(*tensors):
    return all(t is not None and t.is_cuda and t.dtype == torch.bfloat16 for t in tensors)


def rms_norm(x, weight, eps, residual=None):
    """weight * bf16(h * rsqrt(mean(h^2) + eps)) over the last dim, h = x (+
    residual).  Returns (out, h) with h the new residual stream (None without
    a residual)."""
    x2 = _as_rows(x)
    rows, hidden = x2.shape
    out = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    r2 = ores = None
    if residual is not None:
        r2 = _as_rows(residual)
        ores = torch.empty(rows, hidden, dtype=x.dtype, device=x.device)
    w = weight if weight.is_contiguous() else weight.contiguous()
    st = _lib.lib().wgkv_rms_norm(_ptr(x2), x2.stride(0), _ptr(r2), 0 if r2 is None else r2.stride(0), _ptr(w),
                                  _ptr(out), hidden, _ptr(ores), 0 if ores is None else hidden, rows, hidden,
                                  float(eps), _lib.stream_handle(x.device))
    _lib.check(st, "wgkv_rms_norm")
    return out.view(x.shape), None if ores is None else ores.view(x.shape)


def rope_qkv(q, k, v, cos, sin, q_norm_weight=None, k_norm_weight=None, eps=1e-6, ring=None):
    """q (B,Hq,S,D), k / v (B,Hkv,S,D) views (d contiguous), cos/sin (B,S,D)
    -> (rotated q, rotated k, v) as (B,H,S,D) views of one contiguous
    (B, S, Hq+2*Hkv, D) buffer, so k and v share strides.  With Qwen3's head
    norm weights (both given) q and k are normalised per head first and the
    normalised, unrotated k is returned as a fourth (B,Hkv,S,D) view.

    ring = (cache, layer, cache_seqlens), for one decode row (B = S = 1) of a
    DualCache with device ring pointers and deferred gating: the same launch
    also does the step's ring write (wgkv_rope_qkv_norm_ring_write), as
    qkv_rope's ring argument does."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if cos.stride(-1) != 1:
        cos, sin = cos.contiguous(), sin.contiguous()
    buf = torch.empty(B, S, Hq + 2 * Hkv, D, dtype=q.dtype, device=q.device)
    qo, ko, vo = buf[:, :, :Hq], buf[:, :, Hq:Hq + Hkv], buf[:, :, Hq + Hkv:]
    norm = q_norm_weight is not None
    if ring is not None:
        if B != 1 or S != 1:
            raise ValueError("rope_qkv: the ring write takes one decode row")
        cache, layer, seqlens = ring
        kp = torch.empty(B, S, Hkv, D, dtype=q.dtype, device=q.device) if norm else None
        r = _lib.lib().wgkv_rope_qkv_norm_ring_write(
            _ptr(q), q.stride(1), _ptr(k), k.stride(1), _ptr(v), v.stride(1), _ptr(cos), _ptr(sin),
            _ptr(qo), qo.stride(2), _ptr(ko), ko.stride(2), _ptr(vo), vo.stride(2), Hq, Hkv, D,
            _ptr(q_norm_weight), _ptr(k_norm_weight), float(eps), _ptr(kp), kp.stride(2) if norm else 0,
            layer, cache.num_layers, cache.local_window_size, _ptr(cache.ring_state),
            _ptr(cache.block_pool_k), _ptr(cache.block_pool_v), _ptr(cache.local_pre_key),
            _ptr(cache.global_lengths), _ptr(seqlens), _lib.stream_handle(q.device))
        _lib.check(r, "wgkv_rope_qkv_norm_ring_write")
        if norm:
            return qo.transpose(1, 2), ko.transpose(1, 2), vo.transpose(1, 2), kp.transpose(1, 2)
        return qo.transpose(1, 2), ko.transpose(1, 2), vo.transpose(1, 2)

    def st(t):  # (batch, seq, head) strides of a (B, H, S, D) view
        return t.stride(0), t.stride(2), t.stride(1)

    def so(t):  # of a (B, S, H, D) view
        return t.stride(0), t.stride(1), t.stride(2)

    kp = torch.empty(B, S, Hkv, D, dtype=q.dtype, device=q.device) if norm else None
    r = _lib.lib().wgkv_rope_qkv_norm(
        _ptr(q), *st(q), _ptr(k), *st(k), _ptr(v), *st(v), _ptr(cos), _ptr(sin), cos.stride(0), cos.stride(1),
        _ptr(qo), *so(qo), _ptr(ko), *so(ko), _ptr(vo), *so(vo), B, S, Hq, Hkv, D,
        _ptr(q_norm_weight), _ptr(k_norm_weight), float(eps), _ptr(kp), *(so(kp) if norm else (0, 0, 0)),
        _lib.stream_handle(q.device))
    _lib.check(r, "wgkv_rope_qkv_norm")
    if norm:
        return qo.transpose(1, 2), ko.transpose(1, 2), vo.transpose(1, 2), kp.transpose(1, 2)
    return qo.transpose(1, 2), ko.transpose(1, 2), vo.transpose(1, 2)


def silu_mul(gate, up):
    """bf16(bf16(silu(gate)) * up) over the last dim for same-shape tensors
    whose rows may be strided (the halves of one fused projection); returns
    a contiguous tensor."""
    g2, u2 = _as_rows(gate), _as_rows(up)
    rows, cols = g2.shape
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    st = _lib.lib().wgkv_silu_mul(_ptr(g2), g2.stride(0), _ptr(u2), u2.stride(0), _ptr(out), rows, cols,
                                  _lib.stream_handle(gate.device))
    _lib.check(st, "wgkv_silu_mul")
    return out


def gemv_usable(x, weight):
    """x is one row (a decode step's activation) that wgkv_gemv takes with
    this (n, k) weight."""
    return (usable(x, weight) and x.numel() == x.shape[-1] == weight.shape[-1] and x.is_contiguous()
            and weight.dim() == 2 and weight.stride(-1) == 1 and weight.stride(0) % 8 == 0
            and weight.shape[-1] % 8 == 0 and weight.shape[-1] <= 32768
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


def _gemv(x, weight, n, mode, residual=None):
    y = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=x.device)
    st = _lib.lib().wgkv_gemv(_ptr(weight), weight.stride(0), n, weight.shape[-1], _ptr(x), _ptr(y), mode,
                              _ptr(residual), _lib.stream_handle(x.device))
    _lib.check(st, "wgkv_gemv")
    return y


def linear(x, weight, residual=None):
    """x @ weight.T (+ residual): for one bf16 row on the decode GEMV
    (wgkv_gemv mode 0, or mode 1 with the residual add fused), otherwise
    F.linear (then residual + y, as torch rounds it)."""
    n = weight.shape[0]
    if gemv_usable(x, weight) and (residual is None or (usable(residual) and residual.is_contiguous()
                                                        and residual.numel() == n)):
        return _gemv(x, weight, n, 0 if residual is None else 1, residual)
    y = F.linear(x, weight)
    return y if residual is None else residual + y


def swiglu_linear(x, gate_up_weight):
    """bf16(silu(x @ W_gate.T)) * (x @ W_up.T) for the stacked (2n, k)
    [gate; up] weight: one wgkv_gemv (mode 2) for a single bf16 row,
    otherwise two F.linear and the SwiGLU product."""
    n = gate_up_weight.shape[0] // 2
    if gemv_usable(x, gate_up_weight):
        return _gemv(x, gate_up_weight, n, 2)
    g, u = F.linear(x, gate_up_weight[:n]), F.linear(x, gate_up_weight[n:])
    if usable(g, u) and n % 8 == 0:
        return silu_mul(g, u)
    return F.silu(g) * u


def qkv_rope(x, w_qkv, cos, sin, num_q_heads, num_kv_heads, head_dim, norm_weight=None, eps=1e-5, ring=None):
    """One decode row's q/k/v projection with rotary embedding (wgkv_gemv_ex
    mode 3), optionally after the input RMSNorm: x (1, 1, hidden) bf16 (the
    residual stream when norm_weight is given), w_qkv the stacked (n, hidden)
    weight, cos / sin (1, 1, head_dim).  Returns (buf (1, 1, Hq + 2 Hkv, D)
    with rotated q, rotated k and v, the unrotated k (1, 1, Hkv, D)), the
    values wgkv_rms_norm, the product and wgkv_rope_qkv give.

    ring = (cache, layer, cache_seqlens): the same launch also does the
    decode step's ring write of a DualCache with device ring pointers and
    deferred gating (wgkv_qkv_rope_ring_write): rotated k, v and the
    unrotated k into the ring slot, cache_seqlens (the layer's (Hkv,) int32)
    and the written slot, as wgkv_decode_append_ring without a mask, a
    migration or an advance would."""
    n = (num_q_heads + 2 * num_kv_heads) * head_dim
    buf = torch.empty(1, 1, num_q_heads + 2 * num_kv_heads, head_dim, dtype=x.dtype, device=x.device)
    kraw = torch.empty(1, 1, num_kv_heads, head_dim, dtype=x.dtype, device=x.device)
    c, s_ = cos.reshape(-1), sin.reshape(-1)
    if ring is not None:
        cache, layer, seqlens = ring
        st = _lib.lib().wgkv_qkv_rope_ring_write(
            _ptr(w_qkv), w_qkv.stride(0), w_qkv.shape[-1], _ptr(x), _ptr(buf), _ptr(norm_weight), float(eps),
            _ptr(c), _ptr(s_), _ptr(kraw), num_q_heads, num_kv_heads, head_dim,
            layer, cache.num_layers, cache.local_window_size, _ptr(cache.ring_state),
            _ptr(cache.block_pool_k), _ptr(cache.block_pool_v), _ptr(cache.local_pre_key),
            _ptr(cache.global_lengths), _ptr(seqlens), _lib.stream_handle(x.device))
        _lib.check(st, "wgkv_qkv_rope_ring_write")
        return buf, kraw
    st = _lib.lib().wgkv_gemv_ex(_ptr(w_qkv), w_qkv.stride(0), n, w_qkv.shape[-1], _ptr(x), _ptr(buf), 3, None,
                                 _ptr(norm_weight), None, None, float(eps), _ptr(c), _ptr(s_), _ptr(kraw),
                                 num_q_heads, num_kv_heads, head_dim, _lib.stream_handle(x.device))
    _lib.check(st, "wgkv_gemv_ex")
    return buf, kraw


def rms_norm_linear(x, norm_weight, eps, weight, residual=None, mode=0):
    """weight @ RMSNorm(x (+ residual)) for one decode row in one launch
    (wgkv_gemv_ex with the norm prologue; mode 0 plain, 2 the SwiGLU product
    of a stacked [gate; up] weight).  Returns (y, h) with h = x + residual
    (None without a residual), bit for bit rms_norm followed by linear /
    swiglu_linear."""
    n = weight.shape[0] // 2 if mode == 2 else weight.shape[0]
    y = torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=x.device)
    h = torch.empty_like(x) if residual is not None else None
    st = _lib.lib().wgkv_gemv_ex(_ptr(weight), weight.stride(0), n, weight.shape[-1], _ptr(x), _ptr(y), mode, None,
                                 _ptr(norm_weight), _ptr(residual), _ptr(h), float(eps), None, None, None, 0, 0, 0,
                                 _lib.stream_handle(x.device))
    _lib.check(st, "wgkv_gemv_ex")
    return y, h


def rms_norm_linear_usable(x, norm_weight, weight, residual=None):
    """rms_norm_linear takes this row, norm weight, product weight and
    residual (the norm prologue handles rows of up to 8192 elements)."""
    return (gemv_usable(x, weight) and usable(norm_weight) and norm_weight.is_contiguous()
            and norm_weight.numel() == x.shape[-1] <= 8192 and norm_weight.data_ptr() % 16 == 0
            and (residual is None or (usable(residual) and residual.is_contiguous()
                                      and residual.numel() == x.numel() and residual.data_ptr() % 16 == 0)))


def qkv_rope_usable(x, w_qkv, cos, sin, norm_weight=None):
    return (gemv_usable(x, w_qkv) and usable(cos, sin) and cos.numel() == sin.numel() == cos.shape[-1]
            and cos.is_contiguous() and sin.is_contiguous()
            and (norm_weight is None or (usable(norm_weight) and norm_weight.is_contiguous()
                                         and norm_weight.data_ptr() % 16 == 0 and x.shape[-1] <= 8192)))


class Linear(nn.Linear):
    """nn.Linear (same parameters and state-dict names) whose bias-free
    one-row products -- a decode step's -- run on wgkv_gemv."""

    def forward(self, x):
        if self.bias is None:
            return linear(x, self.weight)
        return super().forward(x)
