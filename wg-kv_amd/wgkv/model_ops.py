"""Fused bf16 decoder building blocks for the end-to-end harness
(csrc/model_ops.hip): RMSNorm with the residual add before it, rotary
embedding of q and k, and the SwiGLU product.  Each replaces a chain of
small torch kernels of the reference model (src/modeling_llama.py:61-76,
:115-146, :149-161, :366, :399) with one launch and rounds to bf16 where the
torch composition does.  ``usable`` says when a call qualifies (bf16 CUDA
tensors of supported shapes); callers keep the torch ops otherwise."""
import torch

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


def rope_qkv(q, k, v, cos, sin):
    """q (B,Hq,S,D), k / v (B,Hkv,S,D) views (d contiguous), cos/sin (B,S,D)
    -> (rotated q, rotated k, v) as (B,H,S,D) views of one contiguous
    (B, S, Hq+2*Hkv, D) buffer, so k and v share strides."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    if cos.stride(-1) != 1:
        cos, sin = cos.contiguous(), sin.contiguous()
    buf = torch.empty(B, S, Hq + 2 * Hkv, D, dtype=q.dtype, device=q.device)
    qo, ko, vo = buf[:, :, :Hq], buf[:, :, Hq:Hq + Hkv], buf[:, :, Hq + Hkv:]

    def st(t):  # (batch, seq, head) strides of a (B, H, S, D) view
        return t.stride(0), t.stride(2), t.stride(1)

    def so(t):  # of a (B, S, H, D) view
        return t.stride(0), t.stride(1), t.stride(2)

    r = _lib.lib().wgkv_rope_qkv(
        _ptr(q), *st(q), _ptr(k), *st(k), _ptr(v), *st(v), _ptr(cos), _ptr(sin), cos.stride(0), cos.stride(1),
        _ptr(qo), *so(qo), _ptr(ko), *so(ko), _ptr(vo), *so(vo), B, S, Hq, Hkv, D, _lib.stream_handle(q.device))
    _lib.check(r, "wgkv_rope_qkv")
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
