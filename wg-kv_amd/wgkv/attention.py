"""A Llama/Qwen3-style attention layer whose forward is the reference's.

LlamaAttention.forward (src/modeling_llama.py:252-323, gating_mode 3):
project q/k/v, keep the pre-RoPE key (:269), apply RoPE (:270-271), hand over
to ``self.self_attn_forward_patch`` and project the result with o_proj.  The
swap-point attributes are bound as in the reference (:240-250), so harnesses
that re-bind them (scripts/profiling.py:273-341) keep working.  Qwen3's
variant applies per-head k_norm (and q_norm) before the pre-RoPE key is taken
(src/modeling_qwen3.py:235-239); ``qk_norm=True`` selects it.

The attention kernels and the dual cache are bf16 (as the reference's are);
with an fp32 model the gate still sees fp32 keys and produces fp32 scores,
and q/k/v are rounded to bf16 after gating.
"""
import torch
import torch.nn as nn

from . import layers, model_ops, ops, torch_ops
from .gate import GatingPredictor


class LlamaRotaryEmbedding(nn.Module):
    """Default RoPE (src/modeling_llama.py:81-119): cos/sin of
    position * theta^(-2i/D), duplicated over the two halves."""

    def __init__(self, head_dim, rope_theta=10000.0, device=None):
        super().__init__()
        inv = 1.0 / (rope_theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float().to(device) / head_dim))
        self.register_buffer("inv_freq", inv, persistent=False)

    @torch.no_grad()
    def forward(self, x, position_ids):
        inv = self.inv_freq[None, :, None].float().expand(position_ids.shape[0], -1, 1).to(x.device)
        pos = position_ids[:, None, :].float()
        freqs = (inv @ pos).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1):
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


class HeadRMSNorm(nn.Module):
    """Qwen3's per-head q_norm / k_norm (RMSNorm over head_dim)."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x):
        dt = x.dtype
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * xf.to(dt)


class LlamaAttention(nn.Module):
    def __init__(self, config, layer_idx, qk_norm=False):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = config.head_dim
        self.num_key_value_groups = config.num_attention_heads // config.num_key_value_heads
        self.scaling = self.head_dim ** -0.5
        bias = config.attention_bias
        # nn.Linear modules whose one-row (decode-step) products run on wgkv_gemv
        self.q_proj = model_ops.Linear(config.hidden_size, config.num_attention_heads * self.head_dim, bias=bias)
        self.k_proj = model_ops.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim, bias=bias)
        self.v_proj = model_ops.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim, bias=bias)
        self.o_proj = model_ops.Linear(config.num_attention_heads * self.head_dim, config.hidden_size, bias=bias)
        self.qk_norm = qk_norm
        if qk_norm:
            self.q_norm = HeadRMSNorm(self.head_dim)
            self.k_norm = HeadRMSNorm(self.head_dim)
        if not config.use_baseline and config.g_expand != 0.0:
            self.g_predictors = GatingPredictor(self.head_dim, config.num_key_value_heads, config.g_inputs,
                                                config.g_act_fn, config.g_expand, config.g_epsilon,
                                                config.g_rms, config.g_fast_path)
        # swap points (src/modeling_llama.py:240-250)
        self.self_attn_forward_patch = layers.self_attn_forward_patch
        self.prefill_wrapper = layers.prefill_wrapper
        self.decode_wrapper = layers.decode_wrapper
        self.prefill_kernel = torch_ops.sparse_attn_func  # torch.ops.wgkv.sparse_attn
        self.chunk_prefill_kernel = ops.chunk_attend  # prompt chunks after the first (no reference counterpart)
        self.decode_kernel_handle = torch_ops.paged_decode_attn_handle  # torch.ops.wgkv.paged_decode_attn
        self.decode_kernel_executor = lambda func: func()
        self._qkv_weight = None
        # a decode step's ring write done by the q/k/v projection's launch
        # where layers.ring_write_in_projection allows it
        self.ring_write_fused = True

    @torch.no_grad()
    def fuse_qkv(self):
        """Put q_proj, k_proj and v_proj's weights into one (Nq+2Nk, hidden)
        buffer (the parameters become views of it, names and values kept), so
        the forward projects q, k and v with one GEMM.  Not for biased
        projections."""
        if self._qkv_weight is not None or self.q_proj.bias is not None:
            return
        w = torch.cat([self.q_proj.weight, self.k_proj.weight, self.v_proj.weight], dim=0)
        nq, nk = self.q_proj.weight.shape[0], self.k_proj.weight.shape[0]
        self.q_proj.weight = nn.Parameter(w[:nq], requires_grad=False)
        self.k_proj.weight = nn.Parameter(w[nq:nq + nk], requires_grad=False)
        self.v_proj.weight = nn.Parameter(w[nq + nk:], requires_grad=False)
        self._qkv_weight = w

    def forward(self, gating_mode, hidden_states, position_embeddings, attention_mask=None, past_key_value=None,
                cache_position=None, input_norm=None, **kwargs):
        """input_norm (optional): the decoder's input RMSNorm module, applied
        to hidden_states here; a decode step's single row then takes the
        norm, the q/k/v product and RoPE in one launch (wgkv_gemv_ex)."""
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        cos, sin = position_embeddings
        w = self._qkv_weight
        nw = input_norm.weight if input_norm is not None else None
        if (w is not None and w.device == hidden_states.device and not self.qk_norm and cos.dim() == 3
                and model_ops.qkv_rope_usable(hidden_states, w, cos, sin, nw)):
            Hq, Hkv = self.config.num_attention_heads, self.config.num_key_value_heads
            c = past_key_value
            ring = None
            if self.ring_write_fused and layers.ring_write_in_projection(self, c):
                ring = (c, self.layer_idx, c.cache_seqlens[self.layer_idx][0])
            buf, kraw = model_ops.qkv_rope(hidden_states, w, cos, sin, Hq, Hkv, self.head_dim, nw,
                                           input_norm.eps if input_norm is not None else 1e-5, ring=ring)
            if ring is not None or getattr(c, "ring_written_by", None) is not None:
                c.ring_written_by = self.layer_idx if ring is not None else None
            q = buf[:, :, :Hq].transpose(1, 2)
            k = buf[:, :, Hq:Hq + Hkv].transpose(1, 2)
            v = buf[:, :, Hq + Hkv:].transpose(1, 2)
            pre_key = kraw.transpose(1, 2) if "pre_k" in self.config.g_inputs else None
            out, attn_weights, g_scores = self.self_attn_forward_patch(
                self, gating_mode, attention_mask, past_key_value, input_shape, q, pre_key, k, v)
            out = out.reshape(*input_shape, -1).to(hidden_states.dtype).contiguous()
            return self.o_proj(out), attn_weights, g_scores
        qkv = None
        if (input_norm is not None and w is not None and w.device == hidden_states.device
                and model_ops.rms_norm_linear_usable(hidden_states, input_norm.weight, w)):
            # a decode row without the fused RoPE (Qwen3's q/k norms sit between
            # the product and RoPE): the input norm as the product's prologue
            qkv, _ = model_ops.rms_norm_linear(hidden_states, input_norm.weight, input_norm.eps, w)
        elif input_norm is not None:
            hidden_states = input_norm(hidden_states)
        if self._qkv_weight is not None and self._qkv_weight.device == hidden_states.device:
            nq, nk = self.q_proj.weight.shape[0], self.k_proj.weight.shape[0]
            if qkv is None:
                qkv = model_ops.linear(hidden_states, self._qkv_weight)
            q = qkv[..., :nq].view(hidden_shape)
            k = qkv[..., nq:nq + nk].view(hidden_shape)
            v_src = qkv[..., nq + nk:]
        else:
            q = self.q_proj(hidden_states).view(hidden_shape)
            k = self.k_proj(hidden_states).view(hidden_shape)
            v_src = None
        v = (v_src if v_src is not None else self.v_proj(hidden_states)).view(hidden_shape)
        fused_rope = (model_ops.usable(q, k, v, cos, sin) and self.head_dim % 16 == 0 and q.stride(3) == 1
                      and k.stride(3) == 1 and v.stride(3) == 1 and cos.dim() == 3)
        # Qwen3's head norms go into the RoPE launch when its weights are bf16
        fused_norm = (self.qk_norm and fused_rope and self.head_dim <= 256
                      and model_ops.usable(self.q_norm.weight, self.k_norm.weight)
                      and self.q_norm.eps == self.k_norm.eps)
        if self.qk_norm and not fused_norm:
            q, k = self.q_norm(q), self.k_norm(k)
        q = q.transpose(1, 2)
        k = k.transpose(1, 2)
        v = v.transpose(1, 2)
        pre_key = k if "pre_k" in self.config.g_inputs else None
        c = past_key_value
        ring = None
        if (fused_rope and input_shape.numel() == 1 and self.ring_write_fused
                and layers.ring_write_in_projection(self, c)):
            # a decode row: the rotation's launch also writes the ring slot
            ring = (c, self.layer_idx, c.cache_seqlens[self.layer_idx][0])
        if fused_norm:
            # one launch: per-head norms, then the rotation; the normalised,
            # unrotated k is the gate's pre-RoPE key (modeling_qwen3.py:235-239)
            q, k, v, kn = model_ops.rope_qkv(q, k, v, cos, sin, self.q_norm.weight, self.k_norm.weight,
                                             self.q_norm.eps, ring=ring)
            pre_key = kn if "pre_k" in self.config.g_inputs else None
        elif fused_rope:
            # one launch, the same bf16 rounding; v copied beside k
            q, k, v = model_ops.rope_qkv(q, k, v, cos, sin, ring=ring)
        else:
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
        if ring is not None or getattr(c, "ring_written_by", None) is not None:
            c.ring_written_by = self.layer_idx if ring is not None else None
        out, attn_weights, g_scores = self.self_attn_forward_patch(
            self, gating_mode, attention_mask, past_key_value, input_shape, q, pre_key, k, v)
        out = out.reshape(*input_shape, -1).to(hidden_states.dtype).contiguous()
        return self.o_proj(out), attn_weights, g_scores
