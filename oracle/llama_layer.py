"""One write-gated Llama attention layer on the CPU (the config-1 path).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restates, in float32 on the CPU:
* LlamaAttention.forward for gating_mode 3 -- src/modeling_llama.py:252-287
  (projections, pre-RoPE key, RoPE :81-146, o_proj), and Qwen3's variant
  with per-head q/k norms before the pre-RoPE key (src/modeling_qwen3.py:
  235-239; ``qk_norm=True``);
* self_attn_forward_patch / _inference -- src/modeling_layers.py:1534-1629,
  :1452-1509 (gate, threshold, migration trigger, prefill/decode dispatch);
* the cache through ``oracle.dualcache``, the gate through ``oracle.gate``,
  the prefill attention through the ideal mask of utils/test_sparse_attn.py
  (``oracle.meta`` + ``oracle.attention.masked_prefill``) and the decode
  attention through ``oracle.attention.paged_decode``.

Weights come in as a dict with the reference's names
(``q_proj.weight`` ... ``o_proj.weight`` and the gate's
``g_predictors.*``).  This is also the CPU baseline timed by bench.py (``kv_dtype=float32``: the
reference's fp32 CPU path).  With ``kv_dtype=bfloat16`` q/k/v are rounded to
bf16 after gating, as on the GPU, whose attention kernels (like the
reference's) are bf16-only.
"""
import torch

from . import attention, gate, meta
from .dualcache import DualCacheOracle


def rope_cos_sin(positions, head_dim, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = positions.float()[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def head_rms_norm(x, weight, eps=1e-6):
    """Qwen3RMSNorm over the last dimension (src/modeling_qwen3.py:62-76):
    fp32 normalisation, cast back to the input dtype, then the weight; applied
    per head to q and k (:235-236)."""
    dt = x.dtype
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(dt)


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class OracleLayer:
    def __init__(self, weights, hidden, Hq, Hkv, D, W, max_tokens_per_head, threshold=0.1, g_defer=False,
                 theta=10000.0, page=16, kv_dtype=torch.float32, qk_norm=False):
        self.w = {k: v.float() for k, v in weights.items()}
        self.gp = {k[len("g_predictors."):]: v for k, v in self.w.items() if k.startswith("g_predictors.")}
        self.hidden, self.Hq, self.Hkv, self.D, self.W = hidden, Hq, Hkv, D, W
        self.G = Hq // Hkv
        self.threshold = threshold
        self.g_defer = g_defer
        self.theta = theta
        self.kv_dtype = kv_dtype
        self.qk_norm = qk_norm
        self.cache = DualCacheOracle(1, Hkv, D, W, Hkv * max_tokens_per_head, max_tokens_per_head,
                                     block_size=page, g_defer=g_defer, dtype=kv_dtype)

    def _project(self, x, positions):
        S = x.shape[1]
        q = (x @ self.w["q_proj.weight"].T).view(1, S, self.Hq, self.D)
        k = (x @ self.w["k_proj.weight"].T).view(1, S, self.Hkv, self.D)
        if self.qk_norm:  # Qwen3: per-head norms before the pre-RoPE key is taken
            q = head_rms_norm(q, self.w["q_norm.weight"])
            k = head_rms_norm(k, self.w["k_norm.weight"])
        q, k = q.transpose(1, 2), k.transpose(1, 2)
        v = (x @ self.w["v_proj.weight"].T).view(1, S, self.Hkv, self.D).transpose(1, 2)
        pre_k = k
        cos, sin = rope_cos_sin(positions, self.D, self.theta)
        q = q * cos + rotate_half(q) * sin
        k = k * cos + rotate_half(k) * sin
        return q, pre_k, k, v

    def _regate(self, layer, pk, k, v):
        s = gate.gate_scores(pk[None], k[None], v[None], self.gp)
        return s[0] > self.threshold

    def prefill(self, x, positions):
        """x (1, S, hidden) float32 -> (out (1, S, hidden), g_mask (Hkv, S))."""
        S = x.shape[1]
        q, pre_k, k, v = self._project(x, positions)
        g = gate.gate_scores(pre_k, k, v, self.gp)
        mask = g > self.threshold
        dt = self.kv_dtype
        kb, vb, qb = k.to(dt), v.to(dt), q.to(dt)
        self.cache.prefill(0, kb[0], vb[0], mask[0], pre_key=pre_k.to(dt)[0])
        attn = attention.masked_prefill(qb, kb, vb, meta.ideal_mask(mask.numpy(), self.W, self.G)).float()
        out = attn.transpose(1, 2).reshape(1, S, self.Hq * self.D) @ self.w["o_proj.weight"].T
        return out, mask[0], g[0]

    def decode(self, x, position):
        """x (1, 1, hidden) -> (out (1, 1, hidden), g_mask (Hkv,) or None)."""
        q, pre_k, k, v = self._project(x, torch.tensor([position]))
        mask = None
        g = None
        if not self.g_defer:
            g = gate.gate_scores(pre_k, k, v, self.gp)
            mask = (g > self.threshold)[0, :, 0]
        dt = self.kv_dtype
        sl, bt = self.cache.decode(0, k.to(dt)[0, :, 0], v.to(dt)[0, :, 0], mask,
                                   pre_key=pre_k.to(dt)[0, :, 0], regate=self._regate)
        attn = attention.paged_decode(q.transpose(1, 2).to(dt),
                                      self.cache.block_pool_k.view(-1, self.cache.P, self.D),
                                      self.cache.block_pool_v.view(-1, self.cache.P, self.D),
                                      sl[None], bt[None], self.D ** -0.5)
        out = attn.reshape(1, 1, self.Hq * self.D) @ self.w["o_proj.weight"].T
        return out, mask, None if g is None else g[0, :, 0]
