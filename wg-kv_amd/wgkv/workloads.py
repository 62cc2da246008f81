"""Synthetic decode workloads at the shapes the benchmarks are quoted on.

* ``decode_beta``   -- batch B, per-KV-head admitted count
  ``round(f * (ctx - W))`` with ``f ~ Beta(2, 8)`` (mean 20 %), plus the
  full local window W; Llama-3.1-8B head shapes.
* ``decode_ragged`` -- per (sequence, head) fraction ``f ~ U[lo, hi]``
  independently, same token count rule.

The physical pages of all heads are a random permutation of the pool (as the
reference's decode benchmark does, utils/benchmark_decode.py:72-77); K/V and
q are N(0,1) bf16.  Everything is generated on ``device`` from a seeded
generator.
"""
from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class DecodeWorkload:
    q: torch.Tensor            # (B, 1, Hq, D) bf16
    k_cache: torch.Tensor      # (num_pages, page, D) bf16
    v_cache: torch.Tensor
    cache_seqlens: torch.Tensor  # (B, Hkv) int32
    block_table: torch.Tensor    # (B, Hkv, max_pages) int32, -1 past the end
    softmax_scale: float
    name: str

    @property
    def total_tokens(self):
        return int(self.cache_seqlens.sum().item())

    def algorithmic_bytes(self):
        """K+V rows read, page-table entries read, q read and out written."""
        B, _, Hq, D = self.q.shape
        page = self.k_cache.shape[1]
        sl = self.cache_seqlens.to(torch.int64)
        kv = int(sl.sum().item()) * D * 2 * 2
        table = int(((sl + page - 1) // page).sum().item()) * 4
        return kv + table + 2 * B * Hq * D * 2 + 4 * sl.numel()


def _build(seqlens, Hq, D, page, device, seed, name):
    B, Hkv = seqlens.shape
    pages = (seqlens + page - 1) // page
    total = int(pages.sum())
    max_pages = int(pages.max())
    g = torch.Generator(device="cpu").manual_seed(seed)
    perm = torch.randperm(total, generator=g).to(torch.int32)
    table = torch.full((B, Hkv, max_pages), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        for h in range(Hkv):
            n = int(pages[b, h])
            table[b, h, :n] = perm[off:off + n]
            off += n
    gd = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(total, page, D, generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn(total, page, D, generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    q = torch.randn(B, 1, Hq, D, generator=gd, device=device, dtype=torch.float32).to(torch.bfloat16)
    return DecodeWorkload(q, k, v, torch.as_tensor(seqlens, dtype=torch.int32).to(device),
                          table.to(device), D ** -0.5, name)


def decode_beta(ctx=32768, batch=1, Hq=32, Hkv=8, D=128, window=1024, page=16, device="cuda", seed=0):
    rng = np.random.default_rng(seed)
    f = rng.beta(2.0, 8.0, size=(batch, Hkv))
    seqlens = window + np.rint(f * (ctx - window)).astype(np.int64)
    return _build(seqlens, Hq, D, page, device, seed, f"decode_beta_b{batch}_{ctx // 1024}k")


def decode_ragged(ctx=131072, batch=8, Hq=32, Hkv=8, D=128, window=1024, page=16,
                  lo=0.02, hi=0.60, device="cuda", seed=0):
    rng = np.random.default_rng(seed)
    f = rng.uniform(lo, hi, size=(batch, Hkv))
    seqlens = window + np.rint(f * (ctx - window)).astype(np.int64)
    return _build(seqlens, Hq, D, page, device, seed, f"decode_ragged_b{batch}_{ctx // 1024}k")


def config1_layer(seed=0, hidden=512, Hq=8, Hkv=2, D=64, S=2048, steps=32, W=128, frac=0.2, threshold=0.1,
                  g_defer=False, qk_norm=False, g_expand=4.0):
    """BASELINE config 1 on the host (CPU tensors): weights, prompt, decode inputs.

    torch.manual_seed(seed); q/k/v/o ~ N(0, 0.02); gate with the reference's
    default init (RMSNorm weights 1, Conv1d uniform), inner = 4*D; prompt
    x ~ N(0, 1) (1, S, hidden); ``steps`` decode inputs ~ N(0, 1) at explicit
    positions S, S+1, ...  ``conv2.bias[h]`` is shifted afterwards by
    logit(threshold) - q_{1-frac}(pre-sigmoid logits of head h over the prompt),
    so about ``frac`` of the prompt is admitted; that shift needs the gate's
    scores of the prompt, which the caller computes (``shift_gate_bias``).
    Returns (config kwargs, weights dict, prompt, decode inputs).
    """
    import math
    torch.manual_seed(seed)
    inner = int(D * g_expand)
    w = {
        "q_proj.weight": torch.randn(Hq * D, hidden) * 0.02,
        "k_proj.weight": torch.randn(Hkv * D, hidden) * 0.02,
        "v_proj.weight": torch.randn(Hkv * D, hidden) * 0.02,
        "o_proj.weight": torch.randn(hidden, Hq * D) * 0.02,
    }
    if qk_norm:  # Qwen3's per-head norms, weights near 1 so that they matter
        w["q_norm.weight"] = 1.0 + 0.1 * torch.randn(D)
        w["k_norm.weight"] = 1.0 + 0.1 * torch.randn(D)
    conv1 = torch.nn.Conv1d(Hkv * 2 * D, Hkv * inner, 1, groups=Hkv)
    conv2 = torch.nn.Conv1d(Hkv * inner, Hkv, 1, groups=Hkv)
    w["g_predictors.pre_key_norm.weight"] = torch.ones(D)
    w["g_predictors.post_key_norm.weight"] = torch.ones(D)
    w["g_predictors.conv1.weight"] = conv1.weight.detach().clone()
    w["g_predictors.conv1.bias"] = conv1.bias.detach().clone()
    w["g_predictors.conv2.weight"] = conv2.weight.detach().clone()
    w["g_predictors.conv2.bias"] = conv2.bias.detach().clone()
    x = torch.randn(1, S, hidden)
    xs = [torch.randn(1, 1, hidden) for _ in range(steps)]
    cfg = dict(hidden_size=hidden, num_hidden_layers=1, num_attention_heads=Hq, num_key_value_heads=Hkv,
               head_dim=D, local_window_size=W, block_size=16, max_tokens_per_head=S + steps + 2 * W,
               max_total_tokens=Hkv * (S + steps + 2 * W), g_threshold=threshold, g_defer=g_defer,
               g_fast_path=True, rope_theta=10000.0, g_expand=g_expand)
    cfg["_frac"] = frac
    cfg["_logit_threshold"] = math.log(threshold / (1 - threshold))
    return cfg, w, x, xs


def shift_gate_bias(weights, logits, frac, logit_threshold):
    """Shift conv2.bias[h] so that a fraction ``frac`` of the tokens of head h
    have logits above ``logit_threshold``; ``logits`` (Hkv, S) pre-sigmoid."""
    w = dict(weights)
    b = w["g_predictors.conv2.bias"].clone()
    for h in range(logits.shape[0]):
        qv = torch.quantile(logits[h].double(), 1.0 - frac).item()
        b[h] += float(logit_threshold - qv)
    w["g_predictors.conv2.bias"] = b
    return w


def visible_pairs(g_mask, local_window_size, bs=64):
    """Number of (query, key) pairs the sparse prefill evaluates, per KV head.

    Row i of block r sees keys j <= i that are admitted or lie in
    [r*bs - W + 1, i] (the vertical-slash ideal mask); computed in closed form
    from the admitted prefix counts.  g_mask (Hkv, S) bool on any device."""
    m = g_mask.to(torch.int64)
    H, S = m.shape
    cum = torch.cumsum(m, dim=1)                       # admitted in [0, j]
    i = torch.arange(S, device=m.device)
    start = torch.clamp((i // bs) * bs - local_window_size + 1, min=0)
    band = i - start + 1
    before = torch.where(start > 0, cum[:, (start - 1).clamp(min=0)], torch.zeros_like(cum[:, :1]))
    return (band[None, :] + before).sum(dim=1)        # (H,)


@dataclass
class PrefillWorkload:
    q: torch.Tensor        # (1, S, Hq, D) bf16
    k: torch.Tensor        # (1, S, Hkv, D) bf16 (post-RoPE)
    v: torch.Tensor
    pre_k: torch.Tensor    # (1, S, Hkv, D) bf16
    gate: object           # wgkv.gate.GatingPredictor on the device
    threshold: float
    local_window: int


def prefill_llama(S=32768, Hq=32, Hkv=8, D=128, W=1024, frac=0.2, threshold=0.1, device="cuda", seed=0,
                  gate_dtype=torch.bfloat16):
    """Config-4 shapes: bf16 q/k/v/pre-RoPE k ~ N(0,1) in (B, S, H, D) layout,
    a gate with the reference's default init whose conv2 bias is shifted per
    head so ~``frac`` of the prompt scores above ``threshold``.  The gate's
    parameters are bf16 by default, as the reference's profiling run loads
    them (scripts/profiling.py:222-226)."""
    import math
    from .gate import GatingPredictor
    g = torch.Generator(device=device).manual_seed(seed)

    def rn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)

    q, k, v, pk = rn(1, S, Hq, D), rn(1, S, Hkv, D), rn(1, S, Hkv, D), rn(1, S, Hkv, D)
    torch.manual_seed(seed)
    gate = GatingPredictor(D, Hkv, ["pre_k", "post_k"], "gelu", 4.0, 1e-3, True, True).to(device=device,
                                                                                         dtype=gate_dtype)
    scores, _ = gate.scores_and_mask(pk.transpose(1, 2), k.transpose(1, 2), None, 0.5)
    logit = torch.log(scores.double()) - torch.log1p(-scores.double())
    with torch.no_grad():
        for h in range(Hkv):
            qv = torch.quantile(logit[0, h].float(), 1.0 - frac).item()
            gate.conv2.bias[h] += math.log(threshold / (1 - threshold)) - qv
    return PrefillWorkload(q, k, v, pk, gate, threshold, W)
