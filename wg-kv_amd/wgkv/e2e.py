"""A minimal Llama decoder stack around the write-gated path, for end-to-end
runs (the reference's scripts/profiling.py:198-420).

Embedding, RMSNorm, the gated attention layer (``wgkv.attention.LlamaAttention``
with its swap points), SwiGLU MLP and LM head, random-initialised in bf16 on
the device; the dense projections of a prompt are torch GEMMs (hipBLASLt), a
decode step's one-row products run on wgkv_gemv (with the SwiGLU product and
the residual adds fused).  The prompt is
prefilled in chunks through the cache's chunk continuation and then decoded
greedily, as profiling.py does (argmax of the last logits, :146-147).  The
"full" run admits every token -- ``use_baseline`` (src/modeling_layers.py:1556)
or the reference's README recipe, g_expand 0 with random_sparsity 0.0 -- so
the same kernels compute dense causal attention over the whole prefix.

Reported as profiling.py reports (:395-410): prefill time and throughput,
average tokens per (layer, head) in the cache before and after decoding
(next_free_block * block_size / (L * Hkv), :150-153), decode time per token,
model and KV-cache memory (:165-186).
"""
import math
import time
from dataclasses import dataclass, field
from typing import List

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import model_ops
from .attention import LlamaAttention, LlamaRotaryEmbedding
from .cache import DualCache
from .layers import WGKVConfig


class RMSNorm(nn.Module):
    def __init__(self, hidden, eps=1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden))
        self.eps = eps

    def forward(self, x, residual=None):
        """RMSNorm of x (+ residual); with a residual returns (out, x + residual).
        bf16 on the GPU: one fused launch (wgkv_rms_norm)."""
        if model_ops.usable(x, self.weight) and x.shape[-1] % 8 == 0 and x.shape[-1] <= 8192:
            out, h = model_ops.rms_norm(x, self.weight, self.eps, residual)
            return out if residual is None else (out, h)
        if residual is not None:
            x = x + residual
        dt = x.dtype
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        out = self.weight * xf.to(dt)
        return out if residual is None else (out, x)


class MLP(nn.Module):
    def __init__(self, hidden, inter):
        super().__init__()
        self.gate_proj = model_ops.Linear(hidden, inter, bias=False)
        self.up_proj = model_ops.Linear(hidden, inter, bias=False)
        self.down_proj = model_ops.Linear(inter, hidden, bias=False)
        self._gate_up = None

    @torch.no_grad()
    def fuse_gate_up(self):
        """Put gate_proj and up_proj's weights into one (2*inter, hidden)
        buffer (the parameters become views of it, names and values kept), for
        the one-launch SwiGLU product of a decode step."""
        if self._gate_up is not None:
            return
        w = torch.cat([self.gate_proj.weight, self.up_proj.weight], dim=0)
        n = self.gate_proj.weight.shape[0]
        self.gate_proj.weight = nn.Parameter(w[:n], requires_grad=False)
        self.up_proj.weight = nn.Parameter(w[n:], requires_grad=False)
        self._gate_up = w

    def forward(self, x, residual=None, norm=None):
        """down(silu(gate(x)) * up(x)) (+ residual, the decoder's add after
        the MLP).  A decode step's row: two launches (the stacked gate/up
        product with SwiGLU, the down product with the residual add).  With
        norm (the post-attention RMSNorm) x is the attention output and the
        MLP's input is norm(x + residual), whose sum is also the residual the
        down product adds; for a decode row the norm and the add run in the
        workgroups of the gate/up product, bit for bit the separate norm."""
        gu = self._gate_up
        if norm is not None:
            if (gu is not None and gu.device == x.device and residual is not None
                    and model_ops.rms_norm_linear_usable(x, norm.weight, gu, residual)):
                act, h = model_ops.rms_norm_linear(x, norm.weight, norm.eps, gu, residual=residual, mode=2)
                return model_ops.linear(act, self.down_proj.weight, residual=h)
            if residual is None:
                x = norm(x)
            else:
                x, residual = norm(x, residual=residual)
        if gu is not None and gu.device == x.device and model_ops.gemv_usable(x, gu):
            return model_ops.linear(model_ops.swiglu_linear(x, gu), self.down_proj.weight, residual=residual)
        # prompts: one GEMM for gate and up (hipBLASLt at 4096 rows: 635 us
        # against 2 x 365 us), then the fused SwiGLU product of its halves
        if gu is not None and gu.device == x.device:
            n = gu.shape[0] // 2
            gup = F.linear(x, gu)
            g, u = gup[..., :n], gup[..., n:]
        else:
            g, u = self.gate_proj(x), self.up_proj(x)
        if model_ops.usable(g, u) and g.shape[-1] % 8 == 0 and g.stride(-1) == 1 and u.stride(-1) == 1:
            out = self.down_proj(model_ops.silu_mul(g, u))
        else:
            out = self.down_proj(F.silu(g) * u)
        return out if residual is None else residual + out


class DecoderLayer(nn.Module):
    def __init__(self, cfg, idx, inter, qk_norm=False):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size)
        self.self_attn = LlamaAttention(cfg, idx, qk_norm=qk_norm)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size)
        self.mlp = MLP(cfg.hidden_size, inter)
        # a decode row's post-attention norm runs inside the MLP's first
        # product; off when a timer must see it with the attention
        self.post_norm_in_mlp = True

    def rmsnorm_and_self_attn(self, x, pos_emb, cache):
        """Input norm, attention, residual add and the post-attention norm
        (src/modeling_llama.py:337-371): returns (residual, MLP input).  The
        attention module applies the input norm (for a decode step fused with
        the q/k/v product and RoPE)."""
        h, _, _ = self.self_attn(3, x, pos_emb, None, cache, input_norm=self.input_layernorm)
        mlp_in, x = self.post_attention_layernorm(h, residual=x)  # residual add fused into the norm
        return x, mlp_in

    def forward(self, x, pos_emb, cache):
        if self.post_norm_in_mlp and x.numel() == x.shape[-1]:
            h, _, _ = self.self_attn(3, x, pos_emb, None, cache, input_norm=self.input_layernorm)
            return self.mlp(h, residual=x, norm=self.post_attention_layernorm)
        residual, h = self.rmsnorm_and_self_attn(x, pos_emb, cache)
        return self.mlp(h, residual=residual)  # residual + mlp(h)


@dataclass
class E2EConfig:
    """Llama-3.1-8B shapes (hidden 4096, FFN 14336, 32 layers, 32 q / 8 KV
    heads, vocab 128256, rope_theta 500000) and the run's cache settings."""
    hidden_size: int = 4096
    intermediate_size: int = 14336
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    vocab_size: int = 128256
    rope_theta: float = 500000.0
    local_window_size: int = 1024
    g_threshold: float = 0.1
    qk_norm: bool = False
    g_expand: float = 4.0
    # deferred gating, as the reference's profiling harness forces
    # (scripts/profiling.py:212-213): decode steps store the pre-RoPE key and
    # re-gate the whole window when its last slot is written
    g_defer: bool = True

    @staticmethod
    def qwen3_8b(**kw):
        """Qwen3-8B shapes: 36 layers, FFN 12288, vocab 151936, rope_theta 1e6,
        per-head q/k norms and gate width g_expand = 1.5
        (src/configuration_qwen3.py:183)."""
        base = dict(intermediate_size=12288, num_hidden_layers=36, vocab_size=151936, rope_theta=1000000.0,
                    qk_norm=True, g_expand=1.5)
        base.update(kw)
        return E2EConfig(**base)


class LlamaLite(nn.Module):
    def __init__(self, ec: E2EConfig, gated: bool, max_tokens_per_head: int, max_total_tokens: int):
        super().__init__()
        self.ec = ec
        self.cfg = WGKVConfig(hidden_size=ec.hidden_size, num_hidden_layers=ec.num_hidden_layers,
                              num_attention_heads=ec.num_attention_heads, num_key_value_heads=ec.num_key_value_heads,
                              rope_theta=ec.rope_theta, local_window_size=ec.local_window_size,
                              g_threshold=ec.g_threshold, g_expand=ec.g_expand, g_defer=ec.g_defer,
                              use_baseline=not gated,
                              max_tokens_per_head=max_tokens_per_head, max_total_tokens=max_total_tokens,
                              check_capacity=False)
        self.embed_tokens = nn.Embedding(ec.vocab_size, ec.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(self.cfg, i, ec.intermediate_size, ec.qk_norm)
                                    for i in range(ec.num_hidden_layers))
        self.norm = RMSNorm(ec.hidden_size)
        self.lm_head = model_ops.Linear(ec.hidden_size, ec.vocab_size, bias=False)
        self.rotary_emb = LlamaRotaryEmbedding(self.cfg.head_dim, ec.rope_theta)
        for layer in self.layers:  # q, k, v (and gate, up) projected by one product each
            layer.self_attn.fuse_qkv()
            layer.mlp.fuse_gate_up()

    @torch.no_grad()
    def init_weights(self, seed=0, std=0.02):
        """N(0, std) projections and embeddings, unit norms; the gates keep
        the reference's default Conv1d init (src/modeling_layers.py:163-168)."""
        g = torch.Generator(device=self.lm_head.weight.device).manual_seed(seed)
        for name, p in self.named_parameters():
            if "g_predictors" in name or name.endswith("norm.weight"):
                continue
            p.normal_(0.0, std, generator=g)

    @torch.no_grad()
    def forward_tokens(self, ids, start, cache):
        """ids (1, n) at positions start..start+n-1 -> logits of the last token."""
        pos = torch.arange(start, start + ids.shape[1], device=ids.device)[None]
        return self.forward_at(ids, pos, cache)

    @torch.no_grad()
    def forward_at(self, ids, pos, cache):
        """ids (1, n) at the positions of the device tensor pos (1, n)."""
        x = self.embed_tokens(ids)
        pe = self.rotary_emb(x, pos)
        for layer in self.layers:
            x = layer(x, pe, cache)
        return self.lm_head(self.norm(x[:, -1:]))


def greedy_token(logits):
    """argmax over the vocabulary of logits (1, 1, V) -> (1, 1) int64, in two
    single-workgroup reductions (rows of V/128, then the 128 row maxima) so
    that no multi-workgroup reduction (which clears its semaphores with a
    memset) is recorded into a captured graph.  Ties resolve to the lowest
    index, as torch.argmax does."""
    V = logits.shape[-1]
    flat = logits.reshape(-1)
    if V % 128:
        return torch.argmax(flat).view(1, 1)
    vals, idx = flat.view(128, V // 128).max(dim=1)
    r = torch.argmax(vals).view(1)
    return (r * (V // 128) + torch.gather(idx, 0, r)).view(1, 1)  # no host read of r


class GraphDecoder:
    """One greedy decode step of the whole model (every layer, the LM head
    and the argmax) captured in a HIP graph and replayed.  The cache runs on
    its device ring pointers; the token and the position live in device
    tensors the step itself advances.  The ring must already be full (any
    prompt of at least W tokens).  With deferred gating every layer's window
    is re-gated after the steps that write the ring's last slot: a second
    captured graph (the re-gate of all layers) is replayed after those steps
    only, which the host knows from its mirror of the ring pointers, so the
    other steps launch no re-gate at all."""

    def __init__(self, model, cache, token, pos, warmup=2):
        dev = token.device
        self.model, self.cache = model, cache
        self.tok = token.clone().view(1, 1)
        self.pos = torch.tensor([[pos]], dtype=torch.int64, device=dev)
        if cache.local_length != cache.local_window_size:
            raise AssertionError("graph decode needs a full ring")
        cfg = model.cfg
        # decode steps carry no admission mask (and re-gate the window) with
        # deferred gating, unless every token is admitted (use_baseline)
        self.regate = (bool(cfg.g_defer) and not cfg.use_baseline
                       and (cfg.random_sparsity is not None or cfg.g_expand != 0.0))
        cache.use_device_ring(True)
        cache.refresh_by_caller = self.regate
        self.attn = [layer.self_attn for layer in model.layers]
        if self.regate and cfg.random_sparsity is None:
            for attn in self.attn:  # the gates' packed weights exist before any capture
                gp = attn.g_predictors
                if cache.block_pool_k.dtype == torch.bfloat16:
                    gp.packed_weights(gp.precision(torch.bfloat16))
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):  # real decode steps: workspaces and library state before capture
                wrote_last = self._writes_last_slot()
                self._step()
                if wrote_last:
                    self._regate()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.warm_tokens = warmup
        host = (cache.local_ptr, cache.local_length)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._step()
        cache.local_ptr, cache.local_length = host  # capture ran the host side once, the device side not
        self.regate_graph = None
        if self.regate:
            self.regate_graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.regate_graph):
                self._regate()

    def _writes_last_slot(self):
        c = self.cache
        insert = c.local_length if c.local_length < c.local_window_size else c.local_ptr
        return self.regate and insert == c.local_window_size - 1

    def _regate(self):
        from .layers import refresh_windows
        refresh_windows(self.attn, self.cache, self.tok.device)

    def _step(self):
        logits = self.model.forward_at(self.tok, self.pos, self.cache)
        self.tok.copy_(greedy_token(logits))
        self.pos += 1
        return logits

    def step(self):
        """Replay one step (and, after a step that wrote the ring's last slot,
        the windows' re-gate); returns the (device) token it produced."""
        wrote_last = self._writes_last_slot()
        self.graph.replay()
        if wrote_last:
            self.regate_graph.replay()
        self.cache.advance_host_ring()
        return self.tok


def calibrate_gates(model, ids, frac, chunk=4096):
    """Shift each layer's conv2.bias per head so that about ``frac`` of the
    first ``chunk`` prompt tokens score above the threshold: logit(tau) minus
    the (1-frac) quantile of that head's pre-sigmoid logits, taken layer by
    layer on the activations the earlier (already shifted) layers produce."""
    tau = model.cfg.g_threshold
    shift_to = math.log(tau / (1.0 - tau))
    originals = []
    for layer in model.layers:
        gp = layer.self_attn.g_predictors
        orig = gp.scores_and_mask

        def calibrated(pre_key, post_key, value, threshold, _gp=gp, _orig=orig, **kw):
            s, _ = _orig(pre_key, post_key, value, 0.5)
            sd = s[0].double().clamp(1e-12, 1 - 1e-12)
            logit = torch.log(sd) - torch.log1p(-sd)
            with torch.no_grad():
                for h in range(logit.shape[0]):
                    q = torch.quantile(logit[h].float(), 1.0 - frac).item()
                    _gp.conv2.bias[h] += shift_to - q
            return _orig(pre_key, post_key, value, threshold, **kw)

        gp.scores_and_mask = calibrated
        originals.append((gp, orig))
    cache = DualCache()
    model.forward_tokens(ids[:, :chunk], 0, cache)
    for gp, orig in originals:
        gp.scores_and_mask = orig
    del cache


GRANULARITIES = ("rms_linear_attn", "linear_attn", "attn", "wrapper", "kernel", "predictor")


class PhaseTimers:
    """Accumulated attention / MLP / LM-head time (ms) per phase, as
    profiling.py's ElapsedTimeTracker / TimingPhase pair (:8-13, :241-268).
    ``phase`` is "warmup", "prefill" or "decode"; nothing is recorded in
    the warm-up phase."""

    def __init__(self, granularity):
        self.granularity = granularity
        self.phase = "warmup"
        self.ms = {(part, ph): 0.0 for part in ("attn", "mlp", "lm_head") for ph in ("prefill", "decode")}

    def timed(self, part, func):
        """func wrapped as profiling.py's get_func_with_timing (:186-194):
        synchronise, record, call, record, synchronise (measure_time,
        :113-120), and add the time to the tracker of the current phase."""
        events = []

        def wrapper(*args, **kwargs):
            if self.phase not in ("prefill", "decode"):
                return func(*args, **kwargs)
            if not events:
                events.extend(torch.cuda.Event(enable_timing=True) for _ in range(2))
            start, end = events
            torch.cuda.synchronize()
            start.record()
            out = func(*args, **kwargs)
            end.record()
            torch.cuda.synchronize()
            self.ms[(part, self.phase)] += start.elapsed_time(end)
            return out
        return wrapper

    def report(self):
        """The lines profiling.py prints for --profile_attn_mlp (:411-417)."""
        return {f"{ph}_{part}_ms": round(v, 3) for (part, ph), v in self.ms.items()}


def install_timing(model, granularity="kernel"):
    """Wrap, in every layer, the function that the reference's
    ``--attn_granularity`` names (profiling.py:273-334) plus the MLP and the
    LM head (:336-343), each with a HIP-event timer; returns the timers.
    ``kernel`` also wraps ``chunk_prefill_kernel``, the attention of prompt
    chunks after the first; ``predictor`` wraps the gate's fused
    score-and-admit call, which is what this build's layer calls for the
    predictor.  The timers synchronise
    around every call, so they are for eager runs (not captured graphs)."""
    if granularity not in GRANULARITIES:
        raise ValueError(f"granularity must be one of {GRANULARITIES}")
    t = PhaseTimers(granularity)
    for layer in model.layers:
        a = layer.self_attn
        if granularity == "rms_linear_attn":
            layer.post_norm_in_mlp = False
            layer.rmsnorm_and_self_attn = t.timed("attn", layer.rmsnorm_and_self_attn)
        elif granularity == "linear_attn":
            a.forward = t.timed("attn", a.forward)
        elif granularity == "attn":
            a.self_attn_forward_patch = t.timed("attn", a.self_attn_forward_patch)
        elif granularity == "wrapper":
            a.prefill_wrapper = t.timed("attn", a.prefill_wrapper)
            a.decode_wrapper = t.timed("attn", a.decode_wrapper)
        elif granularity == "kernel":
            a.prefill_kernel = t.timed("attn", a.prefill_kernel)
            a.chunk_prefill_kernel = t.timed("attn", a.chunk_prefill_kernel)
            a.decode_kernel_executor = t.timed("attn", a.decode_kernel_executor)
        else:
            gp = getattr(a, "g_predictors", None)
            if gp is not None:
                gp.scores_and_mask = t.timed("attn", gp.scores_and_mask)
        layer.mlp.forward = t.timed("mlp", layer.mlp.forward)
    model.lm_head.forward = t.timed("lm_head", model.lm_head.forward)
    return t


@dataclass
class E2EResult:
    prompt_length: int
    prefill_ms: float
    decode_ms: List[float] = field(default_factory=list)
    tokens_before: float = 0.0
    tokens_after: float = 0.0
    model_mib: float = 0.0
    kv_mib: float = 0.0
    tokens: List[int] = field(default_factory=list)


def avg_tokens_in_cache(cache, model):
    """profiling.py:150-153."""
    return cache.next_free_block * model.cfg.block_size / (model.cfg.num_hidden_layers * model.cfg.num_key_value_heads)


def kv_cache_mib(cache):
    """profiling.py:180-186: the block table plus the used share of the pools."""
    ratio = cache.next_free_block / cache.total_blocks
    b = cache.block_table.numel() * 4 + (cache.block_pool_k.numel() + cache.block_pool_v.numel()) * 2 * ratio
    return b / (1024 * 1024)


def prompt_chunks(S, chunk, W):
    """[start, end) spans of a prompt of S tokens fed in chunks: every chunk
    after the first must start at a multiple of 64 and hold at least W
    tokens, so ``chunk`` must be a multiple of 64 and at least W, and a tail
    shorter than W joins the chunk before it.  Checked before any prefill
    work starts."""
    if chunk % 64 or chunk < W:
        raise ValueError(f"prompt chunks must be a multiple of 64 and at least W={W} tokens (got {chunk})")
    spans = [[c0, min(c0 + chunk, S)] for c0 in range(0, S, chunk)]
    if len(spans) > 1 and spans[-1][1] - spans[-1][0] < W:
        tail = spans.pop()
        spans[-1][1] = tail[1]
    return [tuple(sp) for sp in spans]


@torch.no_grad()
def run(model, ids, steps, chunk=4096, warmup_steps=2, progress=None, graph=False, timers=None):
    """Chunked prefill of ids (1, S), then ``steps`` greedy decode steps, each
    timed with HIP events on the launch stream after a synchronisation (as
    profiling.py's measure_time, :113-120); with ``graph`` every step is a
    replay of a captured HIP graph (GraphDecoder).  ``timers`` (from
    ``install_timing``) is switched to the phase being run."""
    if timers is not None and graph:
        raise ValueError("per-granularity timers synchronise around each call; use an eager run")
    phase = (lambda name: setattr(timers, "phase", name)) if timers is not None else (lambda name: None)
    S = ids.shape[1]
    spans = prompt_chunks(S, chunk, model.cfg.local_window_size)
    cache = DualCache()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    phase("prefill")
    ev0.record()
    logits = None
    for n, (c0, c1) in enumerate(spans):
        logits = model.forward_tokens(ids[:, c0:c1], c0, cache)
        if progress is not None and n % 16 == 0:
            progress(f"prefill chunk {n + 1}/{len(spans)}")
    ev1.record()
    torch.cuda.synchronize()
    res = E2EResult(prompt_length=S, prefill_ms=ev0.elapsed_time(ev1))
    cache.raise_if_failed("prefill")
    res.tokens_before = avg_tokens_in_cache(cache, model)
    tok = greedy_token(logits)
    pos = S
    gd = None
    if graph:
        gd = GraphDecoder(model, cache, tok, pos)
        warmup_steps = max(0, warmup_steps - gd.warm_tokens)
    for i in range(warmup_steps + steps):
        phase("decode" if i >= warmup_steps else "warmup")
        torch.cuda.synchronize()
        ev0.record()
        if gd is not None:
            tok = gd.step()
        else:
            logits = model.forward_tokens(tok, pos, cache)
            tok = greedy_token(logits)
        ev1.record()
        torch.cuda.synchronize()
        if i >= warmup_steps:
            res.decode_ms.append(ev0.elapsed_time(ev1))
            res.tokens.append(int(tok.item()))
        pos += 1
    phase("warmup")
    cache.raise_if_failed("decode")
    res.tokens_after = avg_tokens_in_cache(cache, model)
    res.model_mib = sum(p.numel() * p.element_size() for p in model.parameters()) / (1024 * 1024)
    res.kv_mib = kv_cache_mib(cache)
    del cache
    return res
