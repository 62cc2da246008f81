"""Write-gated attention functions behind the reference's swap points.

The reference binds these as function attributes of its attention module
(src/modeling_llama.py:240-250) and calls them with an explicit ``self``:
``self_attn_forward_patch``, ``prefill_wrapper``, ``decode_wrapper``,
``prefill_kernel``, ``decode_kernel_handle``, ``decode_kernel_executor``.
Same names, signatures and call order here; the device work goes through the
HIP library (kernels (1)-(4)).  ``self`` needs ``config``, ``layer_idx``,
``head_dim``, ``scaling``, ``num_key_value_groups`` and the attributes above
(and ``g_predictors`` when the gate is learned).

Only inference (gating_mode 3) is on the hot path.  Of the comparison
baselines, QUEST page selection (``use_quest``) and SnapKV eviction
(``snapkv_enabled``, scored, selected and packed by device kernels) run on
the same page tables; the training
modes, DuoAttention and AdaEA are outside it and raise NotImplementedError.
"""
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from . import ops
from .cache import DualCache


@dataclass
class WGKVConfig:
    """The configuration fields the path reads, with the reference's names and
    defaults (src/configuration_llama.py:185-214; Qwen3 differs only in
    g_expand = 1.5, src/configuration_qwen3.py:183)."""
    hidden_size: int = 4096
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: Optional[int] = None
    rope_theta: float = 10000.0
    attention_bias: bool = False
    local_window_size: int = 256
    g_inputs: List[str] = field(default_factory=lambda: ["pre_k", "post_k"])
    g_act_fn: str = "gelu"
    g_expand: float = 4.0
    g_epsilon: float = 1e-3
    g_rms: bool = True
    g_threshold: float = 0.1
    use_baseline: bool = False
    block_size: int = 16
    max_total_tokens: Optional[int] = None
    max_tokens_per_head: Optional[int] = None
    random_sparsity: Optional[float] = None
    # seed of the decode-step random draws (random_sparsity); not a reference field
    random_seed: int = 0
    g_fast_path: bool = False
    g_defer: bool = False
    use_triton_kernel: bool = False
    use_duo_attn: bool = False
    use_adaea: bool = False
    use_quest: bool = False
    quest_token_budget: Optional[int] = None
    snapkv_enabled: bool = False
    snapkv_max_cached_tokens: int = -1
    snapkv_evict_ratio: float = 0.0
    snapkv_window_size: int = 256
    snapkv_kernel_size: int = 5
    # Capacity failures are latched in the cache's device ``status`` (the
    # failing write stores nothing).  check_capacity reads it after each
    # layer's prefill (one host sync per layer and chunk); a decode step reads
    # it only with check_capacity_decode (a host sync per step, as the
    # reference's asserts make).  Otherwise a decode-time overflow stays latched
    # until DualCache.raise_if_failed is called.
    check_capacity: bool = True
    check_capacity_decode: bool = False

    def __post_init__(self):
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads


def _layer_cache_check(self, cache, where, decode=False):
    if getattr(self.config, "check_capacity_decode" if decode else "check_capacity", not decode):
        cache.raise_if_failed(where)


def get_random_g_scores(self, batch_size, kv_seq_len, device):
    """src/modeling_layers.py:1160-1166: 1 where U[0,1) >= random_sparsity."""
    r = torch.rand(batch_size, self.config.num_key_value_heads, kv_seq_len, dtype=torch.bfloat16, device=device)
    return (r >= self.config.random_sparsity).to(torch.bfloat16)


def decode_random_admission(self, past_key_value, flags, active=None):
    """A decode step's get_random_g_scores(...) > g_threshold
    (src/modeling_layers.py:1160-1166 with :1465): flags (H, n) bool <- admit
    iff r >= random_sparsity, for draws r in [0, 1) made on the device by a
    counter-based generator (seed ``cache.random_seed``, one counter per
    layer), so that a captured decode step draws exactly as the eager one.
    The reference draws with torch.rand; its values cannot be reproduced
    bit for bit, only the rule.  g_threshold < 1 is assumed, as for every
    score of 1 to admit."""
    c = past_key_value
    if not self.config.g_threshold < 1.0:
        raise AssertionError("random admission scores are 0 or 1; g_threshold must be below 1")
    ops.random_admission(flags, self.config.random_sparsity, c.random_seed,
                         c.random_draws[self.layer_idx:self.layer_idx + 1], active=active)


def snapkv_record_queries(self, past_key_value, query_states):
    """src/modeling_layers.py:579-592: keep the last snapkv_window_size
    queries of each layer (the prompt's tail at prefill, one per decode step)."""
    c = past_key_value
    win = self.config.snapkv_window_size
    q_len = query_states.shape[2]
    if q_len > 1:
        take = min(win, q_len)
        c.snapkv_query_buffer[self.layer_idx, :take] = query_states[0, :, -take:, :].transpose(0, 1)
        if self.layer_idx == self.config.num_hidden_layers - 1:
            c.snapkv_query_length = take
            c.snapkv_query_ptr = take % win
    else:
        c.snapkv_query_buffer[self.layer_idx, c.snapkv_query_ptr] = query_states[0, :, 0, :]
        if self.layer_idx == self.config.num_hidden_layers - 1:
            c.snapkv_query_length = min(win, c.snapkv_query_length + 1)
            c.snapkv_query_ptr = (c.snapkv_query_ptr + 1) % win


@torch.no_grad()
def snapkv_evict(self, past_key_value, device, local_blocks_per_head, max_cached_tokens=None):
    """src/modeling_layers.py:595-671 on the device (wgkv_snapkv_evict): per
    (layer, KV head), score the global tokens by the window queries'
    attention (logits rounded as the reference's bf16 product, softmax in
    fp32, max over the grouped heads, mean over the window, max-pooled),
    drop the int(len * ratio) lowest (equal scores: lower position first),
    pack the kept tokens into the head's first pages, release the rest to the
    free list and reset their table slots -- no host synchronisation.

    With ``max_cached_tokens`` the eviction runs only if the global lengths
    sum to more (the trigger of :1503-1506, decided on the device, which
    also counts the eviction); without it, it always runs, as the reference's
    function does."""
    c = past_key_value
    cfg = self.config
    if max_cached_tokens is None and c.snapkv_query_length != cfg.snapkv_window_size:
        raise AssertionError("SnapKV eviction needs a full query window")  # :597
    ops.snapkv_evict(c, cfg.num_attention_heads // cfg.num_key_value_heads, self.scaling, cfg.snapkv_window_size,
                     cfg.snapkv_kernel_size, cfg.snapkv_evict_ratio,
                     -1 if max_cached_tokens is None else max_cached_tokens)


def refresh_local_is_global(self, past_key_value, device, on_device=False):
    """src/modeling_layers.py:1169-1180: re-gate the whole local window of this
    layer (deferred gating) and store the flags.  With ``on_device`` the
    caller has not tested the condition (slot W-1 just written, :1404): the
    gate launch reads the slot from the cache's device ring state and does
    nothing on other steps, so a captured decode step can include it."""
    c = past_key_value
    layer = self.layer_idx
    H, W, D = c.num_kv_heads, c.local_window_size, c.head_dim
    if self.config.random_sparsity is not None:
        # :1177-1178 -- admitted iff r >= random_sparsity (the score 1 or 0
        # against g_threshold); the draws are made on the device, so eager
        # steps and graph replays continue one sequence
        decode_random_admission(self, c, c.local_is_global[layer],
                                active=(c.ring_state[2:], W - 1) if on_device else None)
        return
    if self.config.g_expand != 0.0:
        start = layer * H * W
        k = c.block_pool_k[start:start + H * W].view(1, H, W, D)
        v = c.block_pool_v[start:start + H * W].view(1, H, W, D)
        self.g_predictors.scores_and_mask(c.local_pre_key[layer].unsqueeze(0), k, v, self.config.g_threshold,
                                          mask_out=c.local_is_global[layer].unsqueeze(0), want_scores=False,
                                          active=(c.ring_state[2:], W - 1) if on_device else None)


def refresh_windows(attention_layers, past_key_value, device):
    """The deferred re-gate of every layer's window (refresh_local_is_global,
    src/modeling_layers.py:1169-1180), for a caller that set
    ``cache.refresh_by_caller`` and runs it after a decode step that wrote the
    ring's last slot.  Equivalent to the per-layer refresh inside the step:
    a layer's flags are next read by the promotion at the start of the next
    step, and its window's keys and values do not change after its own write
    within the step."""
    for attn in attention_layers:
        refresh_local_is_global(attn, past_key_value, device)


def migrate_local_kv_to_global(self, past_key_value, device, local_blocks_per_head):
    """src/modeling_layers.py:674-763 on the device (no host syncs unless
    check_capacity_decode asks for the reference's per-step overflow assert)."""
    ops.decode_append(past_key_value, 0, migrate=True, write=False)
    _layer_cache_check(self, past_key_value, "migrate_local_kv_to_global", decode=True)


def prefill_wrapper(self, past_key_value, query_states, pre_key, key_states, value_states,
                    batch_size, q_seq_len, device, g_mask, local_blocks_per_head):
    """src/modeling_layers.py:1183-1376.  Tensors are (B, H, S, D); B = 1.

    The first call initialises the cache and prefills as the reference does.
    A later call before any decode step continues the prompt as a chunk at
    position ``cache.prefill_length`` (the reference asserts a single
    initialisation, :1197): the cache ends as a one-shot prefill of the
    whole prompt would, up to page numbering, and the chunk's queries attend
    exactly as that prompt's rows would.  Continuation needs a full ring
    (prefill_length >= W), chunks of at least W tokens and a prefill_length
    that is a multiple of 64."""
    c = past_key_value
    W = self.config.local_window_size
    if self.layer_idx == 0 and not (c.gated_kv_initialized and c.prefill_length > 0):
        c.initialize(self.config, self.head_dim, key_states.dtype, device)
    defer = c.local_pre_key is not None
    c0 = c.prefill_length
    if c0 > 0:
        if c.decode_started:
            raise AssertionError("prefill continuation after decode steps is not supported")
        if c0 < W or q_seq_len < W or c0 % 64:
            raise AssertionError(f"chunked prefill needs prefill_length >= W, chunk >= W and a 64-aligned start "
                                 f"(prefill_length={c0}, chunk={q_seq_len}, W={W})")
        before = c.global_lengths[self.layer_idx].clone() if self.config.use_quest else None
        step = ops.ChunkStep(c, self.layer_idx, query_states[0].transpose(0, 1), key_states[0].transpose(0, 1),
                             value_states[0].transpose(0, 1), g_mask[0], c0, self.scaling,
                             pre_key=pre_key[0].transpose(0, 1) if (defer and pre_key is not None) else None)
        step.admit()
        # the chunk's attention kernel behind its own swap point (the one-shot path's is prefill_kernel)
        out = getattr(self, "chunk_prefill_kernel", ops.chunk_attend)(step)
        step.ring()
        _layer_cache_check(self, c, f"prefill_wrapper chunk at {c0} (layer {self.layer_idx})")
        if self.config.use_quest:
            ops.quest_update_bounds(c, self.layer_idx, from_lengths=before)
        c.local_length = min(c0 + q_seq_len, W)
        if self.layer_idx == self.config.num_hidden_layers - 1:
            c.prefill_length = c0 + q_seq_len
        return out.unsqueeze(0)
    ops.prefill_admit(c, self.layer_idx, key_states[0], value_states[0], g_mask[0],
                      pre_key=pre_key[0] if (defer and pre_key is not None) else None)
    _layer_cache_check(self, c, f"prefill_wrapper (layer {self.layer_idx})")
    if self.config.use_quest:  # :1333-1347
        ops.quest_update_bounds(c, self.layer_idx)
    c.local_length = min(q_seq_len, W)  # :1297
    if self.layer_idx == self.config.num_hidden_layers - 1:
        c.prefill_length = q_seq_len
    meta = ops.generate_sparse_indices(g_mask, W, batch_size,
                                       self.config.num_key_value_heads, q_seq_len, device)
    return self.prefill_kernel(
        query_states.transpose(1, 2), key_states.transpose(1, 2), value_states.transpose(1, 2),
        *meta, softmax_scale=self.scaling, causal=True, return_softmax_lse=False)


def ring_write_in_projection(self, c):
    """Whether this layer's decode-step ring write (decode_wrapper's append
    without a mask) can run inside the q/k/v projection's launch
    (model_ops.qkv_rope with ring): device ring pointers, deferred gating (a
    decode token gets no mask and its pre-RoPE key is stored), no QUEST or
    SnapKV bookkeeping, and a layer between the first (whose lazy promotion
    must read the oldest slot before it is overwritten) and the last (whose
    append advances the ring pointers)."""
    cfg = self.config
    return (c is not None and getattr(c, "device_ring", False) and getattr(c, "gated_kv_initialized", False)
            and c.prefill_length > 0 and c.local_pre_key is not None and "pre_k" in cfg.g_inputs
            and cfg.g_defer and not cfg.use_baseline and not cfg.use_quest and not cfg.snapkv_enabled
            and 0 < self.layer_idx < cfg.num_hidden_layers - 1)


def decode_wrapper(self, past_key_value, query_states, pre_key, key_states, value_states,
                   device, g_mask, local_blocks_per_head):
    """src/modeling_layers.py:1379-1449.  Tensors are (1, H, 1, D)."""
    c = past_key_value
    W = self.config.local_window_size
    c.decode_started = True
    insert_pos = c.local_length if c.local_length < W else c.local_ptr
    seqlens = c.cache_seqlens[self.layer_idx]
    last = self.layer_idx == self.config.num_hidden_layers - 1
    if getattr(c, "ring_written_by", None) == self.layer_idx and g_mask is None:
        c.ring_written_by = None  # the q/k/v projection's launch wrote the slot (ring_write_in_projection)
    else:
        ops.decode_append(c, self.layer_idx, key_states[0, :, 0], value_states[0, :, 0],
                          g_mask=None if g_mask is None else g_mask[0, :, 0],
                          pre_key=pre_key[0, :, 0] if g_mask is None else None,
                          migrate=False, write=True, cache_seqlens=seqlens[0], advance=last)
    if g_mask is None:
        if c.refresh_by_caller:
            pass  # the caller re-gates the windows after the step (refresh_windows)
        elif c.device_ring:
            refresh_local_is_global(self, c, device, on_device=True)  # runs only if slot W-1 was written
        elif insert_pos == W - 1:
            refresh_local_is_global(self, c, device)
    if self.config.use_quest:  # :1419-1427
        if c.device_ring:
            raise AssertionError("QUEST selection takes the host ring length; it cannot run with device_ring")
        if self.config.quest_token_budget is None:
            raise AssertionError("use_quest needs quest_token_budget")
        local_tokens = min(c.local_length + 1, W)
        seqlens, table = ops.quest_select(c, self.layer_idx, query_states[0, :, 0], local_tokens,
                                          self.config.quest_token_budget)
    else:
        table = c.block_table[self.layer_idx].unsqueeze(0)
    if last:
        c.advance_host_ring()
    handle = self.decode_kernel_handle(
        query_states.transpose(1, 2), c.k_cache(), c.v_cache(), seqlens, table, self.scaling)
    return self.decode_kernel_executor(handle)


def self_attn_forward_patch_inference(self, past_key_value, input_shape, query_states, pre_key, key_states,
                                      value_states, g_scores, g_mask=None):
    """src/modeling_layers.py:1452-1509.  ``g_mask`` may be passed directly
    (the fused gate produces it); otherwise it is ``g_scores > g_threshold``."""
    batch_size, q_seq_len = input_shape
    device = query_states.device
    is_prefilling = q_seq_len > 1
    if g_mask is None and g_scores is not None:
        g_mask = g_scores > self.config.g_threshold
    if self.config.local_window_size % self.config.block_size:
        raise AssertionError("local_window_size % block_size != 0")
    lbph = self.config.local_window_size // self.config.block_size
    if (not is_prefilling) and self.layer_idx == 0 and (past_key_value.device_ring or
                                                        past_key_value.local_length == self.config.local_window_size):
        # with device_ring the ring-full condition is evaluated on the device
        migrate_local_kv_to_global(self, past_key_value, device, lbph)
    if is_prefilling:
        out = self.prefill_wrapper(self, past_key_value, query_states, pre_key, key_states, value_states,
                                   batch_size, q_seq_len, device, g_mask, lbph)
    else:
        out = self.decode_wrapper(self, past_key_value, query_states, pre_key, key_states, value_states,
                                  device, g_mask, lbph)
    if self.config.snapkv_enabled:  # :1500-1507
        c = past_key_value
        if c.device_ring:
            raise AssertionError("the SnapKV query window advances on the host; it cannot run with device_ring")
        snapkv_record_queries(self, c, query_states)
        if self.layer_idx == self.config.num_hidden_layers - 1:
            budget = self.config.snapkv_max_cached_tokens
            if c.snapkv_query_length == self.config.snapkv_window_size:
                snapkv_evict(self, c, device, lbph, max_cached_tokens=budget)  # trigger decided on the device
            elif int(c.global_lengths.sum().item()) > budget:
                # the reference's eviction asserts a full window (:597); only a
                # window not yet full reads the trigger back to raise it here
                raise AssertionError("SnapKV eviction needs a full query window")
    return out


_ALL_ADMITTED = {}


def _all_admitted(batch_size, num_kv_heads, kv_seq_len, device):
    """The use_baseline mask (every token admitted, src/modeling_layers.py:1556),
    made once per shape and device (it is only read) rather than filled in
    every layer of every step; not cached while a graph is being captured."""
    key = (batch_size, num_kv_heads, kv_seq_len, device)
    m = _ALL_ADMITTED.get(key)
    if m is None:
        m = torch.ones(batch_size, num_kv_heads, kv_seq_len, dtype=torch.bool, device=device)
        if not (device.type == "cuda" and torch.cuda.is_current_stream_capturing()):
            _ALL_ADMITTED[key] = m
    return m


def self_attn_forward_patch(self, gating_mode, attention_mask, past_key_value, input_shape, query_states,
                            pre_key, key_states, value_states):
    """src/modeling_layers.py:1534-1629, inference mode (gating_mode 3)."""
    batch_size, _ = input_shape
    device = query_states.device
    cfg = self.config
    if gating_mode != 3:
        raise NotImplementedError("only inference (gating_mode 3) is on the MI355X path")
    if cfg.use_duo_attn or cfg.use_adaea:
        raise NotImplementedError("DuoAttention / AdaEA baselines are outside the hot path")
    kv_seq_len = key_states.size(2)
    g_scores = None
    g_mask = None
    if cfg.use_baseline:
        g_mask = _all_admitted(batch_size, cfg.num_key_value_heads, kv_seq_len, device)
    elif not (kv_seq_len == 1 and cfg.g_defer):
        if cfg.random_sparsity is not None and kv_seq_len == 1 and past_key_value is not None \
                and getattr(past_key_value, "gated_kv_initialized", False):
            # a decode step's draws on the device (graph-capturable)
            g_mask = torch.empty(batch_size, cfg.num_key_value_heads, kv_seq_len, dtype=torch.bool, device=device)
            decode_random_admission(self, past_key_value, g_mask[0])
        elif cfg.random_sparsity is not None:
            g_scores = get_random_g_scores(self, batch_size, kv_seq_len, device)
        elif cfg.g_expand != 0.0:
            g_scores, g_mask = self.g_predictors.scores_and_mask(pre_key, key_states, value_states, cfg.g_threshold)
    if query_states.dtype != torch.bfloat16:
        # the cache and attention kernels are bf16 (as the reference's are); the
        # gate above has already seen the model-dtype keys
        query_states = query_states.to(torch.bfloat16)
        key_states = key_states.to(torch.bfloat16)
        value_states = value_states.to(torch.bfloat16)
        pre_key = pre_key.to(torch.bfloat16) if pre_key is not None else None
    if batch_size != 1:
        raise AssertionError("gating_mode 3 runs batch 1")
    if attention_mask is not None:
        raise AssertionError("gating_mode 3 takes no attention mask")
    if past_key_value is None:
        raise AssertionError("gating_mode 3 needs a cache (DualCache)")
    out = self_attn_forward_patch_inference(self, past_key_value, input_shape, query_states, pre_key,
                                            key_states, value_states, g_scores, g_mask=g_mask)
    return out, None, None


__all__ = [
    "WGKVConfig", "DualCache", "get_random_g_scores", "decode_random_admission", "refresh_local_is_global",
    "refresh_windows", "migrate_local_kv_to_global", "ring_write_in_projection",
    "prefill_wrapper", "decode_wrapper", "self_attn_forward_patch_inference", "self_attn_forward_patch",
]
