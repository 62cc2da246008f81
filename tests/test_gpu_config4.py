"""BASELINE config 4 exactly as bench.py times it: a 32K-token prompt through
one Llama-3.1-8B-shaped layer (32 q / 8 KV heads, head_dim 128, W 1024,
~20 % admission) in 4096-token chunks -- write gate (fp32 scores, mask),
admission into the dual cache, the chunk's sparse attention, ring rewrite.

Checked:
* the per-chunk masks equal the gate over the whole prompt; the gate has
  bf16 parameters (as the reference's profiling run loads them); every score
  lies in the range oracle.gate_outcomes allows the kernel's float32 order,
  every token that range pins to the oracle's restatement of the
  reference's bf16 rounding points (oracle.gate.gate_scores_bf16) carries
  exactly that score, and admission differs only on flagged tokens;
* every chunk's attention rows equal the one-shot kernel's rows over the
  whole prompt bit for bit, and sampled rows of every chunk meet the fp64
  ideal-mask attention (max-abs 2e-2, mean-abs 2e-3);
* the dereferenced logical cache (global lengths, global K/V in order, ring,
  flags) equals both the one-shot prefill's and a DualCacheOracle replay of
  the same mask on the CPU."""
import numpy as np
import pytest

import parity_log
import torch

from oracle import attention
from oracle import gate as ogate
from oracle import gate_outcomes as gout
from oracle.dualcache import DualCacheOracle
from test_gpu_chunked import assert_same_logical_cache, global_entries
from test_gpu_gate_bf16 import check as check_bf16_gate

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
S, HQ, HKV, D, W, CH = 32768, 32, 8, 128, 1024, 4096


def _cache():
    from wgkv.cache import DualCache
    from wgkv.layers import WGKVConfig
    cfg = WGKVConfig(num_hidden_layers=1, num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D,
                     hidden_size=HQ * D, local_window_size=W, max_tokens_per_head=S + W,
                     max_total_tokens=HKV * (S + W) + 4096)
    c = DualCache()
    c.initialize(cfg, D, torch.bfloat16, DEV)
    return c, cfg


def test_config4_chunked_pipeline():
    import wgkv
    from wgkv import ops, workloads
    print("[config 4] 32K prompt, 4096-token chunks, Llama-8B layer shapes", flush=True)
    w = workloads.prefill_llama(S=S, Hq=HQ, Hkv=HKV, D=D, W=W, device=DEV)
    pk, kk = w.pre_k.transpose(1, 2), w.k.transpose(1, 2)  # (1, H, S, D) views
    mask = torch.empty(1, HKV, S, dtype=torch.bool, device=DEV)
    scores = torch.empty(1, HKV, S, dtype=torch.float32, device=DEV)
    out = torch.empty(S, HQ, D, dtype=torch.bfloat16, device=DEV)
    cache, cfg = _cache()
    for c0 in range(0, S, CH):
        sl = slice(c0, c0 + CH)
        w.gate.scores_and_mask(pk[:, :, sl], kk[:, :, sl], None, w.threshold,
                               scores_out=scores[:, :, sl], mask_out=mask[:, :, sl])
        st = ops.ChunkStep(cache, 0, w.q[0, sl], w.k[0, sl], w.v[0, sl], mask[0, :, sl], c0,
                           softmax_scale=D ** -0.5, out=out[sl])
        st.admit()
        st.attend()
        st.ring()
    torch.cuda.synchronize()
    assert int(cache.status.item()) == 0
    admitted = mask.float().mean().item()
    print(f"[config 4] admitted {admitted:.4f}", flush=True)
    assert 0.15 < admitted < 0.25

    # the gate over the whole prompt at once gives the same mask
    s_all, m_all = w.gate.scores_and_mask(pk, kk, None, w.threshold)
    assert torch.equal(m_all, mask) and torch.equal(s_all, scores)

    # admission against the CPU oracle of the bf16-parameter gate
    assert w.gate.conv1.weight.dtype == torch.bfloat16
    params = {k: v.detach().cpu() for k, v in w.gate.state_dict().items()}
    ref = ogate.gate_scores_bf16(pk.cpu(), kk.cpu(), None, params)
    order = gout.kernel_order("packed", D, 2, w.gate.inner_dim)
    lo, hi, _ = gout.score_range(pk.cpu(), kk.cpu(), None, params, order)
    check_bf16_gate("config 4", scores, mask, ref, ogate.bf16_threshold(w.threshold), lo, hi)

    # one-shot prefill of the same prompt and mask
    one, _ = _cache()
    ops.prefill_admit(one, 0, w.k[0].transpose(0, 1), w.v[0].transpose(0, 1), mask[0])
    md = wgkv.generate_sparse_indices(mask, W, 1, HKV, S)
    o1 = wgkv.sparse_attn_func(w.q, w.k, w.v, *md)
    torch.cuda.synchronize()
    assert torch.equal(out, o1[0]), "chunked rows differ from the one-shot kernel's"
    assert_same_logical_cache(cache, one)

    # sampled rows of every chunk against the fp64 ideal-mask attention
    g = torch.Generator().manual_seed(4)
    rows = sorted({int(c0 + x) for c0 in range(0, S, CH) for x in torch.randint(0, CH, (6,), generator=g)}
                  | {0, 63, 64, W - 1, W, S - 1})
    qh = w.q.transpose(1, 2).cpu()
    kh, vh = w.k.transpose(1, 2).cpu(), w.v.transpose(1, 2).cpu()
    refo = attention.sparse_prefill_rows(qh, kh, vh, mask.cpu(), W, rows, D ** -0.5)
    got = out[rows].float().cpu().transpose(0, 1)[None]  # (1, Hq, rows, D)
    err = (got.double() - refo).abs()
    parity_log.report(f"[config 4] {len(rows)} sampled rows vs fp64: max_abs {err.max().item():.2e} "
          f"mean_abs {err.mean().item():.2e}")
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3

    # the logical cache against the oracle's replay of the mask
    orc = DualCacheOracle(1, HKV, D, W, cfg.max_total_tokens, cfg.max_tokens_per_head, dtype=torch.bfloat16)
    orc.prefill(0, kh[0], vh[0], mask[0].cpu())
    assert np.array_equal(cache.global_lengths.cpu().numpy(), orc.global_lengths.numpy())
    assert np.array_equal(cache.local_is_global.cpu().numpy(), orc.local_is_global.numpy())
    ring = slice(0, HKV * W)
    assert torch.equal(cache.block_pool_k[ring].cpu(), orc.block_pool_k[ring])
    assert torch.equal(cache.block_pool_v[ring].cpu(), orc.block_pool_v[ring])
    lb = W // 16
    for h in range(HKV):
        n = int(orc.global_lengths[0, h])
        ids = orc.block_table[0, h, lb:lb + (n + 15) // 16].long()
        r = (ids[:, None] * 16 + torch.arange(16)[None]).reshape(-1)[:n]
        ka, va = global_entries(cache, 0, h)
        assert torch.equal(ka.cpu(), orc.block_pool_k[r]) and torch.equal(va.cpu(), orc.block_pool_v[r]), h
    parity_log.report(f"[config 4] logical cache equals the oracle replay; global lengths "
          f"{cache.global_lengths[0].tolist()}")
