"""SnapKV on the GPU (through the layer path: query window, eviction on the
device, released pages reused by the promotion kernel) against the oracle
(oracle/snapkv.py + oracle/dualcache.py) on the same inputs: after every
step the block tables, global lengths, released-page list and the logical
global caches are identical, and every decode output matches the fp64
attention over the oracle's cache within max-abs 2e-2 / mean-abs 2e-3."""
import types

import pytest
import torch

from oracle import attention, snapkv
from oracle.dualcache import DualCacheOracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_eviction_and_reuse_match_oracle():
    from wgkv import layers, ops
    from wgkv.cache import DualCache
    L, H, G, D, W, S, steps = 2, 2, 2, 64, 64, 800, 220
    win, ratio, ksz = 16, 0.2, 5
    budget = 2 * 2 * 330  # total global tokens over all (layer, head) that triggers an eviction
    print("[snapkv] layer path with eviction", flush=True)
    mtph = S + steps + W
    cfg = layers.WGKVConfig(num_hidden_layers=L, num_attention_heads=H * G, num_key_value_heads=H, head_dim=D,
                            hidden_size=H * G * D, local_window_size=W, block_size=16, max_tokens_per_head=mtph,
                            max_total_tokens=L * H * mtph, snapkv_enabled=True, snapkv_max_cached_tokens=budget,
                            snapkv_evict_ratio=ratio, snapkv_window_size=win, snapkv_kernel_size=ksz,
                            check_capacity=True)
    selves = []
    for l in range(L):
        s = types.SimpleNamespace(config=cfg, layer_idx=l, head_dim=D, scaling=D ** -0.5, num_key_value_groups=G)
        s.prefill_wrapper = layers.prefill_wrapper
        s.decode_wrapper = layers.decode_wrapper
        s.prefill_kernel = ops.sparse_attn_func
        s.decode_kernel_handle = ops.paged_decode_attn_handle
        s.decode_kernel_executor = lambda f: f()
        selves.append(s)
    g = torch.Generator().manual_seed(5)
    bf = lambda *sh: torch.randn(*sh, generator=g).to(torch.bfloat16)
    c = DualCache()
    orc = DualCacheOracle(L, H, D, W, L * H * mtph, mtph, block_size=16, dtype=torch.float32)
    orc.free_block_ids = []
    qwin = snapkv.QueryWindow(L, win, H * G, D)

    def oracle_evict_if_needed():
        if int(orc.global_lengths.sum()) > budget:
            snapkv.evict(orc, qwin, G, D ** -0.5, ratio, ksz)
            return True
        return False

    # prefill
    q, k, v = bf(L, H * G, S, D), bf(L, H, S, D), bf(L, H, S, D)
    gm = torch.rand(L, H, S, generator=g) < 0.45
    for l in range(L):
        layers.self_attn_forward_patch_inference(selves[l], c, (1, S), q[l:l + 1].to(DEV), k[l:l + 1].to(DEV),
                                                 k[l:l + 1].to(DEV), v[l:l + 1].to(DEV), None,
                                                 g_mask=gm[l:l + 1].to(DEV))
        orc.prefill(l, k[l].float(), v[l].float(), gm[l])
        qwin.record(l, q[l].float())
    evictions = int(oracle_evict_if_needed())
    torch.cuda.synchronize()

    def compare(label):
        assert torch.equal(c.global_lengths.cpu(), orc.global_lengths), label
        assert torch.equal(c.block_table.cpu(), orc.block_table), label
        assert c.free_block_ids == orc.free_block_ids, label
        assert c.next_free_block == orc.next_free_block, label
        lb = W // 16
        for l in range(L):
            for h in range(H):
                n = int(orc.global_lengths[l, h])
                ids = orc.block_table[l, h, lb:lb + (n + 15) // 16].long()
                rows = (ids[:, None] * 16 + torch.arange(16)[None]).reshape(-1)[:n]
                assert torch.equal(c.block_pool_k.cpu()[rows].float(), orc.block_pool_k[rows]), (label, l, h)
                assert torch.equal(c.block_pool_v.cpu()[rows].float(), orc.block_pool_v[rows]), (label, l, h)

    compare("after prefill")
    for t in range(steps):
        for l in range(L):
            qi, ki, vi = bf(H * G, D), bf(H, D), bf(H, D)
            mi = torch.rand(H, generator=g) < 0.5
            out = layers.self_attn_forward_patch_inference(
                selves[l], c, (1, 1), qi.view(1, H * G, 1, D).to(DEV), ki.view(1, H, 1, D).to(DEV),
                ki.view(1, H, 1, D).to(DEV), vi.view(1, H, 1, D).to(DEV), None, g_mask=mi.view(1, H, 1).to(DEV))
            sl, bt = orc.decode(l, ki.float(), vi.float(), mi)
            kc = orc.block_pool_k.view(-1, 16, D)
            vc = orc.block_pool_v.view(-1, 16, D)
            ref = attention.paged_decode(qi.float().view(1, 1, H * G, D), kc, vc, sl.view(1, H), bt[None],
                                         D ** -0.5, dtype=torch.float64)
            err = (out.reshape(H * G, D).float().cpu() - ref.reshape(H * G, D).float()).abs()
            assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, (t, l, err.max().item())
            qwin.record(l, qi.float()[:, None, :])
        evictions += int(oracle_evict_if_needed())
        torch.cuda.synchronize()
        compare(f"after step {t}")
    print(f"[snapkv] evictions {evictions} (product {c.snapkv_evict_count}), free list {len(c.free_block_ids)}",
          flush=True)
    assert evictions >= 2 and c.snapkv_evict_count == evictions
