"""GPU dual cache (admission, compaction, page scatter, ring, lazy promotion,
decode lengths) vs golden vectors written by the reference's own
prefill_wrapper / decode_wrapper / migrate_local_kv_to_global, through the
product's self_attn_forward_patch_inference.  Block tables, lengths, flags,
the bump pointer, per-step decode lengths and the logical cache contents must
match bit for bit; each decode step's attention output is checked against the
fp32 oracle over the oracle's own cache."""
import json
import os
import types

import numpy as np
import pytest
import torch

import scenarios
from oracle import attention
from oracle.dualcache import DualCacheOracle

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def gold():
    with open(os.path.join(GOLD, "cache_golden.json")) as f:
        meta = json.load(f)
    return np.load(os.path.join(GOLD, "cache_golden.npz")), meta


def make_self(sc, layer, gates=None):
    import wgkv
    from wgkv import layers
    cfg = layers.WGKVConfig(num_hidden_layers=sc["L"], num_attention_heads=sc["H"] * sc["G"],
                            num_key_value_heads=sc["H"], head_dim=sc["D"], hidden_size=sc["H"] * sc["G"] * sc["D"],
                            local_window_size=sc["W"], block_size=16,
                            max_total_tokens=sc["L"] * sc["H"] * sc["max_tokens_per_head"],
                            max_tokens_per_head=sc["max_tokens_per_head"], g_defer=sc["g_defer"])
    s = types.SimpleNamespace(config=cfg, layer_idx=layer, head_dim=sc["D"], scaling=sc["D"] ** -0.5,
                              num_key_value_groups=sc["G"])
    s.prefill_wrapper = layers.prefill_wrapper
    s.decode_wrapper = layers.decode_wrapper
    s.prefill_kernel = lambda q, k, v, *m, **kw: torch.zeros_like(q)
    s.decode_kernel_handle = wgkv.flash_attn_with_kvcache_wrapper_triton_handle
    s.decode_kernel_executor = lambda f: f()
    if gates is not None:
        s.g_predictors = gates[layer]
    return s


def product_gates(sc, inp):
    from wgkv.gate import GatingPredictor
    gates = []
    for p in inp["gates"]:
        gp = GatingPredictor(sc["D"], sc["H"], ["pre_k", "post_k"], "gelu", 4.0, 1e-3, True, True)
        gp.load_state_dict({k: v.clone() for k, v in scenarios.defer_bias_shift(p).items()}, strict=True)
        gates.append(gp.cuda())
    return gates


def oracle_regate(inp):
    from oracle import gate as ogate
    params = [scenarios.defer_bias_shift(p) for p in inp["gates"]]

    def regate(layer, pk, k, v):
        return ogate.gate_scores(pk[None], k[None], v[None], params[layer])[0] > 0.1
    return regate


@pytest.mark.parametrize("name", list(scenarios.CACHE_SCENARIOS))
def test_cache_matches_reference_golden(name):
    from wgkv import layers
    from wgkv.cache import DualCache
    g, meta = gold()
    sc = scenarios.CACHE_SCENARIOS[name]
    inp = scenarios.cache_inputs(sc)
    L, H, D, W = sc["L"], sc["H"], sc["D"], sc["W"]
    print(f"[cache parity] {name}", flush=True)
    dev = torch.device("cuda:0")
    gates = product_gates(sc, inp) if sc["g_defer"] else None
    regate = oracle_regate(inp) if sc["g_defer"] else None
    mods = [make_self(sc, l, gates) for l in range(L)]
    cache = DualCache()
    orc = DualCacheOracle(L, H, D, W, L * H * sc["max_tokens_per_head"], sc["max_tokens_per_head"],
                          g_defer=sc["g_defer"])
    for l in range(L):
        q, pk, k, v, mask = inp["prompt"][l]
        layers.self_attn_forward_patch_inference(mods[l], cache, (1, sc["S"]), q.to(dev), pk.to(dev), k.to(dev),
                                                 v.to(dev), None, g_mask=mask.to(dev))
        orc.prefill(l, k[0], v[0], mask[0], pre_key=pk[0])
    torch.cuda.synchronize()
    assert np.array_equal(cache.block_table.cpu().numpy(), g[f"{name}.after_prefill.block_table"])
    assert np.array_equal(cache.global_lengths.cpu().numpy(), g[f"{name}.after_prefill.global_lengths"])
    assert np.array_equal(cache.local_is_global.cpu().numpy(), g[f"{name}.after_prefill.local_is_global"])
    assert cache.next_free_block == meta[f"{name}.after_prefill"]["next_free_block"]
    seqlens = []
    worst = 0.0
    for step in inp["steps"]:
        for l in range(L):
            q, pk, k, v, mask = step[l]
            out = layers.self_attn_forward_patch_inference(
                mods[l], cache, (1, 1), q.to(dev), pk.to(dev), k.to(dev), v.to(dev), None,
                g_mask=None if mask is None else mask.to(dev))
            seqlens.append(cache.cache_seqlens[l, 0].clone())
            sl, bt = orc.decode(l, k[0, :, 0], v[0, :, 0], None if mask is None else mask[0, :, 0],
                                pre_key=pk[0, :, 0], regate=regate)
            ref = attention.paged_decode(q.transpose(1, 2), orc.block_pool_k.view(-1, 16, D),
                                         orc.block_pool_v.view(-1, 16, D), sl[None], bt[None], sc["D"] ** -0.5)
            err = (out.float().cpu() - ref).abs()
            worst = max(worst, err.max().item())
            assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
    torch.cuda.synchronize()
    assert np.array_equal(torch.stack(seqlens).cpu().numpy(), g[f"{name}.decode_seqlens"])
    assert np.array_equal(cache.block_table.cpu().numpy(), g[f"{name}.final.block_table"])
    assert np.array_equal(cache.global_lengths.cpu().numpy(), g[f"{name}.final.global_lengths"])
    assert np.array_equal(cache.local_is_global.cpu().numpy(), g[f"{name}.final.local_is_global"])
    assert cache.next_free_block == meta[name]["next_free_block"]
    assert (cache.local_ptr, cache.local_length) == (meta[name]["local_ptr"], meta[name]["local_length"])
    parts = []
    kc = cache.block_pool_k.view(-1, 16, D).cpu()
    vc = cache.block_pool_v.view(-1, 16, D).cpu()
    for l in range(L):
        for h in range(H):
            T = cache.local_length + int(cache.global_lengths[l, h])
            ids = cache.block_table[l, h, :(T + 15) // 16].long().cpu()
            parts += [kc[ids].reshape(-1, D)[:T], vc[ids].reshape(-1, D)[:T]]
    assert scenarios.checksum(*parts) == meta[name]["logical_sha256"]
    print(f"[cache parity] {name}: worst decode max_abs {worst:.2e}", flush=True)


def test_prefill_capacity_error_writes_nothing():
    from wgkv import _lib, layers
    from wgkv.cache import DualCache
    sc = dict(scenarios.CACHE_SCENARIOS["long_prompt"], max_tokens_per_head=256)
    inp = scenarios.cache_inputs(sc)
    dev = torch.device("cuda:0")
    s = make_self(sc, 0)
    cache = DualCache()
    q, pk, k, v, mask = inp["prompt"][0]
    with pytest.raises(AssertionError):
        layers.self_attn_forward_patch_inference(s, cache, (1, sc["S"]), q.to(dev), pk.to(dev), k.to(dev),
                                                 v.to(dev), None, g_mask=mask.to(dev))
    # nothing was written: lengths zero, bump pointer at the local pages, table untouched past them
    assert int(cache.global_lengths.sum()) == 0
    lb = sc["W"] // 16
    assert cache.next_free_block == sc["L"] * sc["H"] * lb
    assert bool((cache.block_table[:, :, lb:] == cache.total_blocks - 1).all())


@pytest.mark.parametrize("per_step", [False, True])
def test_decode_capacity_error_raises(per_step):
    """Every token admitted, tiny per-head budget: promotion overflows.  By
    default the decode steps do not read the device status (no host sync);
    the failure stays latched and raise_if_failed reports it.  With
    check_capacity_decode the step itself raises, as the reference's assert."""
    from wgkv import _lib, layers
    from wgkv.cache import DualCache
    sc = dict(scenarios.CACHE_SCENARIOS["short_prompt"], max_tokens_per_head=128 + 20, step_rate=1.0, rates=(1.0, 1.0))
    inp = scenarios.cache_inputs(sc)
    dev = torch.device("cuda:0")
    mods = [make_self(sc, l) for l in range(sc["L"])]
    for m in mods:
        m.config.check_capacity_decode = per_step
    cache = DualCache()
    for l in range(sc["L"]):
        q, pk, k, v, mask = inp["prompt"][l]
        layers.self_attn_forward_patch_inference(mods[l], cache, (1, sc["S"]), q.to(dev), pk.to(dev), k.to(dev),
                                                 v.to(dev), None, g_mask=mask.to(dev))

    def steps():
        for step in inp["steps"]:
            for l in range(sc["L"]):
                q, pk, k, v, mask = step[l]
                layers.self_attn_forward_patch_inference(mods[l], cache, (1, 1), q.to(dev), pk.to(dev), k.to(dev),
                                                         v.to(dev), None, g_mask=mask.to(dev))

    if per_step:
        with pytest.raises(AssertionError):
            steps()
    else:
        steps()
        torch.cuda.synchronize()
        assert int(cache.status.item()) == _lib.ERR_CAPACITY
        with pytest.raises(_lib.WGKVCapacityError):
            cache.raise_if_failed("decode")
        assert int(cache.status.item()) == 0
    assert int(cache.global_lengths.max()) <= 20
