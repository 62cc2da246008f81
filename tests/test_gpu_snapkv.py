"""SnapKV eviction on the GPU (wgkv_snapkv_evict: scoring, selection,
packing and page release in device kernels, trigger decided on the device).

* Against the reference's own snapkv_evict (tests/golden/snapkv_golden.*,
  bf16 logits and fp32): pooled scores within 1e-5 relative plus, with bf16
  logits, the slack of logit sums lying within float32 accumulation error
  of a bf16 rounding boundary (the kernel's sum in another order may round
  such a logit to the other neighbour; test_oracle_snapkv.bf16_logit_slack
  bounds the score move); lengths, block tables and the free list
  bit-exact; the dropped set a valid choice for the reference's scores
  (every position below its cut dropped, none above, within the same
  tolerances; the reference's topk leaves the order of equal scores
  unspecified) and the kept tokens exactly the others, in order.
* Through the layer path (query window, eviction, released pages reused by
  the promotion kernel) against the oracle (oracle/snapkv.py +
  oracle/dualcache.py) on the same inputs: after every step the block
  tables, global lengths, released-page list and the logical global caches
  are identical, and every decode output matches the fp64 attention over
  the oracle's own cache within max-abs 2e-2 / mean-abs 2e-3."""
import types

import numpy as np
import pytest
import torch

import scenarios
from oracle import attention, snapkv
from oracle.dualcache import DualCacheOracle
from test_oracle_snapkv import assert_tie_equivalent, bf16_logit_slack, golden_heads, snapkv_gold

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
            snapkv.evict(orc, qwin, G, D ** -0.5, ratio, ksz, logits_bf16=True)
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


def device_state(st, sc):
    """A cache object for ops.snapkv_evict holding the scenario's state (bf16
    pools: the fp32 scenario's values are bf16 values)."""
    P, lb = 16, sc["W"] // 16
    maxp = st["block_table"].shape[2]
    i32 = dict(dtype=torch.int32, device=DEV)
    free = torch.zeros(st["total_blocks"], **i32)
    free[:len(st["free_ids"])] = torch.tensor(st["free_ids"], **i32)
    return types.SimpleNamespace(
        num_layers=sc["L"], num_kv_heads=sc["H"], head_dim=sc["D"], block_size=P, local_window_size=sc["W"],
        max_tokens_per_head=maxp * P, total_blocks=st["total_blocks"],
        block_pool_k=st["pool_k"].to(torch.bfloat16).to(DEV), block_pool_v=st["pool_v"].to(torch.bfloat16).to(DEV),
        block_table=st["block_table"].to(DEV), global_lengths=st["global_lengths"].to(DEV),
        free_block_ids_dev=free, free_count_dev=torch.tensor([len(st["free_ids"])], **i32),
        snapkv_query_buffer=st["qbuf"].to(torch.bfloat16).to(DEV).contiguous(), snapkv_state=torch.zeros(2, **i32))


def dropped_positions(before_k, before_v, after_k, after_v):
    """Positions of the original tokens missing from the kept list, checking
    that the kept list is the others in order (rows matched exactly)."""
    dropped, j = [], 0
    for i in range(before_k.shape[0]):
        if j < after_k.shape[0] and torch.equal(before_k[i], after_k[j]) and torch.equal(before_v[i], after_v[j]):
            j += 1
        else:
            dropped.append(i)
    assert j == after_k.shape[0], "the kept tokens are not the original ones in order"
    return dropped


@pytest.mark.parametrize("name", list(scenarios.SNAPKV_SCENARIOS))
def test_evict_matches_reference_golden(name):
    from wgkv import ops
    z, meta = snapkv_gold()
    sc = scenarios.SNAPKV_SCENARIOS[name]
    st = scenarios.snapkv_state(sc)
    assert scenarios.checksum(st["pool_k"], st["pool_v"], st["qbuf"], st["block_table"]) == meta[name]["inputs_sha256"]
    print(f"[snapkv golden] {name}", flush=True)
    c = device_state(st, sc)
    lb = sc["W"] // 16
    L, H = sc["L"], sc["H"]
    before_k = scenarios.logical_tokens(st["pool_k"].to(torch.bfloat16), st["block_table"], st["global_lengths"], lb)
    before_v = scenarios.logical_tokens(st["pool_v"].to(torch.bfloat16), st["block_table"], st["global_lengths"], lb)
    # below the trigger: nothing moves
    ops.snapkv_evict(c, sc["G"], sc["D"] ** -0.5, sc["win"], sc["ksz"], sc["ratio"],
                     max_cached_tokens=int(st["global_lengths"].sum()), logits_bf16=sc["dtype"] == "bf16")
    torch.cuda.synchronize()
    assert c.snapkv_state.tolist() == [0, 0]
    assert torch.equal(c.global_lengths.cpu(), st["global_lengths"]) and torch.equal(c.block_table.cpu(), st["block_table"])
    scores = torch.full((L * H, c.max_tokens_per_head), -1.0, device=DEV)
    ops.snapkv_evict(c, sc["G"], sc["D"] ** -0.5, sc["win"], sc["ksz"], sc["ratio"],
                     max_cached_tokens=int(st["global_lengths"].sum()) - 1, logits_bf16=sc["dtype"] == "bf16",
                     scores_out=scores)
    torch.cuda.synchronize()
    assert c.snapkv_state.tolist() == [1, 1]
    assert np.array_equal(c.global_lengths.cpu().numpy(), z[f"{name}.global_lengths"])
    assert np.array_equal(c.block_table.cpu().numpy(), z[f"{name}.block_table"])
    nf = int(c.free_count_dev.item())
    assert c.free_block_ids_dev[:nf].tolist() == z[f"{name}.free_ids"].tolist()
    after_k = scenarios.logical_tokens(c.block_pool_k.cpu(), c.block_table.cpu(), c.global_lengths.cpu(), lb)
    after_v = scenarios.logical_tokens(c.block_pool_v.cpu(), c.block_table.cpu(), c.global_lengths.cpu(), lb)
    gold = golden_heads(z, name)
    worst, worst_amb, n_amb = 0.0, 0.0, 0
    qbuf = st["qbuf"].float()
    for l in range(L):
        for h in range(H):
            if (l, h) not in gold:
                assert torch.equal(after_k[(l, h)], before_k[(l, h)]), (l, h)
                continue
            s_ref, ev_ref = gold[(l, h)]
            n = s_ref.numel()
            s = scores[l * H + h, :n].double().cpu()
            if sc["dtype"] == "bf16":
                qw = qbuf[l].view(sc["win"], H, sc["G"], sc["D"]).permute(1, 2, 0, 3)[h]
                slack = bf16_logit_slack(qw, before_k[(l, h)].float(), sc["D"] ** -0.5, sc["ksz"])
            else:
                slack = torch.zeros(n, dtype=torch.float64)
            err = (s - s_ref).abs()
            clean = slack == 0
            n_amb += int((~clean).sum())
            rel = err / s_ref.abs().clamp(min=1e-30)
            worst = max(worst, rel[clean].max().item() if clean.any() else 0.0)
            worst_amb = max(worst_amb, (err / (1e-5 * s_ref.abs() + slack))[~clean].max().item() if (~clean).any()
                            else 0.0)
            assert bool((err <= 1e-5 * s_ref.abs() + slack).all()), (l, h, rel.max().item())
            # a flipped logit is rare: most scores agree to float32 rounding whatever their slack
            q50, q90 = torch.quantile(rel, torch.tensor([0.5, 0.9], dtype=torch.float64)).tolist()
            print(f"[snapkv golden] {name} ({l},{h}): rel err p50 {q50:.1e} p90 {q90:.1e} max {rel.max().item():.1e}",
                  flush=True)
            assert q50 <= 2e-6 and q90 <= 1e-5, (q50, q90)
            ev = dropped_positions(before_k[(l, h)], before_v[(l, h)], after_k[(l, h)], after_v[(l, h)])
            assert_tie_equivalent(s_ref, ev_ref, ev, 1e-5, f"{name} {l} {h}", slack=slack)
    print(f"[snapkv golden] {name}: heads {sorted(gold)}, pooled scores max rel {worst:.1e} on tokens clear of "
          f"bf16 logit boundaries; {n_amb} tokens with slack, worst at {worst_amb:.2f} of it; tables/lengths/free "
          f"list exact, drops tie-equivalent", flush=True)
