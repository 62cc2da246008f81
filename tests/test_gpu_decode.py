"""GPU parity of the ragged paged decode kernel (through the C ABI) vs the
fp32 oracle: max-abs <= 2e-2 and mean-abs <= 2e-3 on bf16 outputs.

Grid of utils/test_flash_attn_with_kvcache.py:7-13 (heads, head size, page
size, batch, max length; pool of 4096 pages, random lengths, randperm pages,
-1 padding), the benchmark shapes (32K Beta(2,8) and the 128K ragged batch of
8), and edge cases (empty heads, single tokens, page boundaries, one long head
among short ones).
"""
import pytest
import torch

from oracle import attention

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def run_and_compare(q, k, v, sl, bt, scale, label):
    import wgkv
    dev = torch.device("cuda:0")
    print(f"[decode parity] {label} q={tuple(q.shape)} pages={k.shape[0]}x{k.shape[1]}", flush=True)
    out = wgkv.paged_decode_attn(q.to(dev), k.to(dev), v.to(dev), sl.to(dev), bt.to(dev), scale)
    torch.cuda.synchronize()
    ref = attention.paged_decode(q.cpu(), k.cpu(), v.cpu(), sl.cpu(), bt.cpu(), scale)
    err = (out.float().cpu() - ref).abs()
    assert err.max().item() <= MAX_ABS, f"{label}: max_abs {err.max().item()}"
    assert err.mean().item() <= MEAN_ABS, f"{label}: mean_abs {err.mean().item()}"
    return out


def reference_grid_case(heads, D, page, B, max_len, num_blocks=4096, seed=0):
    g = torch.Generator().manual_seed(seed)
    Hq, Hkv = heads
    maxb = (max_len + page - 1) // page
    # the reference draws from a 4096-page pool; a pool of twice the pages
    # the case can use keeps the random placement and bounds host time
    num_blocks = min(num_blocks, max(256, 2 * B * Hkv * maxb))
    sl = torch.randint(1, max_len + 1, (B, Hkv), generator=g, dtype=torch.int32)
    bt = torch.empty(B, Hkv, maxb, dtype=torch.int32)
    avail = torch.randperm(num_blocks, generator=g)
    off = 0
    for b in range(B):
        for h in range(Hkv):
            n = (int(sl[b, h]) + page - 1) // page
            bt[b, h, :n] = avail[off:off + n].to(torch.int32)
            bt[b, h, n:] = -1
            off += n
    q = torch.randn(B, 1, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(num_blocks, page, D, generator=g).to(torch.bfloat16)
    v = torch.randn(num_blocks, page, D, generator=g).to(torch.bfloat16)
    return q, k, v, sl, bt


@pytest.mark.parametrize("heads", [(4, 4), (8, 2), (8, 4)])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("page", [16, 32, 64])
@pytest.mark.parametrize("B", [1, 3])
@pytest.mark.parametrize("max_len", [123, 456, 789, 4000])
def test_reference_grid(heads, D, page, B, max_len):
    q, k, v, sl, bt = reference_grid_case(heads, D, page, B, max_len, seed=hash((heads, D, page, B, max_len)) & 0xffff)
    out = run_and_compare(q, k, v, sl, bt, D ** -0.5, f"grid {heads} D{D} P{page} B{B} L{max_len}")
    # the reference test's own tolerance (utils/test_flash_attn_with_kvcache.py:134-146)
    ref = attention.paged_decode(q, k, v, sl, bt, D ** -0.5).to(torch.bfloat16)
    torch.testing.assert_close(out.cpu(), ref, atol=1e-2, rtol=1e-2)


def test_edge_lengths():
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, D, P, nb = 2, 32, 8, 128, 16, 2048
    sl = torch.tensor([[0, 1, 15, 16, 17, 63, 64, 65], [0, 0, 1023, 1024, 1025, 4095, 4096, 7000]], dtype=torch.int32)
    maxb = 7000 // 16 + 1
    bt = torch.full((B, Hkv, maxb), -1, dtype=torch.int32)
    avail = torch.randperm(nb, generator=g)
    off = 0
    for b in range(B):
        for h in range(Hkv):
            n = (int(sl[b, h]) + P - 1) // P
            bt[b, h, :n] = avail[off:off + n].to(torch.int32)
            off += n
    q = torch.randn(B, 1, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    v = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    out = run_and_compare(q, k, v, sl, bt, D ** -0.5, "edge lengths")
    assert torch.count_nonzero(out[0, 0, :4].float()) == 0      # empty head -> zeros
    assert torch.count_nonzero(out[1, 0, :8].float()) == 0


def test_one_long_head_among_short():
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, D, P = 1, 8, 2, 128, 16
    sl = torch.tensor([[200_000, 5]], dtype=torch.int32)
    nb = 200_000 // 16 + 1
    bt = torch.full((B, Hkv, nb), -1, dtype=torch.int32)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt[0, 0, :12500] = perm[:12500]
    bt[0, 1, :1] = perm[12500:12501]
    q = torch.randn(B, 1, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    v = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    run_and_compare(q, k, v, sl, bt, D ** -0.5, "one long head")


@pytest.mark.parametrize("cfg", ["beta_32k", "beta_128k", "ragged_b8_128k"])
def test_benchmark_shapes(cfg):
    from wgkv import workloads
    if cfg == "beta_32k":
        w = workloads.decode_beta(ctx=32768, device="cuda")
    elif cfg == "beta_128k":
        w = workloads.decode_beta(ctx=131072, device="cuda")
    else:
        w = workloads.decode_ragged(device="cuda")
    run_and_compare(w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table, w.softmax_scale, cfg)


def test_repeatable_bits():
    import wgkv
    from wgkv import workloads
    w = workloads.decode_ragged(ctx=32768, batch=4, device="cuda", seed=5)
    a = wgkv.paged_decode_attn(w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table, w.softmax_scale)
    b = wgkv.paged_decode_attn(w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table, w.softmax_scale)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_handle_matches_direct_call():
    import wgkv
    from wgkv import workloads
    w = workloads.decode_beta(ctx=8192, device="cuda", seed=2)
    h = wgkv.flash_attn_with_kvcache_wrapper_triton_handle(
        w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table, w.softmax_scale)
    a = h()
    b = wgkv.flash_attn_with_kvcache_wrapper(w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table, w.softmax_scale)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("heads", [(6, 2), (12, 4), (16, 2), (64, 8), (10, 2), (40, 8), (12, 2), (48, 8), (14, 2),
                                   (56, 8), (7, 1)])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("B", [1, 3])
@pytest.mark.parametrize("max_len", [123, 4000])
def test_grouped_heads_3_and_5_to_8(heads, D, B, max_len):
    """G = 3 and G = 5..8 query heads per KV head (G > 4: two MFMA head
    groups, the second partly zero rows for G = 5..7)."""
    q, k, v, sl, bt = reference_grid_case(heads, D, 16, B, max_len, seed=hash((heads, D, B, max_len, 38)) & 0xffff)
    run_and_compare(q, k, v, sl, bt, D ** -0.5, f"G{heads[0] // heads[1]} {heads} D{D} B{B} L{max_len}")


@pytest.mark.parametrize("B,Hkv", [(16, 8), (3, 32), (256, 8)])
def test_block_planner_many_heads(B, Hkv):
    """More than 64 (sequence, KV head) pairs: the plan is built by block
    scans through LDS instead of per wave; a long head split into several
    chunks; bit-identical on a second call."""
    import wgkv
    g = torch.Generator().manual_seed(B * 100 + Hkv)
    D, P = 128, 16
    Hq = Hkv * 4
    max_len = 6000 if B * Hkv <= 128 else 600
    sl = torch.randint(0, max_len + 1, (B, Hkv), generator=g, dtype=torch.int32)
    sl[0, 0] = max_len  # one head long enough to need several chunks
    maxb = (max_len + P - 1) // P
    nb = B * Hkv * maxb + 1
    bt = torch.randperm(nb, generator=g)[: B * Hkv * maxb].view(B, Hkv, maxb).to(torch.int32)
    q = torch.randn(B, 1, Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    v = torch.randn(nb, P, D, generator=g).to(torch.bfloat16)
    out = run_and_compare(q, k, v, sl, bt, D ** -0.5, f"block planner B{B} Hkv{Hkv}")
    dev = torch.device("cuda:0")
    again = wgkv.paged_decode_attn(q.to(dev), k.to(dev), v.to(dev), sl.to(dev), bt.to(dev), D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out, again)


def test_many_chunks_batch1():
    """Batch 1 at 128K context (Beta(2,8) admission, ~27K tokens per head):
    dozens of chunks per head combined by the merge; bit-identical across
    calls."""
    import wgkv
    from wgkv import workloads
    w = workloads.decode_beta(ctx=131072, device="cuda", seed=11)
    outs = [wgkv.paged_decode_attn(w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table, w.softmax_scale)
            for _ in range(3)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    run_and_compare(w.q, w.k_cache, w.v_cache, w.cache_seqlens, w.block_table, w.softmax_scale, "beta 128k seed 11")


def test_shared_workspace_across_shapes():
    """The per-head arrival counters live in the one shared workspace: calls
    that alternate between 8-wave workgroups (batch 1, few heads) and 4-wave
    ones (B*Hkv >= 32), and between head_dim 128 and 64, each match the
    oracle, and repeating the first call gives the same bits (every call
    leaves its counters zero for the next)."""
    cases = [((32, 8), 128, 16, 1, 30000, 21), ((32, 8), 64, 32, 4, 9000, 22), ((8, 2), 64, 16, 1, 20000, 23),
             ((16, 4), 128, 64, 8, 6000, 24)]
    first = None
    for heads, D, page, B, max_len, seed in cases:
        q, k, v, sl, bt = reference_grid_case(heads, D, page, B, max_len, num_blocks=1 << 30, seed=seed)
        out = run_and_compare(q, k, v, sl, bt, D ** -0.5, f"shared workspace B{B} heads{heads} D{D} page{page}")
        if first is None:
            first = (out, (q, k, v, sl, bt, D ** -0.5))
    import wgkv
    dev = torch.device("cuda:0")
    q, k, v, sl, bt, scale = first[1]
    again = wgkv.paged_decode_attn(q.to(dev), k.to(dev), v.to(dev), sl.to(dev), bt.to(dev), scale)
    torch.cuda.synchronize()
    assert torch.equal(first[0], again)
