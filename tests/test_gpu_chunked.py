"""Chunked gated prefill on the GPU vs the one-shot prefill of the same prompt.

The one-shot path (wgkv_prefill_admit + wgkv_sparse_prefill_attn) is pinned
bit for bit to the reference's golden caches and to the oracle elsewhere; a
prompt fed in chunks must leave the same dereferenced logical cache -- per
(layer, head): global length, the global entries' K/V in order, the ring, its
flags and pre-RoPE keys -- and the same bump pointer, and every chunk's
attention output must equal the one-shot rows bit for bit: the admitted
columns form the same 64-key tiles in the same order and the band tiles start
at the same positions, so the arithmetic is the same.  One case is also
checked against the fp64 ideal-mask attention.  Page numbering differs (pages
are allocated per chunk), so block tables are compared through the pages they
name."""
import pytest
import torch

from oracle import attention, meta

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def new_cache(L, H, D, W, mtph, defer=False, total_tokens=None, page=16):
    from wgkv.cache import DualCache
    from wgkv.layers import WGKVConfig
    cfg = WGKVConfig(num_hidden_layers=L, num_attention_heads=H, num_key_value_heads=H, head_dim=D,
                     hidden_size=H * D, local_window_size=W, block_size=page, max_tokens_per_head=mtph,
                     max_total_tokens=total_tokens or L * H * mtph, g_defer=defer)
    c = DualCache()
    c.initialize(cfg, D, torch.bfloat16, DEV)
    return c


def make_prompt(L, H, G, S, D, frac, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(L, H * G, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(L, H, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(L, H, S, D, generator=g).to(torch.bfloat16)
    pk = torch.randn(L, H, S, D, generator=g).to(torch.bfloat16)
    gm = torch.rand(L, H, S, generator=g) < frac
    return [t.to(DEV) for t in (q, k, v, pk, gm)]


def one_shot(c, q, k, v, pk, gm, W):
    import wgkv
    from wgkv import ops
    L, H, S, _ = k.shape
    outs = []
    for l in range(L):
        ops.prefill_admit(c, l, k[l], v[l], gm[l], pre_key=pk[l] if c.local_pre_key is not None else None)
        md = wgkv.generate_sparse_indices(gm[l:l + 1], W, 1, H, S)
        o = wgkv.sparse_attn_func(q[l:l + 1].transpose(1, 2), k[l:l + 1].transpose(1, 2),
                                  v[l:l + 1].transpose(1, 2), *md, causal=True, return_softmax_lse=False)
        outs.append(o[0])
    return outs  # L x (S, Hq, D)


def chunked(c, q, k, v, pk, gm, chunks):
    from wgkv import ops
    L = k.shape[0]
    outs = [[] for _ in range(L)]
    c0 = 0
    for C in chunks:
        for l in range(L):
            sl = slice(c0, c0 + C)
            o = ops.chunk_prefill(c, l, q[l][:, sl].transpose(0, 1), k[l][:, sl].transpose(0, 1),
                                  v[l][:, sl].transpose(0, 1), gm[l][:, sl], c0, softmax_scale=q.shape[-1] ** -0.5,
                                  pre_key=pk[l][:, sl].transpose(0, 1) if c.local_pre_key is not None else None)
            outs[l].append(o)
        c0 += C
    return [torch.cat(o, 0) for o in outs]


def global_entries(c, l, h):
    P = c.block_size
    lb = c.local_window_size // P
    n = int(c.global_lengths[l, h])
    pages = c.block_table[l, h, lb:lb + (n + P - 1) // P].long()
    rows = (pages[:, None] * P + torch.arange(P, device=DEV)[None, :]).reshape(-1)[:n]
    return c.block_pool_k[rows], c.block_pool_v[rows]


def assert_same_logical_cache(a, b):
    L, H, W = a.num_layers, a.num_kv_heads, a.local_window_size
    assert torch.equal(a.global_lengths, b.global_lengths)
    assert torch.equal(a.local_is_global, b.local_is_global)
    assert a.next_free_block == b.next_free_block
    assert int(a.status.item()) == 0 and int(b.status.item()) == 0
    ring = slice(0, L * H * W)
    assert torch.equal(a.block_pool_k[ring], b.block_pool_k[ring])
    assert torch.equal(a.block_pool_v[ring], b.block_pool_v[ring])
    if a.local_pre_key is not None:
        assert torch.equal(a.local_pre_key, b.local_pre_key)
    for l in range(L):
        for h in range(H):
            ka, va = global_entries(a, l, h)
            kb, vb = global_entries(b, l, h)
            assert torch.equal(ka, kb), (l, h)
            assert torch.equal(va, vb), (l, h)


CASES = [
    # L, H, G, D, W, chunks, admit fraction, deferred gating
    (2, 2, 4, 64, 256, [1024, 1024, 1024], 0.3, False),
    (1, 8, 4, 128, 1024, [2048, 2048, 2048, 2048], 0.2, False),
    (2, 2, 4, 64, 256, [512, 320, 1024, 333], 0.5, False),
    (2, 2, 4, 64, 128, [256, 192, 640], 0.25, True),
    (1, 3, 2, 128, 64, [64, 64, 128, 1000], 1.0, False),
    (1, 2, 1, 64, 128, [128, 256, 130], 0.0, False),
    (1, 4, 8, 128, 256, [2000], 0.2, False),
    (1, 2, 8, 128, 256, [1024, 1024, 512], 0.3, False),  # two head groups per KV head, continued chunks
    (1, 2, 3, 32, 128, [256, 320, 512], 0.3, False),     # head_dim 32, three query heads per KV head
    (1, 3, 3, 64, 64, [64, 128, 300], 0.4, True),
]


@pytest.mark.parametrize("L,H,G,D,W,chunks,frac,defer", CASES)
def test_chunked_equals_one_shot(L, H, G, D, W, chunks, frac, defer):
    print(f"[chunked prefill] L{L} H{H} G{G} D{D} W{W} chunks{chunks} admit{frac} defer{defer}", flush=True)
    S = sum(chunks)
    q, k, v, pk, gm = make_prompt(L, H, G, S, D, frac, seed=S + W + G)
    mtph = W + S
    a = new_cache(L, H, D, W, mtph, defer)
    ref = one_shot(a, q, k, v, pk, gm, W)
    b = new_cache(L, H, D, W, mtph, defer)
    got = chunked(b, q, k, v, pk, gm, chunks)
    torch.cuda.synchronize()
    assert_same_logical_cache(a, b)
    if len(chunks) == 1:
        assert torch.equal(a.block_table, b.block_table)  # one chunk = the one-shot allocation
    for l in range(L):
        assert torch.equal(got[l], ref[l]), (l, (got[l].float() - ref[l].float()).abs().max().item())


@pytest.mark.parametrize("page", [32, 64])
@pytest.mark.parametrize("L,H,G,D,W,chunks,frac,defer", [
    (2, 2, 4, 64, 256, [512, 320, 1024, 333], 0.4, False),
    (1, 4, 8, 128, 1024, [1024, 2048, 1500], 0.2, True),
    (1, 3, 3, 32, 128, [128, 192, 700], 0.6, False),
])
def test_chunked_equals_one_shot_larger_pages(L, H, G, D, W, chunks, frac, defer, page):
    """32- and 64-token pages (block_size of the reference's config): the
    chunk kernels address a head's global entries page by page, so a 1 KB
    block of four entries always lies in one page."""
    print(f"[chunked prefill] page {page} L{L} H{H} G{G} D{D} W{W} chunks{chunks} admit{frac} defer{defer}",
          flush=True)
    S = sum(chunks)
    q, k, v, pk, gm = make_prompt(L, H, G, S, D, frac, seed=S + W + G + page)
    mtph = W + S
    a = new_cache(L, H, D, W, mtph, defer, page=page)
    ref = one_shot(a, q, k, v, pk, gm, W)
    b = new_cache(L, H, D, W, mtph, defer, page=page)
    got = chunked(b, q, k, v, pk, gm, chunks)
    torch.cuda.synchronize()
    assert_same_logical_cache(a, b)
    for l in range(L):
        assert torch.equal(got[l], ref[l]), (l, (got[l].float() - ref[l].float()).abs().max().item())


def test_chunked_vs_ideal_mask():
    L, H, G, D, W, chunks = 1, 2, 4, 64, 128, [256, 256, 300]
    print(f"[chunked prefill] ideal mask W{W} chunks{chunks}", flush=True)
    S = sum(chunks)
    q, k, v, pk, gm = make_prompt(L, H, G, S, D, 0.3, seed=7)
    c = new_cache(L, H, D, W, W + S)
    out = chunked(c, q, k, v, pk, gm, chunks)[0].transpose(0, 1)[None].float().cpu()  # (1, Hq, S, D)
    torch.cuda.synchronize()
    gmc = gm[0:1].cpu()
    mask = meta.ideal_mask(gmc.numpy(), W, G)
    ref = attention.masked_prefill(q[0:1].cpu(), k[0:1].cpu(), v[0:1].cpu(), mask).float()
    err = (out - ref).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3, (err.max().item(), err.mean().item())


def test_chunk_capacity_failure_leaves_cache_unchanged():
    from wgkv import ops
    L, H, G, D, W = 1, 2, 4, 64, 128
    chunks = [512, 512]
    S = sum(chunks)
    print("[chunked prefill] capacity failure", flush=True)
    q, k, v, pk, gm = make_prompt(L, H, G, S, D, 1.0, seed=3)
    c = new_cache(L, H, D, W, mtph=W + 600, total_tokens=L * H * (W + S))
    ops.chunk_prefill(c, 0, q[0][:, :512].transpose(0, 1), k[0][:, :512].transpose(0, 1),
                      v[0][:, :512].transpose(0, 1), gm[0][:, :512], 0)
    torch.cuda.synchronize()
    assert int(c.status.item()) == 0
    before = (c.global_lengths.clone(), c.block_table.clone(), c.block_pool_k.clone(), c.local_is_global.clone(),
              c.next_free_block)
    sl = slice(512, 1024)
    out = ops.chunk_prefill(c, 0, q[0][:, sl].transpose(0, 1), k[0][:, sl].transpose(0, 1),
                            v[0][:, sl].transpose(0, 1), gm[0][:, sl], 512)
    torch.cuda.synchronize()
    assert int(c.status.item()) != 0
    assert torch.equal(before[0], c.global_lengths)
    assert torch.equal(before[1], c.block_table)
    assert torch.equal(before[2], c.block_pool_k)
    assert torch.equal(before[3], c.local_is_global)
    assert before[4] == c.next_free_block
    assert torch.isfinite(out.float()).all()
    from wgkv._lib import WGKVCapacityError
    with pytest.raises(WGKVCapacityError):
        c.raise_if_failed("chunk")


def test_layer_chunks_then_decode_match_one_shot():
    """Through prefill_wrapper (chunk continuation at cache.prefill_length) and
    decode_wrapper: the decode outputs after a chunked prompt equal those after
    the one-shot prompt."""
    import types
    import wgkv
    from wgkv import layers
    from wgkv.cache import DualCache
    L, H, G, D, W, chunks, steps = 2, 2, 4, 64, 256, [512, 256, 700], 300
    S = sum(chunks)
    print(f"[chunked prefill] layer path chunks{chunks} then {steps} decode steps", flush=True)
    q, k, v, pk, gm = make_prompt(L, H, G, S + steps, D, 0.3, seed=11)
    cfg = layers.WGKVConfig(num_hidden_layers=L, num_attention_heads=H * G, num_key_value_heads=H, head_dim=D,
                            hidden_size=H * G * D, local_window_size=W, block_size=16,
                            max_total_tokens=L * H * (S + steps + W), max_tokens_per_head=S + steps + W)

    def selves():
        out = []
        for l in range(L):
            s = types.SimpleNamespace(config=cfg, layer_idx=l, head_dim=D, scaling=D ** -0.5, num_key_value_groups=G)
            s.prefill_wrapper = layers.prefill_wrapper
            s.decode_wrapper = layers.decode_wrapper
            s.prefill_kernel = wgkv.sparse_attn_func
            s.decode_kernel_handle = wgkv.flash_attn_with_kvcache_wrapper_triton_handle
            s.decode_kernel_executor = lambda f: f()
            out.append(s)
        return out

    def run(pieces):
        c = DualCache()
        ss = selves()
        pre = [[] for _ in range(L)]
        c0 = 0
        for C in pieces:
            for l in range(L):
                sl = slice(c0, c0 + C)
                o = layers.self_attn_forward_patch_inference(
                    ss[l], c, (1, C), q[l:l + 1, :, sl], pk[l:l + 1, :, sl], k[l:l + 1, :, sl], v[l:l + 1, :, sl],
                    None, g_mask=gm[l:l + 1, :, sl])
                pre[l].append(o[0])  # (C, Hq, D)
            c0 += C
        dec = []
        for t in range(S, S + steps):
            for l in range(L):
                sl = slice(t, t + 1)
                o = layers.self_attn_forward_patch_inference(
                    ss[l], c, (1, 1), q[l:l + 1, :, sl], pk[l:l + 1, :, sl], k[l:l + 1, :, sl], v[l:l + 1, :, sl],
                    None, g_mask=gm[l:l + 1, :, sl])
                dec.append(o.float())
        torch.cuda.synchronize()
        return c, [torch.cat(p, 0) for p in pre], dec

    a, pre_a, dec_a = run([S])
    b, pre_b, dec_b = run(chunks)
    for l in range(L):
        assert torch.equal(pre_a[l], pre_b[l]), l
    assert b.prefill_length == S and a.prefill_length == S
    assert a.local_length == b.local_length and a.local_ptr == b.local_ptr
    assert torch.equal(a.global_lengths, b.global_lengths)
    for i, (x, y) in enumerate(zip(dec_a, dec_b)):
        assert torch.equal(x, y), (i, (x - y).abs().max().item())
