"""BASELINE config 5 at its own length: the random-initialised bf16
Llama-3.1-8B-architecture stack (32 layers, hidden 4096, 32 q / 8 KV heads,
FFN 14336, vocab 128256), a 400,000-token prompt of uniform random ids in
4096-token chunks, deferred gating, as ``bench.py`` times it
(scripts/profiling.py:198-420 is the reference's run).

Gated run:
* every layer's prefill swap point (``prefill_wrapper``) records, on the
  device, each chunk's admitted count per KV head over the positions that
  end in the global cache ([0, S - W)); after the prompt every (layer, head)
  holds exactly that many global tokens, the ring flags are the gate's mask
  of the last W positions, and the bump pointer has handed out exactly the
  pages those lengths need;
* decode: one eager step's attention output of the first and the last layer
  meets the float32 oracle (oracle.attention.paged_decode) over the cache's
  own pages (max-abs 2e-2, mean-abs 2e-3); a second prefill of the same
  prompt decoded by replays of the captured HIP graph gives the eager steps'
  logits and tokens bit for bit.
Full run (the reference's recipe: g_expand 0, random_sparsity 0.0, so every
token is admitted): every (layer, head) holds the S - W tokens that left the
ring, all ring flags are set, and each decode step promotes one more
token."""
import math

import pytest
import torch

import parity_log

from oracle import attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
S, CHUNK, STEPS, ADMIT = 400000, 4096, 6, 0.30


def say(msg):
    print(f"[config 5 400K] {msg}", flush=True)


def record(msg):
    parity_log.report(f"[config 5 400K] {msg}")


@pytest.fixture(scope="module")
def model():
    from wgkv import e2e
    ec = e2e.E2EConfig()
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    W = ec.local_window_size
    with torch.device(DEV):
        m = e2e.LlamaLite(ec, gated=True, max_tokens_per_head=S + STEPS + 2 * W,
                          max_total_tokens=ec.num_hidden_layers * ec.num_key_value_heads * (S + STEPS + 2 * W))
    torch.set_default_dtype(prev)
    m.init_weights(seed=0)
    ids = torch.randint(0, ec.vocab_size, (1, S), generator=torch.Generator().manual_seed(0)).to(DEV)
    say("calibrating the gates")
    e2e.calibrate_gates(m, ids, ADMIT)
    yield m, ids
    del m
    torch.cuda.empty_cache()


def _size_pool(m, gated):
    W = m.cfg.local_window_size
    L, H = m.cfg.num_hidden_layers, m.cfg.num_key_value_heads
    per_head = S + STEPS + 2 * W if not gated else int(S * min(1.0, 1.5 * ADMIT)) + STEPS + 2 * W
    # the full run: the reference's recipe (README.md:128-136), every token
    # admitted by the random rule at random_sparsity 0.0, no gate
    m.cfg.g_expand = 4.0 if gated else 0.0
    m.cfg.random_sparsity = None if gated else 0.0
    m.cfg.max_tokens_per_head = S + STEPS + 2 * W
    m.cfg.max_total_tokens = L * H * per_head


def _prefill(m, ids):
    from wgkv import e2e
    from wgkv.cache import DualCache
    cache = DualCache()
    logits = None
    spans = e2e.prompt_chunks(S, CHUNK, m.cfg.local_window_size)
    for n, (c0, c1) in enumerate(spans):
        logits = m.forward_tokens(ids[:, c0:c1], c0, cache)
        if n % 32 == 0:
            say(f"prefill chunk {n + 1}/{len(spans)}")
    torch.cuda.synchronize()
    cache.raise_if_failed("400K prefill")
    return cache, logits


def _record_admission(m):
    """Wrap every layer's prefill_wrapper: per chunk add the admitted count of
    each head over [chunk start, min(chunk end, S - W)) to a device tensor,
    and keep the chunk's mask (the last chunk's holds the ring's W flags).
    Returns (counts (L, H) int64 on the device, last masks, restore)."""
    L, H, W = m.cfg.num_hidden_layers, m.cfg.num_key_value_heads, m.cfg.local_window_size
    counts = torch.zeros(L, H, dtype=torch.int64, device=DEV)
    last = [None] * L
    saved = []
    for i, layer in enumerate(m.layers):
        a = layer.self_attn
        inner = a.prefill_wrapper

        def wrapped(self, past_key_value, query_states, pre_key, key_states, value_states, batch_size, q_seq_len,
                    device, g_mask, lbph, _i=i, _inner=inner):
            c = past_key_value
            c0 = c.prefill_length if c.gated_kv_initialized else 0
            n = max(0, min(c0 + q_seq_len, S - W) - c0)
            counts[_i] += g_mask[0, :, :n].sum(-1)
            last[_i] = g_mask[0].clone()
            return _inner(self, past_key_value, query_states, pre_key, key_states, value_states, batch_size,
                          q_seq_len, device, g_mask, lbph)

        saved.append((a, inner))
        a.prefill_wrapper = wrapped

    def restore():
        for a, inner in saved:
            a.prefill_wrapper = inner
    return counts, last, restore


def _check_layer_output(cache, layer_idx, q, seqlens, table, out, scale):
    """The layer's decode attention output against the float32 oracle over
    the cache's own pages (gathered per head into a compact pool)."""
    H = seqlens.shape[1]
    P = cache.block_size
    rows_k, rows_v, tables = [], [], []
    base = 0
    maxp = 0
    for h in range(H):
        n = int(seqlens[0, h])
        pages = table[0, h, :(n + P - 1) // P].long()
        r = (pages[:, None] * P + torch.arange(P, device=DEV)[None]).reshape(-1)
        rows_k.append(cache.block_pool_k[r].cpu())
        rows_v.append(cache.block_pool_v[r].cpu())
        tables.append(torch.arange(base, base + pages.numel(), dtype=torch.int32))
        base += pages.numel()
        maxp = max(maxp, pages.numel())
    kc = torch.cat(rows_k).view(-1, P, cache.head_dim)
    vc = torch.cat(rows_v).view(-1, P, cache.head_dim)
    tb = torch.zeros(1, H, maxp, dtype=torch.int32)
    for h, t in enumerate(tables):
        tb[0, h, :t.numel()] = t
    ref = attention.paged_decode(q.cpu(), kc, vc, seqlens.cpu(), tb, scale)
    err = (out.float().cpu() - ref).abs()
    record(f"layer {layer_idx} step-1 decode vs fp32 oracle over {int(seqlens.sum())} cached tokens: "
        f"max_abs {err.max().item():.2e} mean_abs {err.mean().item():.2e}")
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3


@pytest.mark.timeout(900)
def test_config5_400k_gated(model):
    from wgkv import e2e
    m, ids = model
    L, H, W = m.cfg.num_hidden_layers, m.cfg.num_key_value_heads, m.cfg.local_window_size
    _size_pool(m, gated=True)
    counts, last, restore = _record_admission(m)
    say(f"gated: prefill {S} tokens in {CHUNK}-token chunks")
    try:
        cache, logits = _prefill(m, ids)
    finally:
        restore()
    gl = cache.global_lengths.to(torch.int64)
    assert torch.equal(gl, counts), "global lengths differ from the admitted counts"
    for l in range(L):
        assert torch.equal(cache.local_is_global[l], last[l][:, -W:]), f"ring flags of layer {l}"
    n_local = L * H * W // cache.block_size
    pages = int(((gl + cache.block_size - 1) // cache.block_size).sum())
    assert cache.next_free_block == n_local + pages
    record(f"gated: global lengths equal the admitted counts (per head {int(gl.min())}..{int(gl.max())}, "
        f"mean {gl.double().mean().item():.0f}); ring flags equal the last {W} mask bits; "
        f"{pages} global pages handed out")

    # eager decode; step 1's attention of the first and the last layer vs the oracle
    captured = {}
    watch = (0, L - 1)
    saved = []
    for l in watch:
        a = m.layers[l].self_attn
        h0, e0 = a.decode_kernel_handle, a.decode_kernel_executor

        def handle(q, k_cache, v_cache, seqlens, table, scale, _h0=h0, _l=l):
            captured[_l] = [q.clone(), seqlens.clone(), table.clone(), scale]
            return _h0(q, k_cache, v_cache, seqlens, table, scale)

        def execute(hd, _e0=e0, _l=l):
            out = _e0(hd)
            captured[_l].append(out.clone())
            return out

        saved.append((a, h0, e0))
        a.decode_kernel_handle, a.decode_kernel_executor = handle, execute
    tok = e2e.greedy_token(logits)
    eager_logits, eager_toks = [], []
    try:
        for i in range(STEPS):
            lg = m.forward_tokens(tok, S + i, cache)
            tok = e2e.greedy_token(lg)
            eager_logits.append(lg.float().clone())
            eager_toks.append(int(tok.item()))
            if i == 1:
                torch.cuda.synchronize()
                for l in watch:
                    q, sl, tb, scale, out = captured[l]
                    _check_layer_output(cache, l, q, sl, tb, out, scale)
    finally:
        for a, h0, e0 in saved:
            a.decode_kernel_handle, a.decode_kernel_executor = h0, e0
    cache.raise_if_failed("400K eager decode")
    say(f"gated: eager tokens {eager_toks}")
    del cache
    torch.cuda.empty_cache()

    # the same prompt again, decoded by graph replays
    cb, logits_b = _prefill(m, ids)
    assert torch.equal(cb.global_lengths.to(torch.int64), counts), "the second prefill admitted differently"
    gd = e2e.GraphDecoder(m, cb, e2e.greedy_token(logits_b), S, warmup=2)
    for i in range(2, STEPS):
        t = gd.step()
        assert int(t.item()) == eager_toks[i], i
        assert torch.equal(gd.logits.float(), eager_logits[i]), i
    torch.cuda.synchronize()
    cb.raise_if_failed("400K graph decode")
    record(f"gated: graph steps 2..{STEPS - 1} equal eager bit for bit")
    del gd, cb
    torch.cuda.empty_cache()


@pytest.mark.timeout(900)
def test_config5_400k_full(model):
    from wgkv import e2e
    m, ids = model
    L, H, W = m.cfg.num_hidden_layers, m.cfg.num_key_value_heads, m.cfg.local_window_size
    _size_pool(m, gated=False)
    say(f"full: prefill {S} tokens in {CHUNK}-token chunks, every token admitted")
    try:
        cache, logits = _prefill(m, ids)
        gl = cache.global_lengths
        assert int(gl.min()) == S - W and int(gl.max()) == S - W
        assert bool(cache.local_is_global.all())
        n_local = L * H * W // cache.block_size
        assert cache.next_free_block == n_local + L * H * math.ceil((S - W) / cache.block_size)
        tok = e2e.greedy_token(logits)
        for i in range(2):
            tok = e2e.greedy_token(m.forward_tokens(tok, S + i, cache))
        torch.cuda.synchronize()
        cache.raise_if_failed("400K full decode")
        assert int(cache.global_lengths.min()) == S - W + 2 and int(cache.global_lengths.max()) == S - W + 2
        record(f"full: every (layer, head) holds the {S - W} tokens that left the ring, then one more per step")
        del cache
    finally:
        m.cfg.g_expand, m.cfg.random_sparsity = 4.0, None
        torch.cuda.empty_cache()
