"""The end-to-end decoder stack (BASELINE config-5 harness) at a small shape:
a prompt prefilled in chunks gives the same last-token logits and the same
decode logits as the prompt prefilled in one piece (the attention is
bit-identical; the dense projections see different GEMM shapes, hence the
tolerance), the gate calibration lands near the requested admission, and the
all-admitted run keeps every token."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def tiny_model(gated=True, S=1000, steps=8, W=128, layers=2, **kw):
    from wgkv import e2e
    ec = e2e.E2EConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=layers, num_attention_heads=4,
                       num_key_value_heads=2, vocab_size=1024, rope_theta=10000.0, local_window_size=W, **kw)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    with torch.device(DEV):
        m = e2e.LlamaLite(ec, gated=gated, max_tokens_per_head=S + steps + 2 * W,
                          max_total_tokens=layers * 2 * (S + steps + 2 * W))
    torch.set_default_dtype(prev)
    m.init_weights(seed=0, std=0.05)
    return m


def prefill_then_decode(m, ids, chunk, steps, feed=None):
    """Greedy decode; with ``feed`` the given tokens are fed instead (so two
    runs see the same inputs even where a near-tie flips an argmax)."""
    from wgkv.cache import DualCache
    cache = DualCache()
    S = ids.shape[1]
    logits = None
    for c0 in range(0, S, chunk):
        logits = m.forward_tokens(ids[:, c0:c0 + chunk], c0, cache)
    outs = [logits.float()]
    toks = []
    tok = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
    for i in range(steps):
        if feed is not None:
            tok = feed[i]
        toks.append(tok)
        logits = m.forward_tokens(tok, S + i, cache)
        outs.append(logits.float())
        tok = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
    torch.cuda.synchronize()
    cache.raise_if_failed("e2e test")
    return outs, cache, toks


@pytest.mark.parametrize("gated", [True, False])
def test_chunked_prefill_matches_one_shot(gated):
    from wgkv import e2e
    print(f"[e2e] tiny model gated={gated}", flush=True)
    m = tiny_model(gated)
    S = 1000
    ids = torch.randint(0, 1000, (1, S), generator=torch.Generator().manual_seed(1)).to(DEV)
    if gated:
        e2e.calibrate_gates(m, ids, 0.3, chunk=256)
    one, c1, toks = prefill_then_decode(m, ids, S, 8)
    chk, c2, _ = prefill_then_decode(m, ids, 256, 8, feed=toks)
    # the gate sees keys from GEMMs of another shape: near-threshold tokens may flip
    dl = (c1.global_lengths - c2.global_lengths).abs().max().item()
    assert dl <= 0.02 * max(1, int(c1.global_lengths.max())), dl
    for a, b in zip(one, chk):
        err = (a - b).abs().max().item()
        assert err <= 5e-2 * max(1.0, a.abs().max().item()), err
    if gated:
        frac = c1.global_lengths.float().mean().item() / (S - 128)
        assert 0.15 <= frac <= 0.45, frac
    else:
        assert int(c1.global_lengths.min()) == S + 8 - 128  # every token left the ring into the global cache


def test_run_reports():
    from wgkv import e2e
    print("[e2e] run() report fields", flush=True)
    m = tiny_model(True)
    ids = torch.randint(0, 1000, (1, 1000), generator=torch.Generator().manual_seed(2)).to(DEV)
    e2e.calibrate_gates(m, ids, 0.3, chunk=256)
    r = e2e.run(m, ids, steps=4, chunk=256, warmup_steps=1)
    assert r.prefill_ms > 0 and len(r.decode_ms) == 4 and len(r.tokens) == 4
    assert r.tokens_after >= r.tokens_before > 128  # page-granular counts
    assert r.kv_mib > 0 and r.model_mib > 0


@pytest.mark.parametrize("qwen3", [False, True])
def test_post_attention_norm_in_mlp_is_bit_identical(qwen3):
    """A decode row's post-attention RMSNorm (with the residual add) run in
    the workgroups of the gate/up product gives the logits of the separate
    norm launch bit for bit, step after step."""
    print(f"[e2e] post-attention norm inside the MLP qwen3={qwen3}", flush=True)
    m = tiny_model(True, **({"qk_norm": True, "g_expand": 1.5} if qwen3 else {}))
    ids = torch.randint(0, 1000, (1, 400), generator=torch.Generator().manual_seed(6)).to(DEV)
    outs = {}
    for fused in (True, False):
        for layer in m.layers:
            layer.post_norm_in_mlp = fused
        outs[fused], _, toks = prefill_then_decode(m, ids, 256, 6, feed=outs.get("toks"))
        outs.setdefault("toks", toks)
    for i, (a, b) in enumerate(zip(outs[True], outs[False])):
        assert torch.equal(a, b), (i, (a - b).abs().max())


@pytest.mark.parametrize("gated,qwen3", [(True, False), (False, False), (True, True)])
def test_graph_decode_matches_eager(gated, qwen3):
    """A captured decode step replayed 6 times (with eager host work and
    synchronisations between replays) gives the eager path's logits and
    tokens bit for bit, and the device ring pointers track the host's.
    qwen3: per-head q/k norms (the decode step's q/k/v product then runs
    without the fused RoPE) and gate width g_expand = 1.5."""
    from wgkv import e2e
    from wgkv.cache import DualCache
    print(f"[e2e] graph decode gated={gated} qwen3={qwen3}", flush=True)
    m = tiny_model(gated, **({"qk_norm": True, "g_expand": 1.5} if qwen3 else {}))
    S, chunk, n = 640, 256, 8  # chunks 256, 256, 128 (each >= W)
    ids = torch.randint(0, 1000, (1, S), generator=torch.Generator().manual_seed(3)).to(DEV)
    if gated:
        e2e.calibrate_gates(m, ids, 0.3, chunk=256)

    def prefill():
        c = DualCache()
        logits = None
        for c0 in range(0, S, chunk):
            logits = m.forward_tokens(ids[:, c0:c0 + chunk], c0, c)
        return c, e2e.greedy_token(logits)

    ca, tok = prefill()
    eager_logits, eager_toks = [], []
    for i in range(n):
        lg = m.forward_tokens(tok, S + i, ca)
        tok = e2e.greedy_token(lg)
        eager_logits.append(lg.float().clone())
        eager_toks.append(int(tok.item()))
    cb, tok_b = prefill()
    gd = e2e.GraphDecoder(m, cb, tok_b, S, warmup=2)
    for i in range(2, n):
        t = gd.step()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device=DEV).sum().item()  # eager work between replays
        assert int(t.item()) == eager_toks[i], i
        assert torch.equal(gd.logits.float(), eager_logits[i]), (i, (gd.logits.float() - eager_logits[i]).abs().max())
        assert cb.ring_state[:2].tolist() == [cb.local_ptr, cb.local_length]
    assert torch.equal(ca.global_lengths, cb.global_lengths)
    assert ca.local_ptr == cb.local_ptr and ca.local_length == cb.local_length


@pytest.mark.parametrize("defer,random_sparsity,qwen3", [(True, None, False), (False, None, False), (True, 0.0, False),
                                                         (True, 0.5, False), (False, 0.5, False), (True, None, True)])
def test_graph_decode_deferred_gating(defer, random_sparsity, qwen3):
    """Deferred gating (the reference profiling harness's mode): 150 captured
    decode steps with a 64-token window re-gate each layer's window twice (on
    the steps that write slot 63, decided on the device) and equal the eager
    path -- which tests the slot on the host -- bit for bit: logits, tokens,
    flags, block tables and lengths.  With immediate gating the same run
    gates every token.  With random_sparsity (the reference's random-admission
    ablation; 0.0 with g_expand 0 is its "full" recipe) the prompt is admitted
    by torch.rand draws and the decode steps by the device's counter-based
    draws, which the graph replays continue exactly as the eager steps.
    Four layers: with deferred gating the captured steps of the two middle
    layers write the ring from the q/k/v projection's launch
    (ring_write_in_projection), the eager steps by the append; with qwen3
    (per-head q/k norms, g_expand 1.5) from the launch of the norms and the
    rotation."""
    from wgkv import e2e, layers
    from wgkv.cache import DualCache
    print(f"[e2e] graph decode, g_defer={defer}, random_sparsity={random_sparsity}, qwen3={qwen3}, 150 steps, W=64",
          flush=True)
    W, S, chunk, n = 64, 640, 256, 150
    m = tiny_model(True, S=S, steps=n, W=W, layers=4, g_defer=defer,
                   **({"qk_norm": True, "g_expand": 1.5} if qwen3 else {}))
    ids = torch.randint(0, 1000, (1, S), generator=torch.Generator().manual_seed(5)).to(DEV)
    if random_sparsity is None:
        e2e.calibrate_gates(m, ids, 0.3, chunk=256)
    else:
        m.cfg.random_sparsity = random_sparsity
        if random_sparsity == 0.0:
            m.cfg.g_expand = 0.0

    def prefill():
        torch.manual_seed(11)  # the prompt's random admission draws (torch.rand)
        c = DualCache()
        logits = None
        for c0 in range(0, S, chunk):
            logits = m.forward_tokens(ids[:, c0:c0 + chunk], c0, c)
        return c, e2e.greedy_token(logits)

    ca, tok = prefill()
    assert (ca.local_pre_key is not None) == defer
    flags0 = ca.local_is_global.clone()
    eager_logits, eager_toks, refreshed = [], [], 0
    for i in range(n):
        before = ca.local_is_global.clone()
        lg = m.forward_tokens(tok, S + i, ca)
        tok = e2e.greedy_token(lg)
        eager_logits.append(lg.float().clone())
        eager_toks.append(int(tok.item()))
        if defer and not torch.equal(before, ca.local_is_global):
            refreshed += 1
            assert ca.local_ptr == 0, "flags may only change when slot W-1 was written"
    if random_sparsity == 0.0:
        assert bool(ca.local_is_global.all()) and refreshed == 0
        assert int(ca.global_lengths.min()) == S + n - W  # every token admitted
    elif defer:
        assert refreshed == 2 and not torch.equal(flags0, ca.local_is_global)
    cb, tok_b = prefill()
    gd = e2e.GraphDecoder(m, cb, tok_b, S, warmup=2)
    for i in range(2, n):
        t = gd.step()
        if i % 16 == 0:
            _ = torch.randn(1000, device=DEV).sum().item()  # eager work between replays
        assert int(t.item()) == eager_toks[i], i
        assert torch.equal(gd.logits.float(), eager_logits[i]), (i, (gd.logits.float() - eager_logits[i]).abs().max())
    torch.cuda.synchronize()
    assert torch.equal(ca.local_is_global, cb.local_is_global)
    assert torch.equal(ca.global_lengths, cb.global_lengths) and torch.equal(ca.block_table, cb.block_table)
    assert cb.ring_state[:2].tolist() == [cb.local_ptr, cb.local_length]
    rows = 4 * 2 * W  # the rings of every (layer, head): the pools' first token rows
    assert torch.equal(ca.block_pool_k[:rows], cb.block_pool_k[:rows])
    assert torch.equal(ca.block_pool_v[:rows], cb.block_pool_v[:rows])
    assert torch.equal(ca.cache_seqlens, cb.cache_seqlens)
    if defer:
        assert torch.equal(ca.local_pre_key, cb.local_pre_key)
        # the captured middle layers wrote the ring from the projection, the eager ones did not
        assert [layers.ring_write_in_projection(l.self_attn, cb) for l in m.layers] == [False, True, True, False]
        assert not layers.ring_write_in_projection(m.layers[1].self_attn, ca)


@pytest.mark.parametrize("granularity", ["rms_linear_attn", "kernel", "predictor"])
def test_timed_run_matches_untimed(granularity):
    """With the per-granularity timers installed (profiling.py
    --profile_attn_mlp), an eager run decodes the same tokens as without
    them, and attention, MLP and LM head each accumulate time in both the
    prefill and the decode phase (nothing in warm-up).  The predictor case
    gates every decode token (with deferred gating a 4-step decode calls no
    predictor, as in the reference)."""
    from wgkv import e2e
    print(f"[e2e] timed run {granularity}", flush=True)
    ids = torch.randint(0, 1000, (1, 640), generator=torch.Generator().manual_seed(4)).to(DEV)
    m = tiny_model(True, g_defer=granularity != "predictor")
    e2e.calibrate_gates(m, ids, 0.3, chunk=256)
    plain = e2e.run(m, ids, steps=4, chunk=256, warmup_steps=1)
    t = e2e.install_timing(m, granularity)
    timed = e2e.run(m, ids, steps=4, chunk=256, warmup_steps=1, timers=t)
    assert timed.tokens == plain.tokens
    rep = t.report()
    for ph in ("prefill", "decode"):
        for part in ("attn", "mlp", "lm_head"):
            assert rep[f"{ph}_{part}_ms"] > 0, (ph, part)
    assert t.phase == "warmup"
    with pytest.raises(ValueError):
        e2e.run(m, ids, steps=1, chunk=256, graph=True, timers=t)
