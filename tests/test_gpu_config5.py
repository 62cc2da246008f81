"""BASELINE config 5's model shape on the GPU: a random-initialised bf16
Llama-3.1-8B-architecture stack (32 layers, hidden 4096, 32 q / 8 KV heads,
head_dim 128, FFN 14336, vocab 128256) around the write-gated path, an 8K
prompt in 4096-token chunks, short enough to replay every layer's cache on
the CPU oracle (tests/test_gpu_config5_400k.py checks the config's own 400K
prompt by admitted counts, ring flags, page accounting, decode outputs and
graph replays).

Checked:
* gated: every layer's logical cache (global lengths, global K/V in order,
  ring, flags, pre-RoPE keys of the deferred gate) equals a DualCacheOracle
  replay of the keys, values and masks that layer's gate produced;
* full (every token admitted): every token has left the ring into the global
  cache of every (layer, head);
* decode: steps replayed from the captured HIP graph give the eager steps'
  logits and tokens bit for bit."""
import numpy as np
import pytest
import torch

from oracle.dualcache import DualCacheOracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
S, CHUNK, STEPS = 8192, 4096, 6


def build(gated):
    from wgkv import e2e
    ec = e2e.E2EConfig()
    W = ec.local_window_size
    mtph = S + STEPS + 2 * W
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    with torch.device(DEV):
        m = e2e.LlamaLite(ec, gated=gated, max_tokens_per_head=mtph,
                          max_total_tokens=ec.num_hidden_layers * ec.num_key_value_heads * mtph)
    torch.set_default_dtype(prev)
    m.init_weights(seed=0)
    return m


def record_prefill_inputs(model):
    """Wrap every layer's prefill_wrapper swap point to keep (keys, values,
    pre-RoPE keys, mask) of each chunk on the host."""
    rec = [[] for _ in model.layers]
    for i, layer in enumerate(model.layers):
        a = layer.self_attn
        inner = a.prefill_wrapper

        def wrapped(self, past_key_value, query_states, pre_key, key_states, value_states, batch_size, q_seq_len,
                    device, g_mask, lbph, _i=i, _inner=inner):
            rec[_i].append((key_states[0].cpu(), value_states[0].cpu(),
                            None if pre_key is None else pre_key[0].to(torch.bfloat16).cpu(), g_mask[0].cpu()))
            return _inner(self, past_key_value, query_states, pre_key, key_states, value_states, batch_size,
                          q_seq_len, device, g_mask, lbph)

        a.prefill_wrapper = wrapped
    return rec


@pytest.mark.timeout(900)
def test_config5_shape_gated_cache_matches_oracle_replay():
    from wgkv import e2e
    from wgkv.cache import DualCache
    print(f"[config 5 shape] gated, 32 layers, {S}-token prompt in {CHUNK}-token chunks", flush=True)
    m = build(True)
    ids = torch.randint(0, m.ec.vocab_size, (1, S), generator=torch.Generator().manual_seed(0)).to(DEV)
    e2e.calibrate_gates(m, ids, 0.3, chunk=CHUNK)
    rec = record_prefill_inputs(m)
    cache = DualCache()
    for c0 in range(0, S, CHUNK):
        m.forward_tokens(ids[:, c0:c0 + CHUNK], c0, cache)
    torch.cuda.synchronize()
    cache.raise_if_failed("config-5 prefill")
    W, L, H = cache.local_window_size, cache.num_layers, cache.num_kv_heads
    assert cache.local_pre_key is not None  # deferred gating, as the reference's profiling run
    adm = []
    for l in range(L):
        k = torch.cat([r[0] for r in rec[l]], 1)
        v = torch.cat([r[1] for r in rec[l]], 1)
        pk = torch.cat([r[2] for r in rec[l]], 1)
        gm = torch.cat([r[3] for r in rec[l]], 1)
        orc = DualCacheOracle(1, H, cache.head_dim, W, H * cache.max_tokens_per_head, cache.max_tokens_per_head,
                              g_defer=True, dtype=torch.bfloat16)
        orc.prefill(0, k, v, gm, pre_key=pk)
        assert np.array_equal(cache.global_lengths[l].cpu().numpy(), orc.global_lengths[0].numpy()), l
        assert np.array_equal(cache.local_is_global[l].cpu().numpy(), orc.local_is_global[0].numpy()), l
        assert torch.equal(cache.local_pre_key[l].cpu(), orc.local_pre_key[0]), l
        ring = slice(l * H * W, (l + 1) * H * W)
        assert torch.equal(cache.block_pool_k[ring].cpu(), orc.block_pool_k[:H * W]), l
        assert torch.equal(cache.block_pool_v[ring].cpu(), orc.block_pool_v[:H * W]), l
        lb = W // 16
        for h in range(H):
            n = int(orc.global_lengths[0, h])
            ids_o = orc.block_table[0, h, lb:lb + (n + 15) // 16].long()
            r_o = (ids_o[:, None] * 16 + torch.arange(16)[None]).reshape(-1)[:n]
            ids_c = cache.block_table[l, h, lb:lb + (n + 15) // 16].long()
            r_c = (ids_c[:, None] * 16 + torch.arange(16, device=DEV)[None]).reshape(-1)[:n]
            assert torch.equal(cache.block_pool_k[r_c].cpu(), orc.block_pool_k[r_o]), (l, h)
            assert torch.equal(cache.block_pool_v[r_c].cpu(), orc.block_pool_v[r_o]), (l, h)
        adm.append(gm[:, :S - W].float().mean().item())
    print(f"[config 5 shape] every layer's logical cache equals the oracle replay; admitted per layer "
          f"{min(adm):.3f}..{max(adm):.3f}", flush=True)
    assert 0.15 < float(np.mean(adm)) < 0.45


@pytest.mark.timeout(900)
@pytest.mark.parametrize("gated", [True, False])
def test_config5_shape_graph_decode_and_full_run(gated):
    from wgkv import e2e
    from wgkv.cache import DualCache
    print(f"[config 5 shape] gated={gated}: eager vs graph decode, {STEPS} steps", flush=True)
    m = build(gated)
    ids = torch.randint(0, m.ec.vocab_size, (1, S), generator=torch.Generator().manual_seed(1)).to(DEV)
    if gated:
        e2e.calibrate_gates(m, ids, 0.3, chunk=CHUNK)

    def prefill():
        c = DualCache()
        logits = None
        for c0 in range(0, S, CHUNK):
            logits = m.forward_tokens(ids[:, c0:c0 + CHUNK], c0, c)
        return c, e2e.greedy_token(logits)

    ca, tok = prefill()
    W = ca.local_window_size
    if not gated:
        assert int(ca.global_lengths.min()) == S - W and int(ca.global_lengths.max()) == S - W
    eager_logits, eager_toks = [], []
    for i in range(STEPS):
        lg = m.forward_tokens(tok, S + i, ca)
        tok = e2e.greedy_token(lg)
        eager_logits.append(lg.float().clone())
        eager_toks.append(int(tok.item()))
    if not gated:  # each step promotes the token leaving the ring
        assert int(ca.global_lengths.min()) == S + STEPS - W
    del ca
    torch.cuda.empty_cache()
    cb, tok_b = prefill()
    gd = e2e.GraphDecoder(m, cb, tok_b, S, warmup=2)
    for i in range(2, STEPS):
        t = gd.step()
        assert int(t.item()) == eager_toks[i], i
        assert torch.equal(gd.logits.float(), eager_logits[i]), i
    torch.cuda.synchronize()
    cb.raise_if_failed("config-5 decode")
    print(f"[config 5 shape] gated={gated}: graph steps equal eager bit for bit", flush=True)
