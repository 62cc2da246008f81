"""Host-side pieces of the end-to-end harness (no GPU): the graph-safe greedy
argmax equals torch.argmax, ties included, for vocabularies that split into
128 rows and for those that do not; the per-granularity timing hooks wrap
the functions the reference's profiling script names."""
import pytest
import torch


@pytest.mark.parametrize("V", [128256, 1024, 1000, 128])
def test_greedy_token_is_argmax(V):
    from wgkv import e2e
    g = torch.Generator().manual_seed(V)
    for trial in range(20):
        x = torch.randn(1, 1, V, generator=g).to(torch.bfloat16)
        if trial % 4 == 0:  # ties: the maximum repeated at random places
            j = torch.randint(0, V, (3,), generator=g)
            x[0, 0, j] = x.max() + 1
        got = e2e.greedy_token(x)
        assert got.shape == (1, 1)
        assert int(got) == int(torch.argmax(x.reshape(-1))), trial


@pytest.mark.parametrize("granularity", ["rms_linear_attn", "linear_attn", "attn", "wrapper", "kernel",
                                         "predictor"])
def test_timing_hooks_wrap_the_named_functions(granularity):
    """install_timing replaces, per layer, the attribute profiling.py's
    --attn_granularity names (:273-334) plus mlp.forward and lm_head.forward
    (:336-343); outside a timed phase each wrapper calls straight through."""
    from wgkv import e2e
    ec = e2e.E2EConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=2,
                       num_key_value_heads=1, vocab_size=64, local_window_size=64)
    m = e2e.LlamaLite(ec, gated=True, max_tokens_per_head=256, max_total_tokens=1024)
    named = {"rms_linear_attn": lambda L: (L, "rmsnorm_and_self_attn"),
             "linear_attn": lambda L: (L.self_attn, "forward"),
             "attn": lambda L: (L.self_attn, "self_attn_forward_patch"),
             "wrapper": lambda L: (L.self_attn, "decode_wrapper"),
             "kernel": lambda L: (L.self_attn, "decode_kernel_executor"),
             "predictor": lambda L: (L.self_attn.g_predictors, "scores_and_mask")}[granularity]
    before = [getattr(*named(L)) for L in m.layers]
    t = e2e.install_timing(m, granularity)
    for L, f in zip(m.layers, before):
        assert getattr(*named(L)) is not f
        assert "forward" in L.mlp.__dict__
    assert "forward" in m.lm_head.__dict__
    x = torch.randn(1, 3, 128)
    assert torch.equal(m.lm_head(x), torch.nn.functional.linear(x, m.lm_head.weight))  # pass-through
    assert t.phase == "warmup" and all(v == 0.0 for v in t.ms.values())
    with pytest.raises(ValueError):
        e2e.install_timing(m, "layer")


def test_prompt_chunks_fold_short_tail_and_reject_bad_sizes():
    """Chunk spans of e2e.run: contiguous, covering the prompt, every chunk
    after the first 64-aligned and at least W long (a short tail joins the
    chunk before it); impossible chunk sizes fail before any prefill work."""
    from wgkv import e2e
    W = 1024
    for S in (400000, 4096 * 3 + 100, 4096 * 3 + 1024, 5000, 700, 4096):
        spans = e2e.prompt_chunks(S, 4096, W)
        assert spans[0][0] == 0 and spans[-1][1] == S
        assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
        assert all(c0 % 64 == 0 and c1 - c0 >= W for c0, c1 in spans[1:])
    assert e2e.prompt_chunks(4096 * 3 + 100, 4096, W)[-1] == (4096 * 2, 4096 * 3 + 100)
    for bad in (1000, 4000, 512):
        with pytest.raises(ValueError):
            e2e.prompt_chunks(10000, bad, W)
