"""Oracle vs golden vectors written by the reference's own code.

The fixtures under tests/golden/ were produced by make_golden.py, which runs
the reference's GatingPredictor and its dual-cache state machine on seeded
inputs; here the oracle replays the same inputs and must agree exactly.
"""
import json
import os

import numpy as np
import pytest
import torch

import scenarios
from oracle import gate
from oracle.dualcache import CapacityError, DualCacheOracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def gate_gold():
    return np.load(os.path.join(GOLD, "gate_golden.npz"))


@pytest.fixture(scope="module")
def cache_gold():
    with open(os.path.join(GOLD, "cache_golden.json")) as f:
        meta = json.load(f)
    return np.load(os.path.join(GOLD, "cache_golden.npz")), meta


@pytest.mark.parametrize("name", list(scenarios.GATE_SCENARIOS))
def test_gate_oracle_matches_reference(gate_gold, name):
    sc = scenarios.GATE_SCENARIOS[name]
    params, pre_k, post_k, value = scenarios.gate_inputs(sc)
    sha = bytes(gate_gold[f"{name}.inputs_sha256"]).decode()
    assert sha == scenarios.checksum(pre_k, post_k, *params.values()), "RNG stream changed"
    fast = gate.gate_scores(pre_k, post_k, value, params, fast_path=True)
    conv = gate.gate_scores(pre_k, post_k, value, params, fast_path=False)
    assert np.allclose(fast.numpy(), gate_gold[f"{name}.fast"], rtol=0, atol=2e-6)
    assert np.allclose(conv.numpy(), gate_gold[f"{name}.conv"], rtol=0, atol=2e-6)
    # admission at tau=0.1 is identical away from the threshold
    ref = gate_gold[f"{name}.fast"]
    far = np.abs(ref - 0.1) > 1e-6
    assert np.array_equal((fast.numpy() > 0.1)[far], (ref > 0.1)[far])


@pytest.mark.parametrize("name", list(scenarios.GATE_BF16_SCENARIOS))
def test_bf16_gate_oracle_matches_reference_bit_for_bit(name):
    """oracle.gate.gate_scores_bf16 (the rounding points of the reference's
    module in bf16) reproduces every bf16 score the reference wrote, on the
    fast and the Conv1d path; the golden admission is score > bf16(0.1)."""
    z = np.load(os.path.join(GOLD, "gate_bf16_golden.npz"))
    sc = scenarios.GATE_BF16_SCENARIOS[name]
    params, pre_k, post_k, value = scenarios.gate_inputs_bf16(sc)
    assert bytes(z[f"{name}.inputs_sha256"]).decode() == scenarios.checksum(pre_k, post_k, value, *params.values())
    for fast in (True, False):
        gold = torch.from_numpy(z[f"{name}.{'fast' if fast else 'conv'}"]).view(torch.bfloat16).double()
        got = gate.gate_scores_bf16(pre_k, post_k, value, params, g_inputs=sc["g_inputs"], g_act_fn=sc["act"],
                                    fast_path=fast)
        assert torch.equal(got, gold), (name, fast)
        # the fp32-parameter graph differs: bf16 rounding moves scores by more than float32 noise
        if sc["S"] > 4:
            f32 = gate.gate_scores(pre_k, post_k, value, {k: v.float() for k, v in params.items()},
                                   g_inputs=sc["g_inputs"], g_act_fn=sc["act"], fast_path=fast).double()
            assert (f32 - gold).abs().max().item() > 1e-4


def test_bf16_threshold_rounds_like_torch():
    assert gate.bf16_threshold(0.1) == 0.10009765625
    x = torch.tensor([0.10009765625, 0.1005859375], dtype=torch.bfloat16)
    assert (x > 0.1).tolist() == [x[i].item() > gate.bf16_threshold(0.1) for i in range(2)] == [False, True]


def test_gate_oracle_matches_float64_loop():
    sc = dict(scenarios.GATE_SCENARIOS["llama_cfg1"], S=6)
    params, pre_k, post_k, value = scenarios.gate_inputs(sc)
    a = gate.gate_scores(pre_k, post_k, value, params).double()
    b = gate.gate_scores_loop(pre_k, post_k, params)
    assert torch.allclose(a, b, atol=1e-6)


def test_gate_closed_form_zero_w1():
    # W1 = 0: every token of head h scores sigmoid(b2 + sum_j w2_j * gelu(b1_j))
    params, pre_k, post_k, value = scenarios.gate_inputs(scenarios.GATE_SCENARIOS["llama_cfg1"])
    params["conv1.weight"].zero_()
    g = gate.gate_scores(pre_k, post_k, value, params).double()
    H = 2
    b1 = params["conv1.bias"].double().view(H, -1)
    w2 = params["conv2.weight"].double().view(H, -1)
    expect = torch.sigmoid((w2 * torch.nn.functional.gelu(b1)).sum(-1) + params["conv2.bias"].double())
    assert torch.allclose(g[0], expect[:, None].expand_as(g[0]), atol=1e-6)


def replay(sc, inp, max_tokens_per_head=None):
    L, H, D, W = sc["L"], sc["H"], sc["D"], sc["W"]
    mtp = max_tokens_per_head or sc["max_tokens_per_head"]
    c = DualCacheOracle(L, H, D, W, L * H * mtp, mtp, g_defer=sc["g_defer"])
    gates = None
    if sc["g_defer"]:
        gates = [scenarios.defer_bias_shift(p) for p in inp["gates"]]

    def regate(layer, pk, k, v):
        s = gate.gate_scores(pk[None], k[None], v[None], gates[layer])
        return s[0] > 0.1

    for l in range(L):
        q, pk, k, v, mask = inp["prompt"][l]
        c.prefill(l, k[0], v[0], mask[0], pre_key=pk[0])
    snap = (c.block_table.clone(), c.global_lengths.clone(), c.local_is_global.clone(),
            c.next_free_block, c.local_ptr, c.local_length)
    seqlens, tables = [], []
    for step in inp["steps"]:
        for l in range(L):
            q, pk, k, v, mask = step[l]
            sl, bt = c.decode(l, k[0, :, 0], v[0, :, 0], None if mask is None else mask[0, :, 0],
                              pre_key=pk[0, :, 0], regate=regate)
            seqlens.append(sl)
            tables.append(bt.unsqueeze(0))
    return c, snap, seqlens, tables


@pytest.mark.parametrize("name", list(scenarios.CACHE_SCENARIOS))
def test_dualcache_oracle_matches_reference(cache_gold, name):
    gold, meta = cache_gold
    sc = scenarios.CACHE_SCENARIOS[name]
    inp = scenarios.cache_inputs(sc)
    sha = scenarios.checksum(*[t for lay in inp["prompt"] for t in lay],
                             *[t for st in inp["steps"] for lay in st for t in lay if t is not None])
    assert sha == meta[name]["inputs_sha256"], "RNG stream changed"
    c, snap, seqlens, tables = replay(sc, inp)
    bt, gl, lig, nfb, lp, ll = snap
    assert np.array_equal(bt.numpy(), gold[f"{name}.after_prefill.block_table"])
    assert np.array_equal(gl.numpy(), gold[f"{name}.after_prefill.global_lengths"])
    assert np.array_equal(lig.numpy(), gold[f"{name}.after_prefill.local_is_global"])
    assert (nfb, lp, ll) == tuple(meta[f"{name}.after_prefill"][k]
                                  for k in ("next_free_block", "local_ptr", "local_length"))
    assert np.array_equal(c.block_table.numpy(), gold[f"{name}.final.block_table"])
    assert np.array_equal(c.global_lengths.numpy(), gold[f"{name}.final.global_lengths"])
    assert np.array_equal(c.local_is_global.numpy(), gold[f"{name}.final.local_is_global"])
    assert np.array_equal(torch.stack(seqlens).numpy(), gold[f"{name}.decode_seqlens"])
    assert scenarios.checksum(*tables) == bytes(gold[f"{name}.decode_block_table_sha256"]).decode()
    assert c.next_free_block == meta[name]["next_free_block"]
    assert (c.local_ptr, c.local_length) == (meta[name]["local_ptr"], meta[name]["local_length"])
    parts = []
    for l in range(sc["L"]):
        for h in range(sc["H"]):
            parts.extend(c.logical_cache(l, h, c.local_length))
    assert scenarios.checksum(*parts) == meta[name]["logical_sha256"]


def test_dualcache_capacity_error(cache_gold):
    _, meta = cache_gold
    assert meta["capacity_error_raises"]
    sc = scenarios.CACHE_SCENARIOS["long_prompt"]
    inp = scenarios.cache_inputs(sc)
    with pytest.raises(CapacityError):
        replay(sc, inp, max_tokens_per_head=256)


@pytest.mark.parametrize("name", list(scenarios.CACHE_SCENARIOS))
def test_dualcache_invariants(name):
    sc = scenarios.CACHE_SCENARIOS[name]
    inp = scenarios.cache_inputs(sc)
    c, _, seqlens, _ = replay(sc, inp)
    P, W = 16, sc["W"]
    lb = W // P
    used = 0
    for l in range(sc["L"]):
        for h in range(sc["H"]):
            gl = int(c.global_lengths[l, h])
            if c.local_length < W:
                assert gl == 0
            n = (gl + P - 1) // P
            used += n
            row = c.block_table[l, h]
            assert (row[:lb] == torch.arange(lb) + (l * sc["H"] + h) * lb).all()
            assert (row[lb + n:] == c.total_blocks - 1).all()   # sentinel never mapped
            assert (row[lb:lb + n] < c.total_blocks - 1).all()
    assert c.next_free_block - sc["L"] * sc["H"] * lb == used
