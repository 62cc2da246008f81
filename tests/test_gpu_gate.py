"""GPU write gate vs the fp32 oracle and the reference-written golden scores.

Scores agree to float32 rounding (summation order differs); admission flags
are bit-exact except tokens whose oracle score lies within 1e-6 of the
threshold and, with bf16 inputs, tokens whose normalised inputs sit within a
few float32 ulps of a bf16 rounding boundary -- two sets counted and
reported separately."""
import os

import numpy as np
import pytest

import parity_log
import torch

import scenarios
from oracle import gate as ogate

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
NEAR = 1e-6


def product_gate(params, H, D, g_expand, fast=True):
    from wgkv.gate import GatingPredictor
    g = GatingPredictor(D, H, ["pre_k", "post_k"], "gelu", g_expand, 1e-3, True, fast)
    g.load_state_dict({k: v.clone() for k, v in params.items()}, strict=True)
    return g.cuda()


def compare(scores, mask, ref, thr, label, ambiguous=None):
    """|dg| <= 2e-6 and admission exact for every token except (a) tokens
    whose oracle score lies within 1e-6 of the threshold and (b) with bf16
    inputs, ``ambiguous`` tokens: an element of a normalised input lies
    within 4 float32 ulps of a bf16 rounding boundary, so the reference's
    cast back to bf16 (src/modeling_layers.py:128) may round it either way
    under another float32 summation order (oracle.gate.bf16_cast_ambiguous).
    Both sets are counted and reported separately; an ambiguous token may
    move by at most one bf16 step of one input element (|dg| <= 1e-3)."""
    s = scores.cpu().double().numpy()
    r = ref.double().numpy()
    d = np.abs(s - r)
    amb = np.zeros(r.shape, dtype=bool) if ambiguous is None else ambiguous.cpu().numpy().reshape(r.shape)
    near = np.abs(r - thr) < NEAR
    got, want = mask.cpu().numpy(), r > thr
    flips = got != want
    clean = ~amb
    dmax_clean = d[clean].max() if clean.any() else 0.0
    dmax_amb = d[amb].max() if amb.any() else 0.0
    parity_log.report(f"[gate parity] {label}: max|dg| {dmax_clean:.2e} (ambiguous tokens {dmax_amb:.2e}); "
          f"near-threshold (|g-tau|<1e-6) {int(near.sum())}; bf16-ambiguous {int(amb.sum())}; "
          f"flips among near {int((flips & near).sum())}, ambiguous {int((flips & amb & ~near).sum())}, "
          f"other {int((flips & ~near & ~amb).sum())}")
    assert dmax_clean <= 2e-6
    assert dmax_amb <= 1e-3
    assert not (flips & ~near & ~amb).any()


def bf16_ambiguous(*inputs):
    """Tokens (B, H, S) with a bf16-rounding-ambiguous normalised input row."""
    amb = None
    for x in inputs:
        a = ogate.bf16_cast_ambiguous(x)
        amb = a if amb is None else amb | a
    return amb


@pytest.mark.parametrize("name", list(scenarios.GATE_SCENARIOS))
@pytest.mark.parametrize("fast", [True, False])
def test_gate_matches_reference_golden(name, fast):
    gold = np.load(os.path.join(GOLD, "gate_golden.npz"))
    sc = scenarios.GATE_SCENARIOS[name]
    params, pre_k, post_k, value = scenarios.gate_inputs(sc)
    g = product_gate(params, sc["H"], sc["D"], sc["g_expand"], fast)
    thr = float(np.median(gold[f"{name}.fast"]))  # a threshold that splits the tokens
    scores, mask = g.scores_and_mask(pre_k.cuda(), post_k.cuda(), value.cuda(), thr)
    ref = torch.from_numpy(gold[f"{name}.{'fast' if fast else 'conv'}"])
    compare(scores, mask, ref, thr, f"{name} fast={fast}")


@pytest.mark.parametrize("D,g_expand,S,H", [(128, 4.0, 4096, 8), (64, 4.0, 2048, 2), (128, 1.5, 1000, 8), (64, 4.0, 37, 2),
                                            (128, 4.0, 1, 8), (128, 1.5, 3, 8), (64, 4.0, 4, 2), (128, 4.0, 5, 8),
                                            (64, 1.5, 300, 2), (64, 1.5, 1, 2)])  # inner 96: Qwen3 width at D 64
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gate_matches_oracle(D, g_expand, S, H, dtype):
    gen = torch.Generator().manual_seed(S + D)
    params = scenarios.gate_params(H, D, g_expand, gen)
    pre_k = torch.randn(1, H, S, D, generator=gen).to(dtype)
    post_k = torch.randn(1, H, S, D, generator=gen).to(dtype)
    g = product_gate(params, H, D, g_expand)
    # threshold at the 80th percentile, like the benchmark's ~20 % admission
    ref = ogate.gate_scores(pre_k, post_k, None, params)
    thr = float(torch.quantile(ref.flatten().double(), 0.8))
    # strided inputs: (B, S, H, D) storage seen as (B, H, S, D)
    pk = pre_k.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    kk = post_k.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    scores, mask = g.scores_and_mask(pk, kk, None, thr)
    amb = bf16_ambiguous(pre_k, post_k) if dtype == torch.bfloat16 else None
    compare(scores, mask, ref, thr, f"D{D} x{g_expand} S{S} {dtype}", ambiguous=amb)


def test_gate_forward_returns_scores_and_bf16_params():
    sc = scenarios.GATE_SCENARIOS["llama_cfg1"]
    params, pre_k, post_k, value = scenarios.gate_inputs(sc)
    g = product_gate(params, sc["H"], sc["D"], sc["g_expand"])
    a = g(pre_k.cuda(), post_k.cuda(), value.cuda())
    ref = ogate.gate_scores(pre_k, post_k, value, params)
    assert (a.cpu() - ref).abs().max().item() <= 2e-6
    # bf16 parameters (a bf16 model) are widened to fp32 for the kernel
    g16 = product_gate(params, sc["H"], sc["D"], sc["g_expand"]).to(torch.bfloat16)
    p16 = {k: v.to(torch.bfloat16).float() for k, v in params.items()}
    ref16 = ogate.gate_scores(pre_k, post_k, value, p16)
    b = g16(pre_k.cuda(), post_k.cuda(), value.cuda())
    assert (b.cpu() - ref16).abs().max().item() <= 2e-6


def test_cached_fp32_weights_follow_in_place_updates():
    """bf16 gate parameters are widened once and cached; an in-place update
    (the benchmark's bias calibration) must reach the kernel."""
    sc = scenarios.GATE_SCENARIOS["llama_cfg1"]
    params, pre_k, post_k, value = scenarios.gate_inputs(sc)
    g16 = product_gate(params, sc["H"], sc["D"], sc["g_expand"]).to(torch.bfloat16)
    first = g16(pre_k.cuda(), post_k.cuda(), value.cuda()).cpu()
    with torch.no_grad():
        g16.conv2.bias += 0.5
    p16 = {k: v.to(torch.bfloat16).float() for k, v in params.items()}
    p16["conv2.bias"] = g16.conv2.bias.detach().float().cpu()
    ref = ogate.gate_scores(pre_k, post_k, value, p16)
    second = g16(pre_k.cuda(), post_k.cuda(), value.cuda()).cpu()
    assert not torch.equal(first, second)
    assert (second - ref).abs().max().item() <= 2e-6


@pytest.mark.parametrize("g_inputs", [("pre_k", "post_k", "v"), ("post_k",), ("pre_k", "v")])
@pytest.mark.parametrize("S", [1, 3, 130])
@pytest.mark.parametrize("D", [128, 64])
def test_gate_input_sets_match_oracle(g_inputs, S, D):
    """The other input sets the reference's GatingPredictor accepts
    (src/modeling_layers.py:135-146, :170-205): one, two or three normalised
    inputs (n_in * D columns of W1), through the few-token decode kernel
    (S <= 4) and the 64-token MFMA kernel."""
    from wgkv.gate import GatingPredictor
    H, g_expand = 4, 4.0
    gen = torch.Generator().manual_seed(7 * S + D + len(g_inputs))
    g = GatingPredictor(D, H, list(g_inputs), "gelu", g_expand, 1e-3, True, True)
    params = {}
    for k, v in g.state_dict().items():
        params[k] = torch.randn(v.shape, generator=gen) * (0.05 if "conv" in k else 1.0) + (1.0 if "norm" in k else 0.0)
    g.load_state_dict(params, strict=True)
    g = g.cuda()
    pre_k, post_k, value = (torch.randn(1, H, S, D, generator=gen) for _ in range(3))
    ref = ogate.gate_scores(pre_k, post_k, value, params, g_inputs=g_inputs)
    thr = float(torch.quantile(ref.flatten().double(), 0.5))
    scores, mask = g.scores_and_mask(pre_k.cuda(), post_k.cuda(), value.cuda(), thr)
    compare(scores, mask, ref, thr, f"inputs {'+'.join(g_inputs)} D{D} S{S}")
