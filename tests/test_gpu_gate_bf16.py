"""The GPU gate with bf16 parameters (the reference's inference: its scripts
load the gate checkpoint in bf16) against scores written by the reference's
own GatingPredictor converted to bf16 (tests/golden/gate_bf16_golden.npz) and
against the oracle's restatement of its bf16 rounding points
(oracle.gate.gate_scores_bf16, which reproduces every golden bit for bit).

Every op of that module returns bf16, so each result is one rounding of a
float32 value; the kernels accumulate the two layers' products in another
order than torch, which can move a sum lying within float32 rounding of a
bf16 rounding boundary to the other neighbour.  So: scores equal the
golden's bit for bit for all but a few tokens, and each of those is the
score of a pre-sigmoid value one bf16 step from the reference's (the
sigmoid's input is bf16, so such a step moves the score by a few bf16
steps); an admission flag (score > bf16(0.1) = 0.10009765625, as a bf16
tensor compares with a Python float) differs only where the score does.  Every path is covered: the matrix-core kernel (packed one-plane
weights), the fp32-MFMA kernel (no packing) and the few-token kernel, on the
fast and the Conv1d path."""
import os

import numpy as np
import pytest
import torch

import scenarios
from oracle import gate as ogate

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
THR = 0.1


def bf16_gate(sc, params, fast):
    from wgkv.gate import GatingPredictor
    g = GatingPredictor(sc["D"], sc["H"], list(sc["g_inputs"]), sc["act"], sc["g_expand"], 1e-3, True, fast)
    g = g.to(torch.bfloat16)
    g.load_state_dict({k: v.clone() for k, v in params.items()}, strict=True)
    return g.cuda()


def bf16_step(x):
    """One bf16 step (ulp) at each value of x (float64, positive)."""
    m, e = torch.frexp(x)
    return torch.ldexp(torch.ones_like(x), e - 8)


def neighbour_scores(y, clamp):
    """The scores of the two bf16 values adjacent to y (one bit-pattern step
    either way, so the step below a power of two is the smaller one)."""
    bits = y.to(torch.bfloat16).view(torch.int16)
    a = (bits + 1).view(torch.bfloat16).double()
    b = (bits - 1).view(torch.bfloat16).double()
    return ogate.sigmoid_bf16(a, clamp), ogate.sigmoid_bf16(b, clamp)


def check(label, scores, mask, gold, thr, y=None, clamp=None):
    """Scores equal gold except at most n/500 tokens (2 at least), each of
    which lies within one bf16 step (the sigmoid's own rounding) of gold or
    of the score of a bf16 neighbour of the oracle's pre-sigmoid y;
    admission differs only where the score does."""
    s = scores.detach().cpu().double().reshape(gold.shape)
    assert torch.equal(s.to(torch.bfloat16).double(), s), "scores are not bf16 values"
    diff = s != gold
    flips = mask.cpu().reshape(gold.shape) != (gold > thr)
    n = gold.numel()
    steps = ((s - gold).abs() / bf16_step(gold))[diff]
    print(f"[gate bf16] {label}: {n} tokens, scores differ {int(diff.sum())} (max {steps.max().item() if diff.any() else 0:.0f} "
          f"score bf16 steps), admission flips {int(flips.sum())}, admitted {(gold > thr).double().mean().item():.3f}",
          flush=True)
    assert int(diff.sum()) <= max(2, n // 500)
    if diff.any():
        assert y is not None, "scores differ and no pre-sigmoid value to place them"
        lo, up = neighbour_scores(y.reshape(gold.shape), clamp)
        step = bf16_step(gold)
        near = ((s - gold).abs() <= step) | ((s - lo).abs() <= step) | ((s - up).abs() <= step)
        assert bool(near[diff].all()), "a score is further than one step from gold and from the neighbours' scores"
    assert not (flips & ~diff).any()


# few-token inputs (S <= 4) take the few-token kernel either way: one case each
CASES = [(n, p) for n, sc in scenarios.GATE_BF16_SCENARIOS.items() for p in ((True,) if sc["S"] <= 4 else (True, False))]


@pytest.mark.parametrize("name,packed", CASES)
@pytest.mark.parametrize("fast", [True, False])
def test_bf16_gate_matches_reference_golden(name, fast, packed):
    from wgkv import gate as wgate
    sc = scenarios.GATE_BF16_SCENARIOS[name]
    z = np.load(os.path.join(GOLD, "gate_bf16_golden.npz"))
    params, pre_k, post_k, value = scenarios.gate_inputs_bf16(sc)
    assert scenarios.checksum(pre_k, post_k, value, *params.values()) == bytes(z[f"{name}.inputs_sha256"]).decode()
    gold = torch.from_numpy(z[f"{name}.{'fast' if fast else 'conv'}"]).view(torch.bfloat16).double()
    orc, y = ogate.gate_scores_bf16(pre_k, post_k, value, params, g_inputs=sc["g_inputs"], g_act_fn=sc["act"],
                                    fast_path=fast, return_logit=True)
    assert torch.equal(orc, gold), "the oracle no longer reproduces the golden"
    g = bf16_gate(sc, params, fast)
    assert g.precision(torch.bfloat16) == (1 if fast else 2)
    dev = torch.device("cuda:0")
    pk, k, v = pre_k.to(dev), post_k.to(dev), value.to(dev)
    if packed:
        scores, mask = g.scores_and_mask(pk, k, v, THR)
    else:  # the fp32-MFMA kernel: same parameters, no packed copy
        wn = g._norm_weights()
        scores, mask = wgate.gate_scores_and_mask(
            pk if "pre_k" in g.g_inputs else None, k, v if "v" in g.g_inputs else None, wn[0], wn[1], wn[2],
            g._f32(g.conv1.weight), g._f32(g.conv1.bias), g._f32(g.conv2.weight), g._f32(g.conv2.bias),
            g.inner_dim, g.act, True, 0.0 if fast else 1e-3, THR, like=k, precision=1 if fast else 2)
    torch.cuda.synchronize()
    check(f"{name} {'fast' if fast else 'conv'} {'packed' if packed else 'fp32-mfma'}", scores, mask, gold,
          ogate.bf16_threshold(THR), y=y, clamp=None if fast else 1e-3)
    out = g(pk, k, v)  # the module's forward returns bf16 scores, as the reference's does
    via_module, _ = g.scores_and_mask(pk, k, v, THR)
    assert out.dtype == torch.bfloat16 and torch.equal(out.double(), via_module.double())


def test_bf16_threshold_is_compared_in_bf16():
    """With bf16 parameters the score is compared with bf16(tau): for
    tau = 0.101, bf16(tau) = 0.10107421875, so a score of exactly that value
    is not admitted (an fp32 comparison would admit it) and the next bf16
    score is.  The scores are steered through conv2.bias (conv2.weight 0):
    y = -2.1875 gives bf16(sigmoid(y)) = 0.10107421875."""
    from wgkv.gate import GatingPredictor
    H, D, tau = 2, 64, 0.101
    g = GatingPredictor(D, H, ["pre_k", "post_k"], "gelu", 4.0, 1e-3, True, True).to(torch.bfloat16).cuda()
    ys = torch.tensor([-2.1875, -2.171875], dtype=torch.bfloat16)
    with torch.no_grad():
        g.conv2.weight.zero_()
        g.conv2.bias.copy_(ys)
    x = torch.randn(1, H, 70, D, device="cuda").to(torch.bfloat16)
    for S in (70, 3):  # the matrix-core and the few-token kernel
        scores, mask = g.scores_and_mask(x[:, :, :S], x[:, :, :S], None, tau)
        want = torch.sigmoid(ys.float()).to(torch.bfloat16).double()
        assert want[0].item() == ogate.bf16_threshold(tau) == 0.10107421875
        assert torch.equal(scores[0].double().cpu(), want[:, None].expand(H, S))
        assert not bool(mask[0, 0].any()) and bool(mask[0, 1].all()), S
