"""The GPU gate with bf16 parameters (the reference's inference: its scripts
load the gate checkpoint in bf16) against scores written by the reference's
own GatingPredictor converted to bf16 (tests/golden/gate_bf16_golden.npz) and
against the oracle's restatement of its bf16 rounding points
(oracle.gate.gate_scores_bf16, which reproduces every golden bit for bit).

Every op of that module returns bf16, so each result is one rounding of a
float32 value; the kernels sum the two layers' products in another float32
order than torch, which can move a value lying within float32 rounding of a
bf16 rounding boundary to the other neighbour.  oracle.gate_outcomes follows
each token through the graph with the error bounds of the kernel's own
summation order and yields the range of bf16 scores that kernel can
produce.  Asserted per token: the score lies in that range; every token the
range pins to the reference's score (all but a few per cent, printed)
carries exactly that score; admission (score > bf16(0.1) = 0.10009765625, as
a bf16 tensor compares with a Python float) follows the kernel's own score,
so it can differ from the reference's only on flagged tokens.  Every path is
covered: the matrix-core kernel (packed one-plane weights), the fp32-MFMA
kernel (no packing) and the few-token kernel, on the fast and the Conv1d
path; the kernel's GELU / SiLU table is checked against torch's entry for
entry."""
import os

import numpy as np
import pytest

import parity_log
import torch

import scenarios
from oracle import gate as ogate
from oracle import gate_outcomes as gout

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
THR = 0.1


def bf16_gate(sc, params, fast):
    from wgkv.gate import GatingPredictor
    g = GatingPredictor(sc["D"], sc["H"], list(sc["g_inputs"]), sc["act"], sc["g_expand"], 1e-3, True, fast)
    g = g.to(torch.bfloat16)
    g.load_state_dict({k: v.clone() for k, v in params.items()}, strict=True)
    return g.cuda()


def check(label, scores, mask, gold, thr, lo, hi, max_flagged_frac=0.04):
    """Per token: the kernel's score lies in [lo, hi] (oracle.gate_outcomes);
    where that range is the golden score alone the score equals it bit for
    bit; the admission flag is the kernel's own score > thr, so it differs
    from the reference's only on flagged tokens; and the flagged share stays
    below max_flagged_frac."""
    s = scores.detach().cpu().double().reshape(gold.shape)
    m = mask.cpu().reshape(gold.shape)
    assert torch.equal(s.to(torch.bfloat16).double(), s), "scores are not bf16 values"
    assert not torch.isnan(lo).any(), "tokens left unclassified"
    flagged = gout.classify(lo, hi, gold)
    diff = s != gold
    flips = m != (gold > thr)
    inside = (s >= lo) & (s <= hi)
    n = gold.numel()
    parity_log.report(f"[gate bf16] {label}: {n} tokens, flagged {int(flagged.sum())}, scores differ {int(diff.sum())} "
          f"(all flagged: {not bool((diff & ~flagged).any())}), admission flips {int(flips.sum())}, "
          f"admitted {(gold > thr).double().mean().item():.3f}")
    assert bool(inside.all()), f"{int((~inside).sum())} scores outside the range the kernel's arithmetic allows"
    assert not bool((diff & ~flagged).any()), "a score pinned to the reference's differs"
    assert torch.equal(m, s > thr), "admission does not follow the kernel's score"
    assert not bool((flips & ~flagged).any())
    assert int(flagged.sum()) <= max(1, int(n * max_flagged_frac)), "the classifier flags too many tokens"


def kernel_path(S, packed):
    """Which kernel wgkv_gate_scores runs (oracle.gate_outcomes.kernel_order)."""
    return "small" if S <= 4 else ("packed" if packed else "fp32")


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
    orc = ogate.gate_scores_bf16(pre_k, post_k, value, params, g_inputs=sc["g_inputs"], g_act_fn=sc["act"],
                                 fast_path=fast)
    assert torch.equal(orc, gold), "the oracle no longer reproduces the golden"
    order = gout.kernel_order(kernel_path(sc["S"], packed), sc["D"], len(sc["g_inputs"]), int(sc["D"] * sc["g_expand"]))
    lo, hi, _ = gout.score_range(pre_k, post_k, value, params, order, g_inputs=sc["g_inputs"], g_act_fn=sc["act"],
                                 fast_path=fast)
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
    check(f"{name} {'fast' if fast else 'conv'} {order.name}", scores, mask, gold, ogate.bf16_threshold(THR), lo, hi)
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


@pytest.mark.parametrize("act", ["gelu", "silu"])
def test_activation_table_within_float32_bounds(act):
    """The bf16 activation table the packed path reads (built on the device
    by the kernels' own activation(), after the weight plane), for every h it
    covers (|h| in [2**-16, 16), both signs): each entry lies in the bounds
    oracle.gate_outcomes.activation_bounds allows a float32 evaluation, and
    only there does it differ from torch's value."""
    from wgkv.gate import GatingPredictor
    H, D = 2, 128
    g = GatingPredictor(D, H, ["pre_k", "post_k"], act, 4.0, 1e-3, True, True).to(torch.bfloat16).cuda()
    packed = g.packed_weights(1).cpu()
    plane = H * g.inner_dim * 2 * D * 2
    n_tab = 2 * 20 * 128
    tabs = packed[plane:plane + 2 * n_tab * 2].view(torch.int16).view(2, n_tab)
    got_bits = tabs[1 if act == "silu" else 0].to(torch.int64) & 0xFFFF
    got = got_bits.to(torch.int32).to(torch.int16).view(torch.bfloat16).double()
    j = torch.arange(n_tab)
    sgn, r = j // (20 * 128), j % (20 * 128)
    bits = (sgn << 15) | ((111 + r // 128) << 7) | (r % 128)
    torch_tab = gout.activation_table(act)[bits]
    lo, hi = gout.activation_bounds(act)
    lo, hi = lo[bits], hi[bits]
    differ = got != torch_tab
    parity_log.report(f"[gate bf16] {act} table: {n_tab} entries, {int(differ.sum())} differ from torch, "
          f"{int((lo != hi).sum())} with two or more float32 outcomes")
    assert bool(((got >= lo) & (got <= hi)).all()), "a table entry outside the float32 bounds"
    assert not bool((differ & (lo == hi)).any())
