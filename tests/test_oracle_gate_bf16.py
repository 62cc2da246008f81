"""Pins oracle.gate.bf16_cast_ambiguous, the classifier the GPU gate tests
use to separate bf16-rounding-ambiguous tokens from the rest: exact
distances of known values from bf16 rounding boundaries, and on random bf16
rows every row whose bf16-cast normalised values differ between float32
evaluations in different summation orders (or with 1/sqrt instead of rsqrt)
is flagged."""
import torch

from oracle import gate as ogate


def test_midpoint_distance_known_values():
    f32ulp = 2.0 ** -23  # float32 ulp in [1, 2); bf16 spacing there is 2**-7
    cases = [
        (1.0, 2 ** 15),                      # a bf16 value: half a bf16 spacing from either midpoint
        (1.0 + 2 ** -8, 0),                  # the midpoint of 1 and 1 + 2**-7
        (1.0 + 2 ** -8 + 3 * f32ulp, 3),     # three float32 ulps above it
        (-(1.0 + 2 ** -8 - 5 * f32ulp), 5),  # sign does not matter
        (1.0 + 2 ** -7, 2 ** 15),            # the next bf16 value
        (1.0 - 2 ** -9, 0),                  # midpoint of 1 - 2**-8 and 1 (binade [0.5, 1))
        (0.0, 2 ** 15),
        (3 * 2 ** -20 + 2 ** -27, 0),        # a midpoint in the binade [2**-19, 2**-18) (bf16 spacing 2**-26)
    ]
    y = torch.tensor([c[0] for c in cases], dtype=torch.float64)
    d = ogate.bf16_midpoint_distance(y)
    for (v, want), got in zip(cases, d.tolist()):
        assert abs(got - want) < 1e-6, (v, want, got)


def _variants(x):
    """The normalised row rounded to bf16 under several float32 evaluations."""
    xf = x.to(torch.float32)
    D = x.shape[-1]
    sq = xf * xf
    outs = []
    for var in (sq.sum(-1, keepdim=True) / D, sq.flip(-1).cumsum(-1)[..., -1:] / D,
                (sq[..., 0::2] + sq[..., 1::2]).sum(-1, keepdim=True) / D, sq.mean(-1, keepdim=True)):
        for inv in (torch.rsqrt(var + 1e-6), 1.0 / torch.sqrt(var + 1e-6)):
            outs.append((xf * inv).to(torch.bfloat16))
    return outs


def test_rows_that_round_differently_are_flagged():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(20000, 128, generator=g).to(torch.bfloat16)
    vs = _variants(x)
    differ = torch.zeros(x.shape[0], dtype=torch.bool)
    for v in vs[1:]:
        differ |= (v != vs[0]).any(-1)
    amb = ogate.bf16_cast_ambiguous(x)
    assert int(differ.sum()) > 0, "the float32 variants should disagree on some rows"
    assert not (differ & ~amb).any(), "a row that rounds differently was not flagged"
    assert amb.float().mean().item() < 0.06  # 4 ulps either side of each boundary: a small minority
