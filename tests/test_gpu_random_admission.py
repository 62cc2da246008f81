"""The random_sparsity ablation's decode-time draws (wgkv_random_admission,
the device form of get_random_g_scores, src/modeling_layers.py:1160-1166):

* the rule: random_sparsity 0 admits every token and 1 none (the reference's
  r >= p with r in [0, 1)), and bf16(p) is the cut, as the reference's bf16
  comparison makes it;
* the generator: the flags equal a host restatement of the documented
  counter-based draws (SplitMix64 finaliser of seed + (counter * 2^32 +
  index + 1) * 0x9E3779B97F4A7C15, top 24 bits), each call advances the
  counter, an inactive call (device flag mismatch) writes nothing and does
  not advance it;
* the draws are uniform: admitted shares and a chi-square over 16 bins of r."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
M64 = (1 << 64) - 1


def host_draws(seed, counter, H, n):
    """r of every (h, i) of one call, restated with Python integers."""
    out = np.empty((H, n))
    base = (seed + (counter << 32)) & M64
    for j in range(H * n):
        z = (base + (j + 1) * 0x9E3779B97F4A7C15) & M64
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        z ^= z >> 31
        out[j // n, j % n] = (z >> 40) / 16777216.0
    return out


def bf16(x):
    return float(torch.tensor(x).to(torch.bfloat16))


def test_rule_and_generator():
    from wgkv import ops
    H, n, seed = 3, 200, 12345
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    flags = torch.zeros(H, n, dtype=torch.bool, device=DEV)
    for call, p in enumerate([0.0, 1.0, 0.3, 0.3, 0.7, 0.123]):
        ops.random_admission(flags, p, seed, counter)
        want = host_draws(seed, call, H, n) >= bf16(p)
        got = flags.cpu().numpy()
        assert np.array_equal(got, want), (call, p)
        assert int(counter.item()) == call + 1
        if p == 0.0:
            assert got.all()
        if p == 1.0:
            assert not got.any()
    print(f"[random admission] 6 calls equal the host restatement; counter {int(counter.item())}", flush=True)


def test_inactive_call_writes_nothing():
    from wgkv import ops
    counter = torch.full((1,), 5, dtype=torch.int32, device=DEV)
    flags = torch.zeros(2, 64, dtype=torch.bool, device=DEV)
    gate = torch.tensor([3], dtype=torch.int32, device=DEV)
    ops.random_admission(flags, 0.0, 1, counter, active=(gate, 4))
    assert not bool(flags.any()) and int(counter.item()) == 5
    ops.random_admission(flags, 0.0, 1, counter, active=(gate, 3))
    assert bool(flags.all()) and int(counter.item()) == 6


def test_draws_are_uniform():
    from wgkv import ops
    H, n = 8, 4096
    counter = torch.zeros(1, dtype=torch.int32, device=DEV)
    flags = torch.zeros(H, n, dtype=torch.bool, device=DEV)
    shares = []
    for p in (0.25, 0.5, 0.9):
        ops.random_admission(flags, p, 99, counter)
        shares.append(flags.float().mean().item())
    for p, s in zip((0.25, 0.5, 0.9), shares):
        assert abs(s - (1 - bf16(p))) < 0.01, (p, s)
    r = host_draws(99, 0, H, n).ravel()
    hist = np.histogram(r, bins=16, range=(0.0, 1.0))[0]
    e = r.size / 16
    chi2 = float(((hist - e) ** 2 / e).sum())
    print(f"[random admission] shares {shares}, chi-square over 16 bins {chi2:.1f}", flush=True)
    assert chi2 < 37.7  # 15 degrees of freedom, p = 0.001
