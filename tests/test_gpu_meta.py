"""GPU metadata builder vs the oracle (which is pinned against the
reference's brute force): the reference's grid of
utils/test_sparse_indices.py:6-12 over (batch, heads, S, W, admitted count),
plus a 400K-token case checked against the closed form."""
import numpy as np
import pytest
import torch

from oracle import meta

pytestmark = pytest.mark.gpu


def random_mask(B, H, S, global_size, seed):
    rng = np.random.default_rng(seed)
    m = np.zeros((B, H, S), dtype=bool)
    for b in range(B):
        for h in range(H):
            m[b, h, rng.permutation(S)[:global_size]] = True
    return m


def check(m, W, bs=64):
    import wgkv
    B, H, S = m.shape
    print(f"[meta parity] B{B} H{H} S{S} W{W}", flush=True)
    got = wgkv.generate_sparse_indices(torch.from_numpy(m).cuda(), W, B, H, S, block_size=bs, exact_width=True)
    got = [t.cpu().numpy() for t in got]
    ref = meta.generate_sparse_indices(m, W, bs)
    assert np.array_equal(got[0], ref[0])
    assert np.array_equal(got[1], ref[1])          # full band table, padding included
    assert np.array_equal(got[2], ref[2])
    assert got[3].shape == ref[3].shape            # exact width = reference max_global_size
    for b in range(B):
        for h in range(H):
            n = int(ref[2][b, h].max(initial=0))
            assert np.array_equal(got[3][b, h, 0, :n], ref[3][b, h, 0, :n])
            listed = np.nonzero(m[b, h])[0]
            listed = listed[listed < 1 + bs * ((S - 1) // bs)]
            assert np.array_equal(got[3][b, h, 0, :len(listed)], listed)


@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("H", [1, 3, 8])
@pytest.mark.parametrize("S", [2, 63, 64, 65, 127, 128, 129, 191, 192, 193, 255, 256, 257, 1000, 2000])
@pytest.mark.parametrize("W", [64, 128, 256])
@pytest.mark.parametrize("global_size", [0, 123, 789, 1000])
def test_reference_grid(B, H, S, W, global_size):
    check(random_mask(B, H, S, min(global_size, S), seed=B * 1000 + H * 100 + S + W + global_size), W)


@pytest.mark.parametrize("S,W", [(32768, 1024), (409600, 1024), (5000, 0)])
def test_long_prompts(S, W):
    rng = np.random.default_rng(S)
    m = rng.random((1, 8, S)) < 0.2
    check(m, W)
