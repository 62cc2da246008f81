"""Metadata oracle vs the reference's brute force and the ideal-mask identity.

The grid is the reference's (utils/test_sparse_indices.py:6-12,
utils/test_sparse_attn.py:7-13), thinned so the CPU suite stays fast; the
admitted set is drawn like utils/test_sparse_utils.py:13-17 (exactly
``min(global_size, S)`` random positions per head).
"""
import numpy as np
import pytest

from oracle import meta


def random_mask(B, H, S, global_size, seed):
    rng = np.random.default_rng(seed)
    m = np.zeros((B, H, S), dtype=bool)
    for b in range(B):
        for h in range(H):
            m[b, h, rng.permutation(S)[:global_size]] = True
    return m


def valid_prefixes_equal(a, b):
    bc, bo, cc, ci = a
    bc2, bo2, cc2, ci2 = b
    assert np.array_equal(bc, bc2)
    for i in range(bc.shape[2]):
        n = bc2[0, 0, i]
        assert np.array_equal(bo[0, 0, i, :n], bo2[0, 0, i, :n]), f"row {i}"
    assert np.array_equal(cc, cc2)
    B, H, R = cc.shape
    for b_ in range(B):
        for h in range(H):
            n = cc2[b_, h].max(initial=0)
            assert np.array_equal(ci[b_, h, 0, :n], ci2[b_, h, 0, :n])


SEQ = [2, 63, 64, 65, 127, 128, 129, 191, 192, 193, 255, 256, 257, 1000, 2000]


@pytest.mark.parametrize("S", SEQ)
@pytest.mark.parametrize("W", [64, 128, 256])
@pytest.mark.parametrize("global_size", [0, 123, 567, 1000])
def test_fast_matches_bruteforce(S, W, global_size):
    m = random_mask(2, 3, S, min(global_size, S), seed=S * 7 + W + global_size)
    valid_prefixes_equal(meta.generate_sparse_indices(m, W), meta.sparse_indices_bruteforce(m, W))


@pytest.mark.parametrize("S", [2, 63, 65, 128, 129, 193, 257, 700])
@pytest.mark.parametrize("W", [64, 128, 256])
@pytest.mark.parametrize("global_size", [0, 123, 345])
@pytest.mark.parametrize("G", [1, 3])
def test_metadata_mask_is_ideal_mask(S, W, global_size, G):
    m = random_mask(1, 2, S, min(global_size, S), seed=S + W * 3 + global_size)
    md = meta.generate_sparse_indices(m, W)
    built = meta.mask_from_metadata(*md, num_kv_groups=G, seq_len=S)
    assert np.array_equal(built, meta.ideal_mask(m, W, G))


def test_band_closed_form():
    # rows past the prologue start exactly at r*64 - W + 1 (src/modeling_layers.py:338-340)
    bc, bo = meta.band_blocks(256, 4096)
    P = 4
    for r in range(P, 64):
        assert bo[0, 0, r, 0] == r * 64 - 256 + 1
        assert bc[0, 0, r] == P + 1
    for r in range(P):
        assert bc[0, 0, r] == r + 1 and list(bo[0, 0, r, :r + 1]) == [64 * i for i in range(r + 1)]


def test_window_not_multiple_of_block_raises():
    with pytest.raises(AssertionError):
        meta.generate_sparse_indices(np.zeros((1, 1, 100), bool), 100)


def test_column_count_is_rank_of_band_start():
    # column_count[r] = number of admitted positions < r*64 - W + 1
    m = random_mask(1, 1, 3000, 900, seed=5)
    _, _, cc, ci = meta.generate_sparse_indices(m, 128)
    pos = np.nonzero(m[0, 0])[0]
    for r in range(cc.shape[2]):
        lo = max(0, r * 64 - 128 + 1)
        assert cc[0, 0, r] == (pos < lo).sum()
    # listed columns: every admitted position below 1 + 64*((S-1)//64), ascending
    below = pos[pos < 1 + 64 * ((3000 - 1) // 64)]
    assert np.array_equal(ci[0, 0, 0], below)


@pytest.mark.parametrize("S,W", [(300, 64), (1000, 128), (129, 256), (2, 64)])
def test_visible_pairs_counts_the_ideal_mask(S, W):
    # the closed form bench.py uses for the attention FLOP count
    import torch
    from wgkv import workloads
    gm = torch.rand(3, S, generator=torch.Generator().manual_seed(S)) < 0.3
    got = workloads.visible_pairs(gm, W).numpy()
    ref = meta.ideal_mask(gm[None].numpy(), W, 1)[0].sum(axis=(1, 2))
    assert np.array_equal(got, ref)
