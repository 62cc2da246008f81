"""Host-side pieces of the end-to-end harness (no GPU): the graph-safe greedy
argmax equals torch.argmax, ties included, for vocabularies that split into
128 rows and for those that do not."""
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
