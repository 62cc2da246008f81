"""GPU sparse prefill attention (through the C ABI) vs the oracle.

Grid after utils/test_sparse_attn.py:7-13 (batch, KV heads, groups, S, head
dim, window, admitted count; admitted set drawn like
utils/test_sparse_utils.py:13-17): every groups x head_dim pair of the
contract at every sequence length, the other parameters rotating.  Acceptance: max-abs
<= 2e-2 and mean-abs <= 2e-3 vs the fp64 masked SDPA, and the reference
test's own criterion |maxdiff(kernel) - maxdiff(bf16 SDPA)| < 0.01
(utils/test_sparse_attn.py:60-74).  The 32K-token shape is checked on a
sample of query rows against the ideal-mask definition."""
import numpy as np
import pytest
import torch

from oracle import attention, meta

pytestmark = pytest.mark.gpu


def make(B, Hkv, G, S, D, global_size, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hkv * G, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    gm = torch.zeros(B, Hkv, S, dtype=torch.bool)
    for b in range(B):
        for h in range(Hkv):
            gm[b, h, torch.randperm(S, generator=g)[:global_size]] = True
    return q, k, v, gm


def run(q, k, v, gm, W):
    import wgkv
    B, Hkv, S = gm.shape
    dev = torch.device("cuda:0")
    md = wgkv.generate_sparse_indices(gm.to(dev), W, B, Hkv, S)
    o = wgkv.sparse_attn_func(q.to(dev).transpose(1, 2), k.to(dev).transpose(1, 2), v.to(dev).transpose(1, 2),
                              *md, causal=True, return_softmax_lse=False)
    torch.cuda.synchronize()
    return o.transpose(1, 2).float().cpu()


CASES = []
# Every (G, D) pair of the reference's contract (num_kv_groups 1-4, head_dim
# 32/64/128) with every sequence length; window, admitted count, batch and
# head count rotate through their values across the cases.
_S = [2, 63, 64, 65, 127, 128, 129, 191, 192, 193, 255, 256, 257, 1000, 2000]
_W = [64, 128, 256]
_GS = [0, 123, 345, 567, 789, 1000]
_BH = [(1, 1), (2, 2), (1, 3), (1, 4), (2, 8), (1, 2)]
_i = 0
for G in [1, 2, 3, 4]:
    for D in [32, 64, 128]:
        for S in _S:
            B, Hkv = _BH[_i % len(_BH)]
            if S >= 1000 and B * Hkv * G > 8:
                B, Hkv = 1, 2
            CASES.append((B, Hkv, G, S, D, _W[_i % len(_W)], _GS[(_i // 3) % len(_GS)]))
            _i += 1

@pytest.mark.parametrize("B,Hkv,G,S,D,W,gs", CASES)
def test_reference_grid(B, Hkv, G, S, D, W, gs):
    print(f"[prefill parity] B{B} Hkv{Hkv} G{G} S{S} D{D} W{W} gs{gs}", flush=True)
    q, k, v, gm = make(B, Hkv, G, S, D, min(gs, S), seed=S * 31 + D + W + gs + G)
    out = run(q, k, v, gm, W)
    mask = meta.ideal_mask(gm.numpy(), W, G)
    ref64 = attention.masked_prefill(q, k, v, mask).float()
    bf = attention.masked_prefill(q, k, v, mask, dtype=torch.float32).to(torch.bfloat16).float()
    err = (out - ref64).abs()
    assert err.max().item() <= 2e-2, err.max().item()
    assert err.mean().item() <= 2e-3, err.mean().item()
    assert abs(err.max().item() - (bf - ref64).abs().max().item()) < 0.01


@pytest.mark.parametrize("S,W,frac", [(32768, 1024, 0.2), (8192, 1024, 1.0), (4096, 256, 0.0)])
def test_long_prompt_sampled_rows(S, W, frac):
    print(f"[prefill parity] S{S} W{W} admit{frac}", flush=True)
    g = torch.Generator().manual_seed(S)
    B, Hkv, G, D = 1, 8, 4, 128
    q = torch.randn(B, Hkv * G, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    gm = torch.rand(B, Hkv, S, generator=g) < frac
    out = run(q, k, v, gm, W)
    rows = sorted(set([0, 1, 63, 64, W - 1, W, W + 63, S // 2, S - 65, S - 64, S - 1] +
                      torch.randint(0, S, (8,), generator=g).tolist()))
    ref = attention.sparse_prefill_rows(q, k, v, gm, W, rows).float()
    err = (out[:, :, rows] - ref).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3


@pytest.mark.parametrize("D", [128, 64])
def test_wide_kv_span_matches_contiguous(D):
    """k/v whose rows span more than 2^31 bytes are loaded through the general
    64-bit address path of the one-shot kernel; the same rows stored densely
    take the 32-bit lane-offset path.  Both must give the same bits."""
    import wgkv
    print(f"[prefill wide span] D{D}", flush=True)
    dev = torch.device("cuda:0")
    B, Hkv, G, S, W = 1, 2, 4, 2048, 256
    q, k, v, gm = make(B, Hkv, G, S, D, 700, seed=97 + D)
    md = wgkv.generate_sparse_indices(gm.to(dev), W, B, Hkv, S)
    qd = q.to(dev).transpose(1, 2)
    kd = k.to(dev).transpose(1, 2).contiguous()  # (B, S, Hkv, D), token stride Hkv * D
    vd = v.to(dev).transpose(1, 2).contiguous()
    dense = wgkv.sparse_attn_func(qd, kd, vd, *md, causal=True)
    T = 1 << 19  # token stride in elements: the rows span S * T * 2 = 2^31 bytes
    assert S * T * 2 > 2**31 - 1
    wide = []
    for src in (kd, vd):
        buf = torch.empty(B, S, T, dtype=torch.bfloat16, device=dev)
        view = buf[:, :, :Hkv * D].view(B, S, Hkv, D)
        view.copy_(src)
        wide.append(view)
    assert wide[0].stride(1) == T
    out = wgkv.sparse_attn_func(qd, wide[0], wide[1], *md, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out, dense)
    mask = meta.ideal_mask(gm.numpy(), W, G)
    ref64 = attention.masked_prefill(q, k, v, mask).float()
    err = (out.transpose(1, 2).float().cpu() - ref64).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
