"""Seeded input scenarios shared by the golden-vector writer and the tests.

Inputs are regenerated from ``torch.Generator`` seeds (CPU Mersenne
Twister); each fixture stores a checksum of its inputs so a change of RNG
stream is detected instead of silently compared.
"""
import hashlib

import numpy as np
import torch

# name -> scenario description (all batch 1, the reference's inference batch)
CACHE_SCENARIOS = {
    # prompt longer than the window: prefill scatter + migration every step
    "long_prompt": dict(L=2, H=2, G=2, D=64, W=128, S=1000, steps=200, rates=(0.2, 0.5),
                        step_rate=0.3, max_tokens_per_head=4096, g_defer=False, seed=1),
    # prompt shorter than the window: ring fills during decode, then migrates
    "short_prompt": dict(L=2, H=2, G=2, D=64, W=128, S=100, steps=160, rates=(0.3, 0.6),
                         step_rate=0.5, max_tokens_per_head=4096, g_defer=False, seed=2),
    # deferred gating: decode steps carry no scores, the full window is re-gated
    "defer": dict(L=2, H=2, G=2, D=64, W=64, S=300, steps=150, rates=(0.25, 0.25),
                  step_rate=None, max_tokens_per_head=4096, g_defer=True, seed=3),
    # three layers, page-boundary lengths
    "three_layers": dict(L=3, H=2, G=1, D=64, W=64, S=64 * 7 + 16, steps=70, rates=(0.5, 0.0625),
                         step_rate=0.25, max_tokens_per_head=2048, g_defer=False, seed=4),
}

GATE_SCENARIOS = {
    "llama_cfg1": dict(H=2, D=64, g_expand=4.0, S=384, seed=10),
    "qwen3_like": dict(H=2, D=128, g_expand=1.5, S=96, seed=11),
}

# The gate with bf16 parameters on bf16 inputs (the reference's inference
# configuration).  conv2.bias is shifted by logit(0.1) so that the scores sit
# around the threshold and admission is decided at every bf16 step near it.
GATE_BF16_SCENARIOS = {
    "llama8b": dict(H=2, D=128, g_expand=4.0, S=2048, seed=20, g_inputs=("pre_k", "post_k"), act="gelu"),
    "qwen3": dict(H=2, D=128, g_expand=1.5, S=1024, seed=21, g_inputs=("pre_k", "post_k"), act="gelu"),
    "d64_kv_silu": dict(H=2, D=64, g_expand=4.0, S=1024, seed=22, g_inputs=("pre_k", "post_k", "v"), act="silu"),
    "decode": dict(H=8, D=128, g_expand=4.0, S=3, seed=23, g_inputs=("pre_k", "post_k"), act="gelu"),
}


def checksum(*tensors):
    h = hashlib.sha256()
    for t in tensors:
        if t is None:
            continue
        a = t.detach().contiguous()
        if a.dtype == torch.bfloat16:
            a = a.view(torch.int16)
        h.update(a.numpy().tobytes())
    return h.hexdigest()


def gate_params(H, D, g_expand, gen):
    inner = int(D * g_expand)
    b1 = 1.0 / np.sqrt(2 * D)
    b2 = 1.0 / np.sqrt(inner)
    return {
        "pre_key_norm.weight": 1.0 + 0.1 * torch.randn(D, generator=gen),
        "post_key_norm.weight": 1.0 + 0.1 * torch.randn(D, generator=gen),
        "conv1.weight": (torch.rand(H * inner, 2 * D, 1, generator=gen) * 2 - 1) * b1,
        "conv1.bias": (torch.rand(H * inner, generator=gen) * 2 - 1) * b1,
        "conv2.weight": (torch.rand(H, inner, 1, generator=gen) * 2 - 1) * b2,
        "conv2.bias": (torch.rand(H, generator=gen) * 2 - 1) * b2,
    }


def gate_inputs(sc):
    gen = torch.Generator().manual_seed(sc["seed"])
    H, D, S = sc["H"], sc["D"], sc["S"]
    params = gate_params(H, D, sc["g_expand"], gen)
    pre_k = torch.randn(1, H, S, D, generator=gen)
    post_k = torch.randn(1, H, S, D, generator=gen)
    value = torch.randn(1, H, S, D, generator=gen)
    return params, pre_k, post_k, value


# SnapKV eviction states: pages of each head's global tokens scattered over
# the pool, a free list already holding two pages, a full query window.
SNAPKV_SCENARIOS = {
    "bf16_k5": dict(L=2, H=2, G=2, D=64, W=64, lengths=((300, 517), (16, 2)), win=32, ksz=5, ratio=0.3,
                    dtype="bf16", seed=30),
    "bf16_k1": dict(L=2, H=2, G=2, D=64, W=64, lengths=((301, 160), (47, 0)), win=16, ksz=1, ratio=0.25,
                    dtype="bf16", seed=31),
    "f32_k5": dict(L=1, H=2, G=2, D=64, W=64, lengths=((257, 400),), win=32, ksz=5, ratio=0.4, dtype="f32", seed=32),
    "d128_g4": dict(L=1, H=2, G=4, D=128, W=128, lengths=((700, 129),), win=48, ksz=3, ratio=0.5, dtype="bf16",
                    seed=33),
    "ratio1": dict(L=1, H=2, G=1, D=64, W=64, lengths=((40, 33),), win=16, ksz=5, ratio=1.0, dtype="bf16", seed=34),
}


# QUEST page selection: cache states with page key bounds, and per scenario
# a list of (local tokens, token budget) decode steps, each with its own query.
QUEST_SCENARIOS = {
    "g4_d128": dict(H=3, G=4, D=128, W=64, lengths=(700, 129, 64), dtype="bf16", seed=40,
                    steps=((64, 320), (17, 200), (64, 40), (1, 4096), (33, 120))),
    "g2_d64_f32": dict(H=2, G=2, D=64, W=64, lengths=(500, 33), dtype="f32", seed=41,
                       steps=((64, 256), (5, 100), (64, 64))),
    "g1_d64": dict(H=2, G=1, D=64, W=64, lengths=(256, 255), dtype="bf16", seed=42,
                   steps=((64, 128), (64, 150), (10, 4000))),
}


def quest_state(sc):
    """One layer's cache state for a QUEST scenario: pool_k, block_table
    (1, H, max_pages), global_lengths (1, H), key_min / key_max (total_blocks,
    D) -- the min / max over each global page's valid rows, as the
    reference's prefill writes them -- and one query (H*G, D) per step."""
    gen = torch.Generator().manual_seed(sc["seed"])
    H, G, D, W, P = sc["H"], sc["G"], sc["D"], sc["W"], 16
    lengths = torch.tensor([sc["lengths"]], dtype=torch.int32)
    lb = W // P
    maxp = lb + (int(lengths.max()) + P - 1) // P + 1
    total = H * lb + int(((lengths + P - 1) // P).sum()) + 4
    perm = torch.randperm(total - 1 - H * lb, generator=gen) + H * lb
    table = torch.full((1, H, maxp), total - 1, dtype=torch.int32)
    table[0, :, :lb] = torch.arange(H * lb, dtype=torch.int32).view(H, lb)
    at = 0
    for h in range(H):
        np_ = (int(lengths[0, h]) + P - 1) // P
        table[0, h, lb:lb + np_] = perm[at:at + np_].to(torch.int32)
        at += np_
    pool_k = torch.randn(total * P, D, generator=gen).to(torch.bfloat16)
    kmin = torch.zeros(total, D, dtype=torch.bfloat16)
    kmax = torch.zeros(total, D, dtype=torch.bfloat16)
    for h in range(H):
        n = int(lengths[0, h])
        for p in range((n + P - 1) // P):
            pg = int(table[0, h, lb + p])
            rows = pool_k[pg * P:pg * P + min(P, n - p * P)]
            kmin[pg], kmax[pg] = rows.amin(0), rows.amax(0)
    qs = [torch.randn(H * G, D, generator=gen).to(torch.bfloat16) for _ in sc["steps"]]
    if sc["dtype"] == "f32":
        pool_k, kmin, kmax, qs = pool_k.float(), kmin.float(), kmax.float(), [q.float() for q in qs]
    return dict(pool_k=pool_k, block_table=table, global_lengths=lengths, key_min=kmin, key_max=kmax, qs=qs,
                total_blocks=total)


def snapkv_state(sc):
    """A dual-cache state for a SnapKV scenario: dict with pool_k, pool_v
    ((total_blocks*16, D); bf16, or fp32 holding bf16 values), block_table
    int32 (L, H, max_pages) (W/16 ring pages, then the global pages, the
    sentinel total_blocks-1 after them), global_lengths int32 (L, H),
    free_ids (list), total_blocks, qbuf (L, win, H*G, D) like the pool."""
    gen = torch.Generator().manual_seed(sc["seed"])
    L, H, G, D, W, P = sc["L"], sc["H"], sc["G"], sc["D"], sc["W"], 16
    lengths = torch.tensor(sc["lengths"], dtype=torch.int32)
    lb = W // P
    maxp = lb + (int(lengths.max()) + P - 1) // P + 2
    need = L * H * lb + int(((lengths + P - 1) // P).sum())
    total = need + 6
    perm = torch.randperm(total - 1 - L * H * lb, generator=gen) + L * H * lb  # pages past the ring pages
    table = torch.full((L, H, maxp), total - 1, dtype=torch.int32)
    table[:, :, :lb] = torch.arange(L * H * lb, dtype=torch.int32).view(L, H, lb)
    at = 0
    for l in range(L):
        for h in range(H):
            np_ = (int(lengths[l, h]) + P - 1) // P
            table[l, h, lb:lb + np_] = perm[at:at + np_].to(torch.int32)
            at += np_
    free_ids = [int(x) for x in perm[at:at + 2]]
    dt = torch.bfloat16
    pool_k = torch.randn(total * P, D, generator=gen).to(dt)
    pool_v = torch.randn(total * P, D, generator=gen).to(dt)
    qbuf = (1.5 * torch.randn(L, sc["win"], H * G, D, generator=gen)).to(dt)
    if sc["dtype"] == "f32":
        pool_k, pool_v, qbuf = pool_k.float(), pool_v.float(), qbuf.float()
    return dict(pool_k=pool_k, pool_v=pool_v, block_table=table, global_lengths=lengths.clone(), free_ids=free_ids,
                total_blocks=total, qbuf=qbuf)


def logical_tokens(pool, table, lengths, lb, P=16):
    """Per (layer, head) the (n, D) rows of the head's global tokens in order."""
    D = pool.shape[1]
    out = {}
    L, H = lengths.shape
    for l in range(L):
        for h in range(H):
            n = int(lengths[l, h])
            ids = table[l, h, lb:lb + (n + P - 1) // P].long()
            out[(l, h)] = pool.view(-1, P, D)[ids].reshape(-1, D)[:n]
    return out


def gate_inputs_bf16(sc):
    """bf16 parameters (the fp32 draw of gate_params, rounded, conv2.bias
    shifted by logit(0.1)) and bf16 (1, H, S, D) inputs."""
    gen = torch.Generator().manual_seed(sc["seed"])
    H, D, S = sc["H"], sc["D"], sc["S"]
    params = gate_params(H, D, sc["g_expand"], gen)
    if len(sc["g_inputs"]) == 3:
        inner = int(D * sc["g_expand"])
        b1 = 1.0 / np.sqrt(3 * D)
        params["value_norm.weight"] = 1.0 + 0.1 * torch.randn(D, generator=gen)
        params["conv1.weight"] = (torch.rand(H * inner, 3 * D, 1, generator=gen) * 2 - 1) * b1
    params["conv2.bias"] = params["conv2.bias"] - 2.1972245773362196
    params = {k: v.to(torch.bfloat16) for k, v in params.items()}
    pre_k = torch.randn(1, H, S, D, generator=gen).to(torch.bfloat16)
    post_k = torch.randn(1, H, S, D, generator=gen).to(torch.bfloat16)
    value = torch.randn(1, H, S, D, generator=gen).to(torch.bfloat16)
    return params, pre_k, post_k, value


def cache_inputs(sc):
    """Prompt tensors, per-step tensors and masks for a cache scenario.

    Returns dict with ``prompt`` = (q, pre_k, k, v, mask) and ``steps`` =
    list of (q, pre_k, k, v, mask-or-None) per step, one entry per layer.
    Masks are drawn directly (rate per head) so the cache logic is tested
    independently of the gate; the deferred scenario re-gates with a gate of
    ``gate_params`` whose bias is shifted per layer.
    """
    gen = torch.Generator().manual_seed(sc["seed"])
    L, H, G, D, S = sc["L"], sc["H"], sc["G"], sc["D"], sc["S"]
    Hq = H * G

    def bf(*shape):
        return torch.randn(*shape, generator=gen).to(torch.bfloat16)

    prompt = []
    for _ in range(L):
        q, pk, k, v = bf(1, Hq, S, D), bf(1, H, S, D), bf(1, H, S, D), bf(1, H, S, D)
        rates = torch.tensor(sc["rates"], dtype=torch.float32)[:H].view(1, H, 1)
        mask = torch.rand(1, H, S, generator=gen) < rates
        prompt.append((q, pk, k, v, mask))
    steps = []
    for _ in range(sc["steps"]):
        per_layer = []
        for _ in range(L):
            q, pk, k, v = bf(1, Hq, 1, D), bf(1, H, 1, D), bf(1, H, 1, D), bf(1, H, 1, D)
            mask = None
            if sc["step_rate"] is not None:
                mask = torch.rand(1, H, 1, generator=gen) < sc["step_rate"]
            per_layer.append((q, pk, k, v, mask))
        steps.append(per_layer)
    gates = None
    if sc["g_defer"]:
        gates = []
        for _ in range(L):
            p = gate_params(H, D, 4.0, gen)
            gates.append(p)
    return {"prompt": prompt, "steps": steps, "gates": gates}


def defer_bias_shift(gate_params_, shift=-0.25):
    """A fixed bias shift so that a fraction of the window is re-admitted."""
    p = {k: v.clone() for k, v in gate_params_.items()}
    p["conv2.bias"] = p["conv2.bias"] + shift
    return p
