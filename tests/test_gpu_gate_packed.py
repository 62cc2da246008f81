"""The gate's bf16 matrix-core path: packed first-layer weights
(wgkv_gate_pack_weights) and wgkv_gate_scores with w1_packed.

The packed buffer must hold, for every weight, three bf16 planes whose sum is
exactly the fp32 product w_norm[d] * conv1.weight[h*inner + j][i*D + d], the
first plane being that product's nearest bf16 (checked against torch's own
fp32 -> bf16 conversion); the buffer is unpacked here from its documented
lane layout, so a wrong index fails the exact-sum check.  Scores of the
packed path meet the oracle to the bf16-input tolerance of the fp32 path
(tests/test_gpu_gate.py), with admission exact away from the threshold."""
import numpy as np
import pytest
import torch

import scenarios
from oracle import gate as ogate
from test_gpu_gate import bf16_ambiguous, compare

pytestmark = pytest.mark.gpu


def make_gate(g_inputs, H, D, g_expand, gen, rms=True):
    from wgkv.gate import GatingPredictor
    g = GatingPredictor(D, H, list(g_inputs), "gelu", g_expand, 1e-3, rms, True)
    params = {}
    for k, v in g.state_dict().items():
        if "norm" in k:
            params[k] = 1.0 + 0.1 * torch.randn(v.shape, generator=gen)
        elif "conv1" in k:
            params[k] = (torch.rand(v.shape, generator=gen) * 2 - 1) / np.sqrt(len(g_inputs) * D)
        else:
            params[k] = (torch.rand(v.shape, generator=gen) * 2 - 1) / np.sqrt(int(D * g_expand))
    g.load_state_dict(params, strict=True)
    return g.cuda(), params


def unpack(packed, H, inner, K):
    """(H, 3, inner, K) float64 planes from the packed layout
    [h][16-column tile][32-input k-step][plane][lane = kg*16 + n][8]."""
    u = packed.cpu().numpy().view(np.uint16).reshape(H, inner // 16, K // 32, 3, 4, 16, 8)
    # -> [h][plane][tile][n][k-step][kg][e]
    u = u.transpose(0, 3, 1, 5, 2, 4, 6).reshape(H, 3, inner, K)
    return (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("g_inputs,D,g_expand,rms", [
    (("pre_k", "post_k"), 128, 4.0, True),
    (("pre_k", "post_k", "v"), 64, 1.5, True),
    (("post_k",), 128, 1.5, True),
    (("pre_k", "post_k"), 64, 4.0, False),
])
def test_packed_planes_are_exact_split(g_inputs, D, g_expand, rms):
    from wgkv import gate as wgate
    H = 4
    gen = torch.Generator().manual_seed(D + len(g_inputs) + int(rms))
    g, params = make_gate(g_inputs, H, D, g_expand, gen, rms)
    inner = int(D * g_expand)
    K = len(g_inputs) * D
    names = {"pre_k": "pre_key_norm.weight", "post_k": "post_key_norm.weight", "v": "value_norm.weight"}
    wn = [params[names[n]].cuda() if rms and n in g_inputs else None for n in ("pre_k", "post_k", "v")]
    w1 = params["conv1.weight"].reshape(H * inner, K).contiguous()
    packed = wgate.pack_weights(wn[0], wn[1], wn[2], w1.cuda(), g_inputs, rms, H, D, inner)
    torch.cuda.synchronize()
    planes = unpack(packed, H, inner, K)
    # the fold in fp32 (one rounding, as on the device)
    scale = torch.cat([params[names[n]] if rms else torch.ones(D) for n in g_inputs])
    fold = (w1.view(H, inner, K) * scale).numpy().astype(np.float64)
    assert np.array_equal(planes.sum(axis=1), fold), "hi + mid + lo must equal the folded weight exactly"
    hi_ref = torch.from_numpy(fold.astype(np.float32)).to(torch.bfloat16).float().numpy().astype(np.float64)
    assert np.array_equal(planes[:, 0], hi_ref), "the first plane is the nearest bf16 of the folded weight"
    mid_ref = torch.from_numpy((fold - planes[:, 0]).astype(np.float32)).to(torch.bfloat16).float().numpy()
    assert np.array_equal(planes[:, 1], mid_ref.astype(np.float64))
    print(f"[gate pack] {'+'.join(g_inputs)} D{D} inner{inner} rms={rms}: {fold.size} weights split exactly, "
          f"max|lo|/|w| = {np.max(np.abs(planes[:, 2]) / np.maximum(np.abs(fold), 1e-30)):.2e}", flush=True)


@pytest.mark.parametrize("g_inputs,D,g_expand,S", [
    (("pre_k", "post_k"), 128, 4.0, 4096),
    (("pre_k", "post_k"), 128, 4.0, 37),
    (("pre_k", "post_k", "v"), 64, 1.5, 300),
    (("post_k",), 128, 1.5, 5),
    (("pre_k", "v"), 64, 4.0, 130),
])
def test_packed_path_matches_oracle_and_fp32_path(g_inputs, D, g_expand, S):
    from wgkv import gate as wgate
    H = 8 if D == 128 else 2
    gen = torch.Generator().manual_seed(S + D)
    g, params = make_gate(g_inputs, H, D, g_expand, gen)
    pre_k, post_k, value = (torch.randn(1, H, S, D, generator=gen).to(torch.bfloat16) for _ in range(3))
    ref = ogate.gate_scores(pre_k, post_k, value, params, g_inputs=g_inputs)
    thr = float(torch.quantile(ref.flatten().double(), 0.8))
    # (B, S, H, D) storage seen as (B, H, S, D), as the layer passes keys
    dev = [t.transpose(1, 2).contiguous().cuda().transpose(1, 2) for t in (pre_k, post_k, value)]
    scores, mask = g.scores_and_mask(dev[0], dev[1], dev[2], thr)
    assert g.__dict__.get("_packed_cache") is not None, "bf16 inputs of more than 4 tokens take the packed path"
    used = {"pre_k": pre_k, "post_k": post_k, "v": value}
    amb = bf16_ambiguous(*(used[n] for n in g_inputs))
    compare(scores, mask, ref, thr, f"packed {'+'.join(g_inputs)} D{D} S{S}", ambiguous=amb)
    # the fp32 MFMA path on the same inputs (no packed weights)
    norms = [g.pre_key_norm, g.post_key_norm, g.value_norm]
    wn = [m.weight.detach() if isinstance(m, wgate.GatingRMSNorm) else None for m in norms]
    use = {n: t for n, t in zip(("pre_k", "post_k", "v"), dev)}
    s32, m32 = wgate.gate_scores_and_mask(
        use["pre_k"] if "pre_k" in g_inputs else None, use["post_k"] if "post_k" in g_inputs else None,
        use["v"] if "v" in g_inputs else None, wn[0], wn[1], wn[2],
        g.conv1.weight.detach(), g.conv1.bias.detach(), g.conv2.weight.detach(), g.conv2.bias.detach(),
        g.inner_dim, g.act, True, 0.0, thr, like=dev[1])
    compare(s32, m32, ref, thr, f"fp32 path {'+'.join(g_inputs)} D{D} S{S}", ambiguous=amb)
    d = (scores - s32).abs()
    print(f"[gate packed vs fp32 path] max|dg|={d.max().item():.2e} tokens |dg|>2e-6: "
          f"{(d > 2e-6).float().mean().item():.4%}", flush=True)
    assert (d > 2e-6).float().mean().item() <= 0.01


def test_packed_weights_follow_in_place_updates_and_misaligned_inputs_fall_back():
    """An in-place change of conv1.weight or a norm weight remakes the packed
    copy; inputs whose rows are not 16-byte aligned take the fp32 path."""
    H, D, S = 4, 128, 256
    gen = torch.Generator().manual_seed(11)
    g, params = make_gate(("pre_k", "post_k"), H, D, 4.0, gen)
    pre_k, post_k = (torch.randn(1, H, S, D, generator=gen).to(torch.bfloat16) for _ in range(2))
    pk, kk = pre_k.cuda(), post_k.cuda()
    first, _ = g.scores_and_mask(pk, kk, None, 0.5)
    with torch.no_grad():
        g.conv1.weight.mul_(1.5)
        g.post_key_norm.weight.add_(0.05)
    p2 = {k: v.detach().cpu().clone() for k, v in g.state_dict().items()}
    ref = ogate.gate_scores(pre_k, post_k, None, p2)
    second, mask = g.scores_and_mask(pk, kk, None, 0.5)
    assert not torch.equal(first, second)
    amb = bf16_ambiguous(pre_k, post_k)
    compare(second, mask, ref, 0.5, "packed after in-place updates", ambiguous=amb)
    # rows starting 2 bytes past a 16-byte boundary: no packed read, same results
    buf = torch.empty(2, H * S * D + 1, dtype=torch.bfloat16, device="cuda")
    pk_m = buf[0, 1:].view(1, H, S, D)
    kk_m = buf[1, 1:].view(1, H, S, D)
    pk_m.copy_(pk)
    kk_m.copy_(kk)
    third, mask3 = g.scores_and_mask(pk_m, kk_m, None, 0.5)
    compare(third, mask3, ref, 0.5, "misaligned inputs (fp32 path)", ambiguous=amb)


def test_packed_path_without_rms_matches_fp32_path():
    """g_rms = False (no input norms, GatingPredictor's Identity norms): the
    packed planes hold conv1.weight itself and the scores equal the fp32
    MFMA path's to fp32 rounding (both multiply the bf16 inputs exactly)."""
    from wgkv import gate as wgate
    H, D, S = 8, 128, 1024
    gen = torch.Generator().manual_seed(21)
    g, params = make_gate(("pre_k", "post_k"), H, D, 4.0, gen, rms=False)
    pre_k, post_k = (torch.randn(1, H, S, D, generator=gen).to(torch.bfloat16).cuda() for _ in range(2))
    scores, mask = g.scores_and_mask(pre_k, post_k, None, 0.5)
    assert g.__dict__.get("_packed_cache") is not None
    s32, m32 = wgate.gate_scores_and_mask(pre_k, post_k, None, None, None, None, g.conv1.weight.detach(),
                                          g.conv1.bias.detach(), g.conv2.weight.detach(), g.conv2.bias.detach(),
                                          g.inner_dim, g.act, False, 0.0, 0.5, like=post_k)
    d = (scores - s32).abs().max().item()
    print(f"[gate packed, no rms] max|dg| vs fp32 path = {d:.2e}", flush=True)
    assert d <= 2e-6
    near = (s32 - 0.5).abs() < 1e-6
    assert torch.equal(mask[~near], m32[~near])
