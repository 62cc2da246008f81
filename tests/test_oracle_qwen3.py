"""Pinning of the oracle's Qwen3 per-head q/k norm (src/modeling_qwen3.py:
62-76): it is the same RMSNorm formula as the gate's GatingRMSNorm
(src/modeling_layers.py:123-128; pinned by the reference's own gate golden
vectors), and with unit weights every output row has unit RMS and is
invariant to scaling the input row."""
import torch

from oracle import gate
from oracle.llama_layer import head_rms_norm


def test_same_formula_as_pinned_gate_norm():
    g = torch.Generator().manual_seed(0)
    w = 1 + 0.1 * torch.randn(64, generator=g)
    for dt in (torch.float32, torch.bfloat16):
        x = torch.randn(3, 5, 64, generator=g).to(dt)
        assert torch.equal(head_rms_norm(x, w).float(), gate.rms_norm(x, w))


def test_unit_rms_and_scale_invariance():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(7, 128, generator=g, dtype=torch.float64).float()
    y = head_rms_norm(x, torch.ones(128))
    rms = y.double().pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-5)
    assert torch.allclose(head_rms_norm(3.5 * x, torch.ones(128)), y, atol=1e-6)


def test_qk_norm_layer_takes_the_normalised_pre_key():
    """The pre-RoPE key handed to the gate is the normalised key (:236-239)."""
    from oracle.llama_layer import OracleLayer
    g = torch.Generator().manual_seed(2)
    D, Hq, Hkv, hidden = 64, 4, 2, 256
    w = {"q_proj.weight": torch.randn(Hq * D, hidden, generator=g) * 0.02,
         "k_proj.weight": torch.randn(Hkv * D, hidden, generator=g) * 0.02,
         "v_proj.weight": torch.randn(Hkv * D, hidden, generator=g) * 0.02,
         "o_proj.weight": torch.randn(hidden, Hq * D, generator=g) * 0.02,
         "q_norm.weight": torch.ones(D), "k_norm.weight": torch.ones(D)}
    o = OracleLayer(w, hidden, Hq, Hkv, D, 64, 512, qk_norm=True)
    x = torch.randn(1, 10, hidden, generator=g)
    q, pre_k, k, v = o._project(x, torch.arange(10))
    rms = pre_k.double().pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-5)
