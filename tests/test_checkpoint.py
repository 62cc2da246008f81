"""Gate checkpoint loading (host only): a dict in the reference's format
(scripts/train.py:331-334: {model parameter name: parameter}) saved with
torch.save loads into the build's gates with weights_only=True, round-trips
exactly, converts dtypes, and rejects wrong shapes and missing keys."""
import pytest
import torch
import torch.nn as nn


def make_gates(L=3, H=2, D=64, g_expand=4.0, dtype=torch.float32):
    from wgkv.gate import GatingPredictor
    torch.manual_seed(0)
    return [GatingPredictor(D, H, ["pre_k", "post_k"], "gelu", g_expand, 1e-3, True, False).to(dtype)
            for _ in range(L)]


def reference_style_checkpoint(gates, seed=1):
    """What train.py saves: named Parameters of the model (gate params only)."""
    g = torch.Generator().manual_seed(seed)
    sd = {}
    for i, gp in enumerate(gates):
        for name, p in gp.named_parameters():
            sd[f"model.layers.{i}.self_attn.g_predictors.{name}"] = nn.Parameter(
                torch.randn(p.shape, generator=g, dtype=torch.float32))
    return sd


def test_round_trip_through_torch_save(tmp_path):
    from wgkv.checkpoint import load_gate_checkpoint
    gates = make_gates()
    sd = reference_style_checkpoint(gates)
    path = str(tmp_path / "other.pt")
    torch.save(sd, path)
    loaded, unexpected = load_gate_checkpoint(gates, path)
    assert unexpected == [] and len(loaded) == len(sd)
    for i, gp in enumerate(gates):
        for name, p in gp.named_parameters():
            assert torch.equal(p, sd[f"model.layers.{i}.self_attn.g_predictors.{name}"].detach())


def test_bf16_target_and_extra_keys(tmp_path):
    from wgkv.checkpoint import load_gate_checkpoint
    gates = make_gates(dtype=torch.bfloat16)
    sd = reference_style_checkpoint(gates)
    sd["model.layers.0.self_attn.duo_attn_alpha"] = torch.zeros(2)  # not a gate parameter
    path = str(tmp_path / "other.pt")
    torch.save(sd, path)
    loaded, unexpected = load_gate_checkpoint(gates, path)
    assert unexpected == ["model.layers.0.self_attn.duo_attn_alpha"]
    w = gates[1].conv1.weight
    assert w.dtype == torch.bfloat16
    assert torch.equal(w, sd["model.layers.1.self_attn.g_predictors.conv1.weight"].detach().to(torch.bfloat16))


def test_safetensors(tmp_path):
    from safetensors.torch import save_file
    from wgkv.checkpoint import load_gate_checkpoint
    gates = make_gates(L=2)
    sd = {k: v.detach().contiguous() for k, v in reference_style_checkpoint(gates).items()}
    path = str(tmp_path / "gates.safetensors")
    save_file(sd, path)
    loaded, _ = load_gate_checkpoint(gates, path)
    assert len(loaded) == len(sd)


def test_errors(tmp_path):
    from wgkv.checkpoint import load_gate_checkpoint
    gates = make_gates(L=2)
    sd = reference_style_checkpoint(gates)
    bad = dict(sd)
    bad["model.layers.0.self_attn.g_predictors.conv2.bias"] = torch.zeros(5)
    with pytest.raises(ValueError):
        load_gate_checkpoint(gates, bad)
    missing = dict(sd)
    del missing["model.layers.1.self_attn.g_predictors.conv1.bias"]
    with pytest.raises(KeyError):
        load_gate_checkpoint(gates, missing)
    loaded, _ = load_gate_checkpoint(gates, missing, strict=False)
    assert len(loaded) == len(sd) - 1
    extra = dict(sd)
    extra["model.layers.7.self_attn.g_predictors.conv1.bias"] = torch.zeros(1)
    with pytest.raises(KeyError):
        load_gate_checkpoint(gates, extra)
    with pytest.raises(FileNotFoundError):
        load_gate_checkpoint(gates, str(tmp_path / "nope.pt"))


def test_model_target_and_threshold():
    from wgkv.checkpoint import effective_threshold, load_gate_checkpoint
    from wgkv.e2e import E2EConfig, LlamaLite
    ec = E2EConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=2, num_attention_heads=2,
                   num_key_value_heads=1, vocab_size=64, local_window_size=64)
    m = LlamaLite(ec, gated=True, max_tokens_per_head=256, max_total_tokens=1024)
    gates = [layer.self_attn.g_predictors for layer in m.layers]
    sd = reference_style_checkpoint(gates)
    loaded, _ = load_gate_checkpoint(m, sd)
    assert len(loaded) == len(sd)
    assert effective_threshold(0.1, torch.bfloat16) == 0.10009765625
    assert effective_threshold(0.1, torch.float32) == pytest.approx(0.1, abs=1e-8)
