"""Loading trained write-gate checkpoints into the gates of this build.

The reference trains only the gate parameters and saves them with
``torch.save`` as one dict ``{parameter name: tensor}`` (scripts/train.py:
331-334, file ``other.pt``); its harnesses load that dict into the model with
``load_state_dict(strict=False)`` (scripts/inference.py:79-80,
scripts/profiling.py:225-226).  The keys are the model's parameter names, e.g.
``model.layers.3.self_attn.g_predictors.conv1.weight`` — conv1/conv2
weight and bias plus the RMSNorm weights ``pre_key_norm``, ``post_key_norm``
and ``value_norm`` (src/modeling_layers.py:148-160).

``load_gate_checkpoint`` reads such a file from a local path only, with
loaders that execute nothing from the file (``torch.load(weights_only=True)``
or safetensors), matches the keys to the gates of a model (anything with a
``layers[i].self_attn.g_predictors``) or of a list of GatingPredictors, checks
every shape and copies the tensors in, converting to the gates' dtype.

Threshold in bf16 models: the reference compares bf16 scores with the Python
float ``g_threshold`` (:1465), which PyTorch rounds to the tensor's dtype, so
the effective threshold of a bf16 model is bf16(0.1) = 0.10009765625.
``effective_threshold`` returns that value; the kernels compare in fp32.
"""
import os
import re

import torch

_KEY = re.compile(r"(?:^|\.)layers\.(\d+)\.self_attn\.g_predictors\.(.+)$")


def effective_threshold(threshold, dtype):
    """The threshold a ``scores > threshold`` comparison uses for scores of
    ``dtype`` (a Python float is rounded to the tensor's dtype)."""
    return float(torch.tensor(threshold, dtype=dtype).item())


def read_state_dict(path):
    """The checkpoint's tensors, read without executing code from the file."""
    if not os.path.isfile(path):
        raise FileNotFoundError(path)
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        return load_file(path, device="cpu")
    sd = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(sd, dict):
        raise TypeError(f"{path}: expected a dict of tensors, got {type(sd).__name__}")
    return sd


def _gates_of(target):
    if isinstance(target, (list, tuple)):
        return list(target)
    layers = getattr(target, "layers", None)
    if layers is None and hasattr(target, "model"):
        layers = getattr(target.model, "layers", None)
    if layers is None:
        raise TypeError("target must be a list of GatingPredictors or a model with .layers[i].self_attn")
    return [getattr(layer.self_attn, "g_predictors", None) for layer in layers]


@torch.no_grad()
def load_gate_checkpoint(target, path_or_state_dict, strict=True):
    """Copy a reference gate checkpoint into ``target``'s gates.

    Returns (loaded keys, keys of the checkpoint that are not gate parameters).
    With ``strict``, every gate parameter of every layer must be present and a
    gate key naming a layer or parameter the target lacks raises KeyError;
    shape mismatches always raise ValueError."""
    sd = path_or_state_dict if isinstance(path_or_state_dict, dict) else read_state_dict(path_or_state_dict)
    gates = _gates_of(target)
    loaded, unexpected = [], []
    seen = set()
    for key, value in sd.items():
        m = _KEY.search(key)
        if m is None:
            unexpected.append(key)
            continue
        layer, name = int(m.group(1)), m.group(2)
        if layer >= len(gates) or gates[layer] is None:
            if strict:
                raise KeyError(f"{key}: the target has no gate for layer {layer}")
            unexpected.append(key)
            continue
        params = dict(gates[layer].named_parameters())
        if name not in params:
            if strict:
                raise KeyError(f"{key}: gate parameter {name!r} does not exist")
            unexpected.append(key)
            continue
        p = params[name]
        v = value.detach() if isinstance(value, torch.Tensor) else torch.as_tensor(value)
        if tuple(v.shape) != tuple(p.shape):
            raise ValueError(f"{key}: shape {tuple(v.shape)} != {tuple(p.shape)}")
        p.copy_(v.to(device=p.device, dtype=p.dtype))
        loaded.append(key)
        seen.add((layer, name))
    if strict:
        missing = [f"layers.{i}.self_attn.g_predictors.{n}" for i, g in enumerate(gates) if g is not None
                   for n, _ in g.named_parameters() if (i, n) not in seen]
        if missing:
            raise KeyError(f"checkpoint lacks {len(missing)} gate parameters, e.g. {missing[:3]}")
    return loaded, unexpected
