"""Write-gate oracle (torch on the CPU, float32) and its float64 loop pin.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restates ``GatingRMSNorm`` (src/modeling_layers.py:113-131) and
``GatingPredictor`` (:134-205):

    x_in = concat([rms(pre_k)*w_pre, rms(post_k)*w_post (, rms(v)*w_v)])  (:173-183)
    h    = act(W1[h] @ x_in + b1[h])           grouped 1x1 conv1 (:148-154, :186-189)
    g    = sigmoid(w2[h] . h + b2[h])           grouped 1x1 conv2 (:155-161, :191-195)
    conv path only: g = max(g, g_epsilon)       (:198-205)

``rms(x) = x * rsqrt(mean(x^2) + 1e-6)`` in float32 (:123-128).  ``act`` is
``nn.GELU()`` (exact erf form) unless ``g_act_fn == "silu"`` (:154).

Parameter names and shapes are the reference's state-dict keys:
``pre_key_norm.weight (D)``, ``post_key_norm.weight (D)``,
``value_norm.weight (D)``, ``conv1.weight (Hkv*inner, n_in*D, 1)``,
``conv1.bias (Hkv*inner)``, ``conv2.weight (Hkv, inner, 1)``,
``conv2.bias (Hkv)`` with ``inner = int(D * g_expand)``.

``gate_scores`` is the graph with float32 parameters (float32 arithmetic after
the bf16 cast of the normalised inputs); ``gate_scores_bf16`` is the graph
with bf16 parameters, the reference's inference configuration, with each
op's bf16 rounding.
"""
import math

import torch

RMS_EPS = 1e-6


def rms_norm(x, weight):
    """float32 normalisation, cast back to the input dtype, then ``* weight``
    (src/modeling_layers.py:124-128): bf16 inputs see their normalised value
    rounded to bf16 before the weight; float32 inputs are unaffected."""
    in_dtype = x.dtype
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    y = (xf * torch.rsqrt(var + RMS_EPS)).to(in_dtype).to(torch.float32)
    return weight.to(torch.float32) * y


def gate_scores(pre_key, post_key, value, params, g_inputs=("pre_k", "post_k"),
                g_act_fn="gelu", fast_path=True, g_epsilon=1e-3):
    """(B,Hkv,S,D) inputs -> (B,Hkv,S) float32 scores."""
    B, H, S, D = post_key.shape
    states = []
    if "pre_k" in g_inputs:
        states.append(rms_norm(pre_key, params["pre_key_norm.weight"]))
    if "post_k" in g_inputs:
        states.append(rms_norm(post_key, params["post_key_norm.weight"]))
    if "v" in g_inputs:
        states.append(rms_norm(value, params["value_norm.weight"]))
    x = torch.cat(states, dim=-1)                       # (B,H,S,n_in*D)
    n_in = x.shape[-1]
    w1 = params["conv1.weight"].to(torch.float32).reshape(H, -1, n_in)
    b1 = params["conv1.bias"].to(torch.float32).reshape(1, H, 1, -1)
    hdn = torch.einsum("bhli,hji->bhlj", x, w1) + b1
    hdn = torch.nn.functional.silu(hdn) if g_act_fn == "silu" else torch.nn.functional.gelu(hdn)
    w2 = params["conv2.weight"].to(torch.float32).reshape(H, 1, -1)
    b2 = params["conv2.bias"].to(torch.float32).reshape(1, H, 1, 1)
    logit = torch.einsum("bhlj,hoj->bhlo", hdn, w2) + b2
    g = torch.sigmoid(logit.squeeze(-1))
    if not fast_path:
        g = torch.clamp(g, min=g_epsilon)
    return g


def _rb(x):
    """Round-to-nearest-even to bf16, kept in the container's dtype."""
    return x.to(torch.bfloat16).to(x.dtype)


def gate_scores_bf16(pre_key, post_key, value, params, g_inputs=("pre_k", "post_k"),
                     g_act_fn="gelu", fast_path=True, g_epsilon=1e-3, return_logit=False):
    """The reference's gate as its inference runs it: bf16 parameters (the
    model loads the gate checkpoint in bf16, scripts/profiling.py:222-226)
    on bf16 inputs.  Every op returns bf16, so its value is rounded once per
    op; products are accumulated here in float64 (the value an exactly
    summed float32 accumulation would round):

        x  = bf16(w_norm * bf16(rms(k)))                       (:124-128)
        fast path (:186-195): h = bf16(bf16(W1 x) + b1), a = bf16(act(h)),
                              y = bf16(bf16(w2 . a) + b2)
        conv path (:197-205): h = bf16(W1 x + b1), a = bf16(act(h)),
                              y = bf16(w2 . a + b2)
        g = bf16(sigmoid(y)); conv path: g = max(g, bf16(g_epsilon))

    The einsum / Conv1d rounding points were read off torch's CPU results
    (an einsum output is rounded before a separate bias add; a Conv1d adds
    its bias before its single rounding).  Inputs (B,H,S,D) bf16; returns
    float64 scores holding bf16 values (and, with return_logit, the bf16
    pre-sigmoid y as well)."""
    B, H, S, D = post_key.shape
    f64 = torch.float64

    def norm(x, w):
        xf = x.to(torch.float32)
        var = xf.pow(2).mean(-1, keepdim=True)
        y = (xf * torch.rsqrt(var + RMS_EPS)).to(torch.bfloat16).to(f64)
        return _rb(w.to(torch.bfloat16).to(f64) * y)

    states = []
    names = {"pre_k": (pre_key, "pre_key_norm.weight"), "post_k": (post_key, "post_key_norm.weight"),
             "v": (value, "value_norm.weight")}
    for name in ("pre_k", "post_k", "v"):
        if name in g_inputs:
            t, wname = names[name]
            states.append(norm(t, params[wname]) if wname in params else t.to(f64))
    x = torch.cat(states, dim=-1)
    n_in = x.shape[-1]
    p16 = {k: v.to(torch.bfloat16).to(f64) for k, v in params.items()}
    w1 = p16["conv1.weight"].reshape(H, -1, n_in)
    b1 = p16["conv1.bias"].reshape(1, H, 1, -1)
    acc = torch.einsum("bhli,hji->bhlj", x, w1)
    hdn = _rb(_rb(acc) + b1) if fast_path else _rb(acc + b1)
    hf = hdn.to(torch.float32)
    act = torch.nn.functional.silu(hf) if g_act_fn == "silu" else torch.nn.functional.gelu(hf)
    a = _rb(act.to(f64))
    w2 = p16["conv2.weight"].reshape(H, 1, -1)
    b2 = p16["conv2.bias"].reshape(1, H, 1, 1)
    acc2 = torch.einsum("bhlj,hoj->bhlo", a, w2)
    y = _rb(_rb(acc2) + b2) if fast_path else _rb(acc2 + b2)
    y = y.squeeze(-1)
    g = sigmoid_bf16(y, None if fast_path else g_epsilon)
    return (g, y) if return_logit else g


def sigmoid_bf16(y, clamp=None):
    """bf16(sigmoid(y)) evaluated in float32 (then max with bf16(clamp))."""
    g = _rb(torch.sigmoid(y.to(torch.float32)).to(torch.float64))
    if clamp is not None:
        g = torch.clamp(g, min=float(torch.tensor(clamp).to(torch.bfloat16)))
    return g


def bf16_threshold(threshold):
    """The threshold a bf16 score tensor is compared with: ``g > tau`` with a
    Python float promotes to the tensor's dtype, so tau is rounded to bf16
    (0.1 -> 0.10009765625)."""
    return float(torch.tensor(threshold).to(torch.bfloat16))


def bf16_midpoint_distance(y):
    """Distance of each float64 value from the nearest bf16 rounding boundary
    (the midpoint of two adjacent bf16 values), in float32 ulps of the
    value's binade.  With frexp, y = m * 2**e, 0.5 <= |m| < 1: bf16 values
    are the integers of |m| * 256 (8 significant bits) and one float32 ulp
    (24 bits) is 2**-16 of their spacing.  Zero is a bf16 value (distance
    2**15)."""
    m, _ = torch.frexp(y.to(torch.float64))
    t = m.abs() * 256.0
    return (t - torch.floor(t) - 0.5).abs() * 65536.0


def bf16_cast_ambiguous(x, ulps=4.0):
    """Per row of x (..., D): True if an element of the normalised row
    x * rsqrt(mean(x^2) + 1e-6), computed in float64, lies within ``ulps``
    float32 ulps of a bf16 rounding boundary.  Only there can a float32
    evaluation in another summation order (or with another rsqrt) round the
    element to the other bf16 neighbour when the reference casts it back to
    bf16 (src/modeling_layers.py:128); every other row's bf16 values are
    fixed by the mathematics."""
    xd = x.to(torch.float64)
    y = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + RMS_EPS)
    return (bf16_midpoint_distance(y) < ulps).any(-1)


def gate_logits(pre_key, post_key, value, params, **kw):
    """Pre-sigmoid logits (used to place the threshold at a quantile)."""
    g = gate_scores(pre_key, post_key, value, params, **kw).double()
    return torch.log(g) - torch.log1p(-g)


def gate_scores_loop(pre_key, post_key, params, g_act_fn="gelu"):
    """Scalar float64 loop of the same MLP for ('pre_k','post_k'); tiny inputs only."""
    B, H, S, D = post_key.shape
    w1 = params["conv1.weight"].double().reshape(H, -1, 2 * D)
    b1 = params["conv1.bias"].double().reshape(H, -1)
    w2 = params["conv2.weight"].double().reshape(H, -1)
    b2 = params["conv2.bias"].double()
    wp = params["pre_key_norm.weight"].double().tolist()
    wk = params["post_key_norm.weight"].double().tolist()
    out = torch.zeros(B, H, S, dtype=torch.float64)

    def norm(vec, w):
        ms = sum(t * t for t in vec) / len(vec)
        r = 1.0 / math.sqrt(ms + RMS_EPS)
        return [wi * t * r for wi, t in zip(w, vec)]

    for b in range(B):
        for h in range(H):
            inner = w1.shape[1]
            for s in range(S):
                x = norm(pre_key[b, h, s].double().tolist(), wp) + norm(post_key[b, h, s].double().tolist(), wk)
                acc = float(b2[h])
                for j in range(inner):
                    z = float(b1[h, j]) + sum(a * c for a, c in zip(w1[h, j].tolist(), x))
                    if g_act_fn == "silu":
                        a = z / (1.0 + math.exp(-z))
                    else:
                        a = 0.5 * z * (1.0 + math.erf(z / math.sqrt(2.0)))
                    acc += float(w2[h, j]) * a
                out[b, h, s] = 1.0 / (1.0 + math.exp(-acc))
    return out


def init_params(head_dim, num_kv_heads, g_expand=4.0, n_inputs=2, generator=None):
    """Random gate parameters with the reference's default init.

    ``reset_parameters`` (src/modeling_layers.py:163-168): RMSNorm weights 1,
    Conv1d default init = U(-1/sqrt(fan_in), 1/sqrt(fan_in)) for weight and
    bias, fan_in = in_channels/groups * kernel_size.
    """
    inner = int(head_dim * g_expand)
    fan1 = n_inputs * head_dim
    fan2 = inner
    b1 = 1.0 / math.sqrt(fan1)
    b2 = 1.0 / math.sqrt(fan2)

    def u(shape, bound):
        return (torch.rand(shape, generator=generator, dtype=torch.float32) * 2 - 1) * bound

    return {
        "pre_key_norm.weight": torch.ones(head_dim),
        "post_key_norm.weight": torch.ones(head_dim),
        "conv1.weight": u((num_kv_heads * inner, fan1, 1), b1),
        "conv1.bias": u((num_kv_heads * inner,), b1),
        "conv2.weight": u((num_kv_heads, inner, 1), b2),
        "conv2.bias": u((num_kv_heads,), b2),
    }


def shift_bias_to_admit(params, pre_key, post_key, value, frac=0.2, threshold=0.1):
    """Shift ``conv2.bias[h]`` so about ``frac`` of tokens score above ``threshold``.

    new_b2[h] = b2[h] + logit(threshold) - q_{1-frac}(logits over tokens of head h)
    (the config-1 recipe).  Works on a copy; returns the new params.
    """
    p = {k: v.clone() for k, v in params.items()}
    lg = gate_logits(pre_key, post_key, value, p)          # (B,H,S)
    H = lg.shape[1]
    tgt = math.log(threshold / (1 - threshold))
    for h in range(H):
        qv = torch.quantile(lg[:, h].reshape(-1), 1.0 - frac).item()
        p["conv2.bias"][h] += float(tgt - qv)
    return p
