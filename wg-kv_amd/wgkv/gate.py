"""The write gate as a module with the reference's parameters.

Parameter names and shapes are GatingPredictor's (src/modeling_layers.py:
134-161), so gate checkpoints (keys ``...g_predictors.pre_key_norm.weight``,
``.post_key_norm.weight``, ``.conv1.{weight,bias}``, ``.conv2.{weight,bias}``)
load with ``load_state_dict``.  The forward runs the HIP kernel
``wgkv_gate_scores`` in the arithmetic the parameters' dtype gives the
reference's module: fp32 parameters compute in fp32 (fp32 scores); bf16
parameters on bf16 inputs -- the reference's inference, whose scripts load
the gate checkpoint in bf16 -- round every op's result to bf16 at the points
torch does and compare the bf16 score with bf16(g_threshold) (precision
1 = g_fast_path, 2 = the Conv1d path).  Parameters reach the kernel as fp32
copies (exact for bf16 values).  For bf16 inputs of more than four tokens
the first layer runs on the bf16 matrix core from a packed copy of
conv1.weight (fp32 parameters: the norm weights folded in, as three bf16
planes that carry the fp32 product exactly; bf16 parameters: one plane),
made once per device, weight version and precision.
"""
import torch
import torch.nn as nn

from . import _lib
from .ops import _ptr, _require_cuda, _retired

_INPUT_BITS = {"pre_k": 1, "post_k": 2, "v": 4}


class GatingRMSNorm(nn.Module):
    """Holds the norm weight (src/modeling_layers.py:113-131); the norm itself
    runs inside the gate kernel."""

    def __init__(self, hidden_size, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps


class GatingPredictor(nn.Module):
    def __init__(self, head_dim, num_kv_heads, g_inputs, g_act_fn, g_expand, g_epsilon, g_rms, g_fast_path):
        super().__init__()
        self.g_inputs = list(g_inputs)
        self.g_epsilon = g_epsilon
        self.g_fast_path = g_fast_path
        self.g_rms = g_rms
        self.act = 1 if g_act_fn == "silu" else 0
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads
        self.input_dim = head_dim * len(self.g_inputs)
        self.inner_dim = int(head_dim * g_expand)
        self.pre_key_norm = GatingRMSNorm(head_dim) if g_rms and "pre_k" in self.g_inputs else nn.Identity()
        self.post_key_norm = GatingRMSNorm(head_dim) if g_rms and "post_k" in self.g_inputs else nn.Identity()
        self.value_norm = GatingRMSNorm(head_dim) if g_rms and "v" in self.g_inputs else nn.Identity()
        self.conv1 = nn.Conv1d(num_kv_heads * self.input_dim, num_kv_heads * self.inner_dim, 1, groups=num_kv_heads)
        self.conv2 = nn.Conv1d(num_kv_heads * self.inner_dim, num_kv_heads, 1, groups=num_kv_heads)

    def reset_parameters(self):
        """src/modeling_layers.py:163-168."""
        for norm in (self.pre_key_norm, self.post_key_norm, self.value_norm):
            if isinstance(norm, GatingRMSNorm):
                nn.init.ones_(norm.weight)
        self.conv1.reset_parameters()
        self.conv2.reset_parameters()

    def _f32(self, p):
        """fp32 contiguous copy of a parameter for the kernel.  Copies of
        non-fp32 parameters are cached per parameter storage and refreshed
        when the parameter's version changes (in-place updates, loading), so
        a decode step does not re-convert the weights."""
        if p is None:
            return None
        if p.dtype == torch.float32 and p.is_contiguous():
            return p.detach()
        cache = self.__dict__.setdefault("_f32_cache", {})
        key = (p.data_ptr(), tuple(p.shape))
        hit = cache.get(key)
        if hit is not None and hit[0] == p._version:
            return hit[1]
        c = p.detach().float().contiguous()
        cache[key] = (p._version, c)
        return c

    def _norm_weights(self):
        norms = [self.pre_key_norm, self.post_key_norm, self.value_norm]
        return [self._f32(m.weight) if isinstance(m, GatingRMSNorm) else None for m in norms]

    def precision(self, input_dtype):
        """wgkv_gate_scores' arithmetic for inputs of ``input_dtype``: 0 with
        fp32 parameters (or fp32 inputs), 1 / 2 with bf16 parameters on bf16
        inputs (fast path / Conv1d path)."""
        if input_dtype == torch.bfloat16 and self.conv1.weight.dtype == torch.bfloat16:
            return 1 if self.g_fast_path else 2
        return 0

    def packed_weights(self, precision=0):
        """Packed first-layer weights (wgkv_gate_pack_weights) for the bf16
        matrix-core path, cached per device and precision and remade when
        conv1.weight or a norm weight changes version."""
        params = [self.conv1.weight] + [m.weight for m in (self.pre_key_norm, self.post_key_norm, self.value_norm)
                                        if isinstance(m, GatingRMSNorm)]
        key = (self.conv1.weight.device, precision, tuple((p.data_ptr(), p._version) for p in params))
        hit = self.__dict__.get("_packed_cache")
        if hit is not None and hit[0] == key:
            return hit[1]
        wn = self._norm_weights()
        packed = pack_weights(wn[0], wn[1], wn[2], self._f32(self.conv1.weight), self.g_inputs, self.g_rms,
                              self.num_kv_heads, self.head_dim, self.inner_dim, precision=precision)
        self.__dict__["_packed_cache"] = (key, packed)
        return packed

    def _launch_plan(self, dtype, device, packed_path):
        """The parameter part of wgkv_gate_scores' arguments (fp32 copies,
        packed weights, arithmetic), made once and remade when a parameter
        is replaced or changes version.  The parameters are read through the
        modules' own dictionaries: a chunked prompt calls the gate once per
        chunk and layer, and nn.Module attribute lookups cost more host time
        than the rest of the call."""
        mods = self._modules
        c1, c2 = mods["conv1"]._parameters, mods["conv2"]._parameters
        params = [c1["weight"], c1["bias"], c2["weight"], c2["bias"]]
        for name in ("pre_key_norm", "post_key_norm", "value_norm"):
            m = mods[name]
            if isinstance(m, GatingRMSNorm):
                params.append(m._parameters["weight"])
        key = (dtype, device, packed_path) + tuple((id(q), q._version) for q in params)
        hit = self.__dict__.get("_plan")
        if hit is not None and hit[0] == key:
            return hit[1]
        wn = self._norm_weights()
        prec = self.precision(dtype)
        packed = self.packed_weights(prec) if packed_path else None
        plan = _GateParams(wn[0], wn[1], wn[2], self._f32(self.conv1.weight), self._f32(self.conv1.bias),
                           self._f32(self.conv2.weight), self._f32(self.conv2.bias), self.inner_dim, self.act,
                           self.g_rms, 0.0 if self.g_fast_path else float(self.g_epsilon), packed, prec)
        self.__dict__["_plan"] = (key, plan)
        return plan

    def scores_and_mask(self, pre_key, post_key, value, threshold, scores_out=None, mask_out=None, want_scores=True,
                        active=None):
        """(B, H, S, D) inputs -> (scores f32 (B,H,S) or None, mask bool (B,H,S)).
        ``active`` = (device int32 tensor, value): the kernel runs only if
        the tensor's first element equals value (decided on the device)."""
        B, H, S, D = post_key.shape
        if H != self.num_kv_heads or D != self.head_dim:
            raise AssertionError("gate input shape does not match the predictor")
        dt = post_key.dtype
        plan = self._launch_plan(dt, post_key.device, dt == torch.bfloat16 and S > 4 and post_key.is_cuda)
        ins = self.g_inputs
        return _run_gate(plan, pre_key if "pre_k" in ins else None, post_key if "post_k" in ins else None,
                         value if "v" in ins else None, threshold, post_key, scores_out, mask_out, want_scores,
                         active)

    def forward(self, pre_key, post_key, value):
        """Scores (B, H, S) as the reference's forward returns them: float32,
        or bf16 with bf16 parameters on bf16 inputs."""
        scores, _ = self.scores_and_mask(pre_key, post_key, value, threshold=0.0)
        return scores.to(torch.bfloat16) if self.precision(post_key.dtype) else scores


def pack_weights(w_pre, w_post, w_v, w1, g_inputs, rms, num_kv_heads, head_dim, inner, precision=0):
    """wgkv_gate_pack_weights: conv1 weight (H*inner, n_in*D[, 1]) fp32 times
    the norm weights (when rms), as three bf16 planes in the matrix-core
    operand layout (precision 0), or conv1 weight alone as one plane
    (precision 1 / 2: bf16 parameters).  Returns a uint8 device tensor."""
    bits = 0
    for name in g_inputs:
        bits |= _INPUT_BITS[name]
    n_in = bin(bits).count("1")
    for w in (w_pre, w_post, w_v, w1):
        if w is not None and (w.dtype != torch.float32 or not w.is_contiguous()):
            raise TypeError("gate parameters must be contiguous fp32")
    _require_cuda(w1)
    L = _lib.lib()
    nbytes = int(L.wgkv_gate_packed_bytes(num_kv_heads, inner, n_in * head_dim, int(precision)))
    if nbytes <= 0:
        raise ValueError("unsupported gate shape for packing")
    packed = torch.empty(nbytes, dtype=torch.uint8, device=w1.device)
    st = L.wgkv_gate_pack_weights(_ptr(w_pre), _ptr(w_post), _ptr(w_v), bits, int(bool(rms)), _ptr(w1),
                                  num_kv_heads, head_dim, inner, int(precision), _ptr(packed), nbytes,
                                  _lib.stream_handle(w1.device))
    _lib.check(st, "wgkv_gate_pack_weights")
    return packed


class _GateParams:
    """wgkv_gate_scores' parameter arguments, checked once: the fp32 tensors
    are held so the pointers stay valid."""

    def __init__(self, w_pre, w_post, w_v, w1, b1, w2, b2, inner, act, rms, clamp_min, w1_packed, precision):
        for w in (w_pre, w_post, w_v, w1, b1, w2, b2):
            if w is not None and (w.dtype != torch.float32 or not w.is_contiguous()):
                raise TypeError("gate parameters must be contiguous fp32")
        self.keep = (w_pre, w_post, w_v, w1, b1, w2, b2, w1_packed)
        self.ptrs = (_ptr(w_pre), _ptr(w_post), _ptr(w_v), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2))
        self.inner = int(inner)
        self.tail = (int(act), int(bool(rms)), int(precision), float(clamp_min))
        self.packed = _ptr(w1_packed)


def gate_scores_and_mask(pre_key, post_key, value, w_pre, w_post, w_v, w1, b1, w2, b2, inner, act, rms,
                         clamp_min, threshold, like=None, scores_out=None, mask_out=None, want_scores=True,
                         w1_packed=None, active=None, precision=0):
    """The gate kernel on explicit fp32 parameters (GatingPredictor.forward,
    src/modeling_layers.py:170-205, with the admission of :1465): inputs
    (B, H, S, D) bf16 or fp32 (None for inputs not used), RMS-norm weights (D)
    or None, conv1 weight (H*inner, n_in*D, 1) / bias, conv2 weight
    (H, inner, 1) / bias, act 0 = GELU (erf) / 1 = SiLU, clamp_min > 0 for the
    conv path's clamp; w1_packed (optional) = pack_weights() of the same
    weights, used for bf16 inputs of more than four tokens; active (optional)
    = (int32 device tensor, value): the launch computes and writes nothing
    unless the tensor's first element equals value; precision 0 (fp32
    parameters) or 1 / 2 (bf16 parameters given as fp32 copies, bf16 inputs;
    fast / Conv1d path rounding, threshold compared in bf16; w1_packed made
    with the same precision).  Returns (scores f32 (B,H,S) or None, mask bool
    (B,H,S))."""
    plan = _GateParams(w_pre, w_post, w_v, w1, b1, w2, b2, inner, act, rms, clamp_min, w1_packed, precision)
    return _run_gate(plan, pre_key, post_key, value, threshold, like, scores_out, mask_out, want_scores, active)


def _run_gate(plan, pre_key, post_key, value, threshold, like, scores_out, mask_out, want_scores, active):
    ref = like if like is not None else next(t for t in (post_key, pre_key, value) if t is not None)
    B, H, S, D = ref.shape
    dt = ref.dtype
    if dt not in (torch.bfloat16, torch.float32):
        raise TypeError("gate inputs must be bf16 or fp32")
    bits = 0
    args = []
    for bit, t in ((1, pre_key), (2, post_key), (4, value)):
        if t is not None:
            if t.dtype != dt or t.shape != ref.shape or t.stride(3) != 1:
                raise AssertionError("gate inputs must share shape/dtype with a contiguous last dim")
            if not t.is_cuda:
                _require_cuda(t)
            bits |= bit
            st = t.stride()
            args += (t.data_ptr(), st[0], st[1], st[2])
        else:
            args += (None, 0, 0, 0)
    if bits == 0:
        raise AssertionError("the gate needs at least one input")
    dev = ref.device
    scores = None
    if want_scores:
        scores = scores_out if scores_out is not None else torch.empty(B, H, S, dtype=torch.float32, device=dev)
    mask = mask_out if mask_out is not None else torch.empty(B, H, S, dtype=torch.bool, device=dev)
    mk = mask.view(torch.uint8)
    if active is not None and (active[0].dtype != torch.int32 or not active[0].is_cuda):
        raise TypeError("active must be a device int32 tensor")
    ws = _decode_workspace(dev, B, H, plan.inner) if S <= 4 else None
    if scores is not None:
        sst = scores.stride()
        sargs = (scores.data_ptr(), sst[0], sst[1])
    else:
        sargs = (None, 0, 0)
    mst = mk.stride()
    st = _lib.lib().wgkv_gate_scores(
        *args,
        0 if dt == torch.bfloat16 else 1, bits,
        *plan.ptrs,
        B, H, S, D, plan.inner,
        *plan.tail, float(threshold),
        *sargs,
        mk.data_ptr(), mst[0], mst[1],
        plan.packed,
        _ptr(active[0]) if active is not None else None, int(active[1]) if active is not None else 0,
        _ptr(ws), 0 if ws is None else ws.numel(),
        _lib.stream_handle(dev))
    _lib.check(st, "wgkv_gate_scores")
    return scores, mask


_DECODE_WS = {}


def _decode_workspace(device, B, H, inner):
    """Zero-filled workspace of the few-token gate (partial logits and
    per-head counters that each launch leaves at zero), one per device, grown
    when a call needs more; calls on one stream reuse it in turn, and calls
    on different streams that may overlap must not be made (they would share
    the counters)."""
    need = int(_lib.lib().wgkv_gate_workspace_bytes(B, H, inner))
    ws = _DECODE_WS.get(device)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _retired.append(ws)  # a captured graph may still hold its address
        ws = torch.zeros(max(need, 65536), dtype=torch.uint8, device=device)
        _DECODE_WS[device] = ws
    return ws
