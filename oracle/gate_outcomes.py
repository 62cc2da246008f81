"""Which bf16 gate scores a float32 kernel can produce, token by token.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

The reference's gate with bf16 parameters (its inference loads the gate in
bf16, scripts/profiling.py:222-226) rounds every op's result to bf16
(``GatingRMSNorm.forward`` src/modeling_layers.py:123-128, the fast path
:185-196, the Conv1d path :197-205).  ``oracle.gate.gate_scores_bf16``
restates that graph with exactly summed products and reproduces every score
the reference wrote.  A kernel that evaluates the same graph with float32
sums in its own order lands on the same bf16 value at a rounding point
unless the exact value lies within the kernel's float32 error of a bf16
rounding boundary, and there it may land on either neighbour.

``score_range`` follows the graph token by token and carries, at every
rounding point, the set of bf16 values the kernel can produce:

* normalised inputs ``bf16(x * rsqrt(mean(x^2) + 1e-6))``: the exact value
  +- the relative error of the kernel's float32 norm; an element whose
  interval straddles a boundary has two candidates, and the token is
  followed once per combination (at most ``MAX_AMBIGUOUS_INPUTS`` of them;
  a token with more is reported as unbounded);
* first layer: exact sum +- the float32 error bound of the kernel's
  accumulation order (``KernelOrder``); fast path ``bf16(bf16(acc) + b1)``,
  Conv1d path ``bf16(acc + b1)``;
* activation: for every candidate h, the bf16 values a float32 GELU / SiLU
  can round to (``activation_bounds``: the exact value +- a float32
  evaluation's error, and torch's value, which the reference computes; the
  GPU tests check that every entry of the kernel's own table lies in these
  bounds);
* second layer: the interval of ``sum_j w2_j a_j`` over the candidates,
  widened by the float32 error bound of the kernel's reduction tree;
* sigmoid: ``bf16(1 / (1 + exp(-y)))`` +- the relative error of a float32
  evaluation; Conv1d path: ``max(g, bf16(g_epsilon))``.

Scores are monotone in the second layer's output, so each token's set is a
contiguous range of bf16 values ``[lo, hi]``.  A token is *determined* when
``lo == hi``; the kernel's score must then equal it, and where it also
equals the oracle's score the kernel must reproduce the reference's bit for
bit.  Every other token is *flagged*: its score may legitimately differ, but
only within ``[lo, hi]``.

The float32 error bounds are first-order rigorous for the stated order: a
rounded addition or fused multiply-add errs by at most u = 2**-24 times its
result, so a chain of accumulations into c_1, ..., c_n errs by at most
u * sum |c_s|, and a tree in which every term passes through at most d
roundings errs by at most u * d * sum |terms|.  Each bound is multiplied by
``SAFETY`` (1.01) to cover second-order terms (relative size about n * u)
and the rounding of the bound itself.  A matrix-core step (``v_mfma_*``) is charged as if it summed its
products sequentially in float32 (``l1_internal`` roundings per product),
which covers any internal order.
"""
import math
from dataclasses import dataclass

import torch

U = 2.0 ** -24          # unit roundoff of float32 (round to nearest)
SAFETY = 1.01
EPS32 = float(torch.tensor(1e-6, dtype=torch.float32))  # 1e-6 as the float32 the norm adds
MAX_AMBIGUOUS_INPUTS = 8


@dataclass(frozen=True)
class KernelOrder:
    """Float32 summation structure of one gate kernel (bf16 parameters).

    perm        -- order of the first layer's input index k: the products
                   of k = perm[s*block : (s+1)*block] are added to the
                   accumulator in step s (None: ascending k);
    block       -- products per accumulation step;
    l1_internal -- roundings a product can pass through inside one step;
    l1_chain    -- True if the steps accumulate sequentially into one float32
                   accumulator (charged u * sum |c_s|); False if the whole
                   sum is one tree (charged through l1_internal only);
    l2_depth    -- roundings a second-layer term w2_j * a_j passes through;
    norm_depth  -- roundings of the norm's sum of squares.
    """
    name: str
    perm: tuple
    block: int
    l1_internal: int
    l1_chain: bool
    l2_depth: int
    norm_depth: int


def kernel_order(path, head_dim, n_in, inner):
    """The summation structure of the kernel the library runs for ``path``:

    * ``"packed"`` -- ``gate_bf16_kernel`` (wg-kv_amd/csrc/gate.hip): K/32
      steps of ``v_mfma_f32_16x16x32_bf16`` over k = 32s .. 32s+31 into one
      accumulator; second layer: per lane an fma chain over its
      ``ceil(inner/64)`` columns, a 16-lane butterfly (4 adds), then two levels over the four
      waves; the norm's sum of squares: an 8-term fma chain per lane and a
      butterfly over the D/8 lanes of a row.
    * ``"fp32"`` -- ``gate_kernel``: K/4 steps of ``v_mfma_f32_16x16x4f32``;
      step (k0, e) sums k = k0 + e + 4q, q = 0..3 (lane group q holds four
      consecutive k); second layer as above; norm: two squares per lane and a
      64-lane butterfly (6 adds).
    * ``"small"`` -- ``gate_small_kernel`` (few-token inputs): per lane an fma
      chain over 4*ceil(K/256) products, then a 6-level butterfly over the
      wave; second layer: the product w2*a rounded, a chain over the column
      passes, a 64-lane butterfly, the four waves and the column splits in
      sequence.
    """
    K = n_in * head_dim
    per_wave = -(-(inner // 16) // 4)  # 16-column tiles per wave
    if path == "packed":
        return KernelOrder("packed", None, 32, 32, True, per_wave + 6, 8 + 4)
    if path == "fp32":
        perm = tuple(k0 + e + 4 * q for k0 in range(0, K, 16) for e in range(4) for q in range(4))
        return KernelOrder("fp32", perm, 4, 4, True, per_wave + 6, 2 + 6)
    if path == "small":
        cpl = -(-K // 256)
        nsplit = -(-inner // 64)
        return KernelOrder("small", None, K, 4 * cpl + 6, False, 1 + inner // 64 + 6 + 4 + nsplit, 2 + 6)
    raise ValueError(path)


# ---- bf16 helpers (float64 tensors holding bf16 values) -------------------

def rne_bf16(x):
    """Round float64 to the nearest bf16 value, ties to even, in one step
    (torch's float64 -> bf16 conversion goes through float32 and can round
    twice): on the float64 bit pattern, keep 7 of the 52 fraction bits,
    rounding the 45 dropped bits to nearest, ties to even (a carry moves
    into the exponent as it should).  Finite values in bf16's normal range."""
    b = x.contiguous().view(torch.int64)
    keep = (b >> 45) & 1
    b = (b + ((1 << 44) - 1) + keep) & ~((1 << 45) - 1)
    return b.view(torch.float64)


def ordinal(x):
    """Integer position of a bf16 value on the number line (consecutive bf16
    values have consecutive ordinals; -0 and +0 share 0)."""
    bits = x.to(torch.float32).to(torch.bfloat16).view(torch.int16).to(torch.int32)
    mag = bits & 0x7FFF
    return torch.where(bits < 0, -mag, mag)


def from_ordinal(o):
    """Inverse of ``ordinal`` (ordinal 0 -> +0)."""
    bits = torch.where(o < 0, (-o) | 0x8000, o).to(torch.int32)
    bits = torch.where(bits >= 0x8000, bits - 0x10000, bits).to(torch.int16)
    return bits.view(torch.bfloat16).to(torch.float64)


def add_bf16_f32(r, b):
    """``bf16(float32(r + b))`` for bf16 values r, b: a bf16 tensor plus a
    bf16 tensor in torch (and in the kernels) is a float32 addition rounded
    to bf16."""
    return (r.to(torch.float32) + b.to(torch.float32)).to(torch.bfloat16).to(torch.float64)


def _all_bf16():
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    return bits, bits.view(torch.bfloat16)


def activation_table(g_act_fn="gelu"):
    """bf16(act(h)) for every bf16 bit pattern h (65536 entries, float64,
    indexed by the unsigned pattern), with torch's float32 GELU (erf form)
    or SiLU -- the reference's ``nn.GELU()`` / SiLU in bf16 compute in
    float32 and round once."""
    bits, h = _all_bf16()
    hf = h.to(torch.float32)
    a = torch.nn.functional.silu(hf) if g_act_fn == "silu" else torch.nn.functional.gelu(hf)
    tab = torch.empty(65536, dtype=torch.float64)
    tab[bits.to(torch.int32) & 0xFFFF] = a.to(torch.bfloat16).to(torch.float64)
    return tab


def activation_bounds(g_act_fn="gelu"):
    """Per bf16 h the bf16 values a float32 evaluation of the activation can
    round to: (lo, hi) tables like ``activation_table``.  The exact value
    (float64) +- the error of a float32 evaluation, widened to include
    torch's value:

    * GELU ``0.5 z (1 + erf(z / sqrt 2))``: erf within 2**-21 absolute (a few
      float32 ulps of 1), the scaling, the add and the product rounded --
      below z of about -3 the sum 1 + erf cancels, so the bound is absolute
      and float32 GELUs (torch's, the kernels') disagree there;
    * SiLU ``z / (1 + exp(-z))``: exp within 2 ulps, add and division rounded
      (relative 4u)."""
    bits, h = _all_bf16()
    hd = h.to(torch.float64)
    if g_act_fn == "silu":
        g = hd * torch.sigmoid(hd)
        err = SAFETY * 4 * U * g.abs()
    else:
        t = hd / math.sqrt(2.0)
        s = 1.0 + torch.erf(t)
        g = 0.5 * hd * s
        err = SAFETY * (0.5 * hd.abs() * (2.0 ** -21 + 2 * U * s.abs() + 1.2 * U * t.abs()) + U * g.abs())
    lo = torch.minimum(rne_bf16(g - err), activation_table(g_act_fn)[bits.to(torch.int32) & 0xFFFF])
    hi = torch.maximum(rne_bf16(g + err), activation_table(g_act_fn)[bits.to(torch.int32) & 0xFFFF])
    bad = ~torch.isfinite(hd)
    lo[bad], hi[bad] = math.nan, math.nan
    tlo = torch.empty(65536, dtype=torch.float64)
    thi = torch.empty(65536, dtype=torch.float64)
    idx = bits.to(torch.int32) & 0xFFFF
    tlo[idx], thi[idx] = lo, hi
    return tlo, thi


def _bits(x):
    return x.to(torch.float32).to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF


# ---- the range propagation -----------------------------------------------

def _norm_candidates(x, w, depth):
    """Kernel's bf16(w * bf16(rms(x))) candidates for bf16 input rows x
    (N, D): (lo, hi) float64 (N, D); equal where the value is determined."""
    xd = x.to(torch.float64)
    var = xd.pow(2).mean(-1, keepdim=True)
    y = xd / torch.sqrt(var + EPS32)
    # sum of squares: depth roundings; /D exact; + eps: 1; sqrt: 1; 1/x: 1;
    # x * scale: 1 (relative errors; the sum's halves under the square root)
    rel = SAFETY * U * (depth / 2.0 + 0.5 + 1.0 + 1.0 + 1.0 + 1.0)
    y_lo, y_hi = rne_bf16(y - rel * y.abs()), rne_bf16(y + rel * y.abs())
    if w is None:
        return y_lo, y_hi
    wd = w.to(torch.float64)
    a, b = rne_bf16(wd * y_lo), rne_bf16(wd * y_hi)
    return torch.minimum(a, b), torch.maximum(a, b)


def _layer1_range(X, w1, b1, order, fast_path):
    """Per (row, column) the ordinal range [olo, ohi] of the kernel's bf16
    first-layer output h.  X (N, K) bf16-valued float64, w1 (inner, K),
    b1 (inner,)."""
    N, K = X.shape
    Xp = X if order.perm is None else X[:, list(order.perm)]
    Wp = w1 if order.perm is None else w1[:, list(order.perm)]
    acc = Xp @ Wp.t()
    sabs = Xp.abs() @ Wp.abs().t()
    # each step adds its `block` products to c_{s-1} in some order: its
    # partial sums are bounded by |c_{s-1}| + sum |p|, and it rounds at most
    # `l1_internal` times
    prev = torch.zeros_like(acc)
    if order.l1_chain:
        ns, bs = K // order.block, order.block
        for t0 in range(0, N, 512):  # per-step sums of 512 rows at a time
            xs = Xp[t0:t0 + 512].reshape(-1, ns, bs).transpose(0, 1)   # (ns, n, bs)
            ws = Wp.reshape(-1, ns, bs).permute(1, 2, 0)                # (ns, bs, inner)
            steps = torch.bmm(xs, ws).cumsum(0)                         # c_1 .. c_ns
            prev[t0:t0 + 512] = steps[:-1].abs().sum(0)                 # |c_1| + ... + |c_{ns-1}|
    err = SAFETY * U * order.l1_internal * (sabs + prev) + 2.0 ** -50 * sabs  # + the float64 evaluation
    b1r = b1[None, :].expand_as(acc)
    if fast_path:
        r_lo, r_hi = rne_bf16(acc - err), rne_bf16(acc + err)
        # h = bf16(float32(r + b1)) is monotone in r: its range ends
        h_lo, h_hi = add_bf16_f32(r_lo, b1r), add_bf16_f32(r_hi, b1r)
    else:
        v = acc + b1r
        e2 = err + SAFETY * U * v.abs()  # the float32 bias add
        h_lo, h_hi = rne_bf16(v - e2), rne_bf16(v + e2)
    return ordinal(h_lo), ordinal(h_hi)


class RangeTable:
    """Exact min of ``tab`` and max of ``tab_hi`` (default ``tab``) over any
    ordinal range [olo, ohi] of bf16 arguments, by a sparse table of
    power-of-two blocks (two lookups per query).  GELU's float32 tail (h below about -3) is not monotone, so
    range ends alone would not bound it."""

    def __init__(self, tab, tab_hi=None):
        o = torch.arange(-32767, 32768, dtype=torch.int32)
        v = tab[_bits(from_ordinal(o))]
        vh = v if tab_hi is None else tab_hi[_bits(from_ordinal(o))]
        self.off = 32767
        mn = [torch.nan_to_num(v, nan=math.inf, posinf=math.inf, neginf=-math.inf)]
        mx = [torch.nan_to_num(vh, nan=-math.inf, posinf=math.inf, neginf=-math.inf)]
        k = 1
        while (1 << k) <= v.numel():
            h = 1 << (k - 1)
            a, b = mn[-1], mx[-1]
            mn.append(torch.minimum(a[:-h], a[h:]))
            mx.append(torch.maximum(b[:-h], b[h:]))
            k += 1
        self.mn, self.mx = mn, mx

    def query(self, olo, ohi):
        i, j = olo.long() + self.off, ohi.long() + self.off
        lo, hi = self.mn[0][i], self.mx[0][i]
        wide = torch.nonzero(j > i, as_tuple=True)
        if wide[0].numel():
            wi, wj = i[wide], j[wide]
            k = torch.floor(torch.log2((wj - wi + 1).double())).long()
            wl, wh = torch.empty(wi.shape, dtype=torch.float64), torch.empty(wi.shape, dtype=torch.float64)
            for kk in torch.unique(k).tolist():
                sel = k == kk
                a, b = wi[sel], wj[sel] - (1 << kk) + 1
                wl[sel] = torch.minimum(self.mn[kk][a], self.mn[kk][b])
                wh[sel] = torch.maximum(self.mx[kk][a], self.mx[kk][b])
            lo[wide], hi[wide] = wl, wh
        return lo, hi


def _layer2_terms(olo, ohi, act_rt, w2):
    """Bounds of each term w2_j * bf16(act(h_j)) over the candidate h_j:
    (lo, hi, mag) float64 (N, inner)."""
    a_min, a_max = act_rt.query(olo, ohi)
    t1, t2 = w2[None, :] * a_min, w2[None, :] * a_max
    lo, hi = torch.minimum(t1, t2), torch.maximum(t1, t2)
    return lo, hi, torch.maximum(lo.abs(), hi.abs())


def _score_range_rows(X, w1, b1, w2, b2, act_tab, order, fast_path, clamp):
    """Score range [g_lo, g_hi] (float64 bf16 values) of rows X of one head."""
    olo, ohi = _layer1_range(X, w1, b1, order, fast_path)
    lo, hi, mag = _layer2_terms(olo, ohi, act_tab, w2)
    L, Uu, T = lo.sum(-1), hi.sum(-1), mag.sum(-1)
    e2 = SAFETY * U * order.l2_depth * T + 2.0 ** -50 * T
    b2r = b2.expand_as(L)
    if fast_path:
        y_lo = add_bf16_f32(rne_bf16(L - e2), b2r)
        y_hi = add_bf16_f32(rne_bf16(Uu + e2), b2r)
    else:
        vl, vh = L + b2r, Uu + b2r
        y_lo = rne_bf16(vl - e2 - SAFETY * U * vl.abs())
        y_hi = rne_bf16(vh + e2 + SAFETY * U * vh.abs())
    # 1 / (1 + exp(-y)) in float32: exp within 2 ulps, the add and the
    # division rounded once each
    rel = SAFETY * U * 6.0
    s_lo, s_hi = torch.sigmoid(y_lo), torch.sigmoid(y_hi)
    g_lo, g_hi = rne_bf16(s_lo * (1 - rel)), rne_bf16(s_hi * (1 + rel))
    if clamp is not None:
        c = float(torch.tensor(clamp).to(torch.bfloat16))
        g_lo, g_hi = g_lo.clamp(min=c), g_hi.clamp(min=c)
    return g_lo, g_hi


def score_range(pre_key, post_key, value, params, order, g_inputs=("pre_k", "post_k"), g_act_fn="gelu",
                fast_path=True, g_epsilon=1e-3, select=None, chunk=4096):
    """Per token the range [lo, hi] of bf16 scores the kernel described by
    ``order`` can produce for the reference's bf16 gate (inputs (B,H,S,D)
    bf16, parameters as in ``oracle.gate.gate_scores_bf16``).  ``select``
    (bool (B,H,S), optional) limits the work to those tokens; the others get
    NaN.  Returns (lo, hi, unbounded): float64 (B,H,S) and a bool mask of
    tokens with more than ``MAX_AMBIGUOUS_INPUTS`` ambiguous normalised
    inputs, whose range is reported as [0, 1]."""
    B, H, S, D = post_key.shape
    p16 = {k: v.to(torch.bfloat16).to(torch.float64) for k, v in params.items()}
    names = {"pre_k": (pre_key, "pre_key_norm.weight"), "post_k": (post_key, "post_key_norm.weight"),
             "v": (value, "value_norm.weight")}
    srcs = [names[n] for n in ("pre_k", "post_k", "v") if n in g_inputs]
    n_in = len(srcs)
    inner = p16["conv1.weight"].shape[0] // H
    w1 = p16["conv1.weight"].reshape(H, inner, n_in * D)
    b1 = p16["conv1.bias"].reshape(H, inner)
    w2 = p16["conv2.weight"].reshape(H, inner)
    b2 = p16["conv2.bias"].reshape(H)
    act_tab = RangeTable(*activation_bounds(g_act_fn))
    clamp = None if fast_path else g_epsilon
    lo = torch.full((B, H, S), math.nan, dtype=torch.float64)
    hi = torch.full((B, H, S), math.nan, dtype=torch.float64)
    unb = torch.zeros(B, H, S, dtype=torch.bool)
    for b in range(B):
        for h in range(H):
            pos = torch.arange(S) if select is None else torch.nonzero(select[b, h]).flatten()
            for s0 in range(0, pos.numel(), chunk):
                sl = pos[s0:s0 + chunk]
                cl, ch = [], []
                for t, wname in srcs:
                    c0, c1 = _norm_candidates(t[b, h, sl], p16.get(wname), order.norm_depth)
                    cl.append(c0)
                    ch.append(c1)
                Xlo, Xhi = torch.cat(cl, -1), torch.cat(ch, -1)
                amb = Xlo != Xhi
                namb = amb.sum(-1)
                g_lo, g_hi = _score_range_rows(Xlo, w1[h], b1[h], w2[h], b2[h:h + 1], act_tab, order,
                                               fast_path, clamp)
                # tokens with ambiguous inputs: every combination of the two
                # candidates, the union of the ranges
                rows = torch.nonzero((namb > 0) & (namb <= MAX_AMBIGUOUS_INPUTS)).flatten().tolist()
                variants, owner = [], []
                for r in rows:
                    idx = torch.nonzero(amb[r]).flatten().tolist()
                    for m in range(1, 1 << len(idx)):
                        xv = Xlo[r].clone()
                        for j, i in enumerate(idx):
                            if m >> j & 1:
                                xv[i] = Xhi[r, i]
                        variants.append(xv)
                        owner.append(r)
                if variants:
                    vlo, vhi = _score_range_rows(torch.stack(variants), w1[h], b1[h], w2[h], b2[h:h + 1], act_tab,
                                                 order, fast_path, clamp)
                    own = torch.tensor(owner)
                    g_lo.scatter_reduce_(0, own, vlo, "amin")
                    g_hi.scatter_reduce_(0, own, vhi, "amax")
                big = namb > MAX_AMBIGUOUS_INPUTS
                g_lo[big], g_hi[big] = 0.0, 1.0
                lo[b, h, sl], hi[b, h, sl], unb[b, h, sl] = g_lo, g_hi, big
    return lo, hi, unb


def classify(lo, hi, oracle_scores):
    """Tokens whose kernel score is not pinned to the oracle's: the range
    holds more than one value or its one value is not the oracle's."""
    return (lo != hi) | (lo != oracle_scores)
