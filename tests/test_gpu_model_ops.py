"""The fused decoder building blocks of the end-to-end harness
(csrc/model_ops.hip) against the torch compositions they replace (the
reference model's LlamaRMSNorm, apply_rotary_pos_emb, SwiGLU): RoPE and the
SwiGLU product bit-identical, the residual add bit-identical, RMSNorm within
one bf16 rounding step (its fp32 mean of squares is summed in another order)."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def torch_rms(x, w, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


@pytest.mark.parametrize("rows,hidden", [(1, 4096), (37, 4096), (5, 512), (3, 8192), (2, 136)])
def test_rms_norm(rows, hidden):
    from wgkv import model_ops
    print(f"[model_ops] rms_norm {rows}x{hidden}", flush=True)
    g = torch.Generator().manual_seed(rows * hidden)
    x = (torch.randn(rows, hidden, generator=g) * 3).to(torch.bfloat16).to(DEV)
    r = torch.randn(rows, hidden, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.rand(hidden, generator=g) + 0.5).to(torch.bfloat16).to(DEV)
    out, none = model_ops.rms_norm(x, w, 1e-5)
    assert none is None
    ref = torch_rms(x, w, 1e-5)
    ulp = (ref.float().abs() * 2 ** -7).clamp_min(1e-30)
    assert ((out.float() - ref.float()).abs() <= ulp * 1.01 + 1e-30).all()
    assert (out == ref).float().mean().item() > 0.99
    out2, h = model_ops.rms_norm(x, w, 1e-5, residual=r)
    assert torch.equal(h, x + r)
    ref2 = torch_rms(x + r, w, 1e-5)
    assert ((out2.float() - ref2.float()).abs() <= (ref2.float().abs() * 2 ** -7) * 1.01 + 1e-30).all()


@pytest.mark.parametrize("B,S,Hq,Hkv,D", [(1, 1, 32, 8, 128), (1, 300, 8, 2, 64), (2, 17, 4, 4, 128)])
def test_rope_bit_identical(B, S, Hq, Hkv, D):
    """q and k rotated bit-identically to apply_rotary_pos_emb; v copied into
    the same buffer (k and v share strides)."""
    from wgkv import model_ops
    from wgkv.attention import LlamaRotaryEmbedding, apply_rotary_pos_emb
    print(f"[model_ops] rope B{B} S{S} Hq{Hq} Hkv{Hkv} D{D}", flush=True)
    g = torch.Generator().manual_seed(S + D)
    qp = torch.randn(B, S, Hq * D, generator=g).to(torch.bfloat16).to(DEV)
    kp = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16).to(DEV)
    q = qp.view(B, S, Hq, D).transpose(1, 2)
    k = kp.view(B, S, Hkv, D).transpose(1, 2)
    rot = LlamaRotaryEmbedding(D, 500000.0).to(DEV)
    pos = torch.arange(1000, 1000 + S, device=DEV)[None].expand(B, S)
    cos, sin = rot(qp, pos)
    rq, rk = apply_rotary_pos_emb(q, k, cos, sin)
    vp = torch.randn(B, S, Hkv * D, generator=g).to(torch.bfloat16).to(DEV)
    v = vp.view(B, S, Hkv, D).transpose(1, 2)
    fq, fk, fv = model_ops.rope_qkv(q, k, v, cos, sin)
    assert torch.equal(fq, rq) and torch.equal(fk, rk) and torch.equal(fv, v)
    assert fk.stride() == fv.stride()


@pytest.mark.parametrize("rows,cols", [(1, 14336), (8, 4096), (3, 96)])
def test_silu_mul_bit_identical(rows, cols):
    """Contiguous inputs and the strided halves of one fused projection."""
    from wgkv import model_ops
    g = torch.Generator().manual_seed(rows * cols)
    a = (torch.randn(rows, cols, generator=g) * 4).to(torch.bfloat16).to(DEV)
    b = torch.randn(rows, cols, generator=g).to(torch.bfloat16).to(DEV)
    assert torch.equal(model_ops.silu_mul(a, b), F.silu(a) * b)
    gu = (torch.randn(rows, 2 * cols, generator=g) * 4).to(torch.bfloat16).to(DEV)
    ga, ua = gu[:, :cols], gu[:, cols:]
    assert torch.equal(model_ops.silu_mul(ga, ua), F.silu(ga) * ua)


@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 14336), (14336, 4096), (37, 72), (3, 8)])
def test_gemv_rows_meet_fp64_products(n, k):
    """wgkv_gemv (mode 0) against the fp64 product: every output is the fp64
    value rounded to bf16, give or take one bf16 unit where the fp32 sum
    lands on the other side of a rounding boundary; repeated calls agree
    bit for bit (no atomics)."""
    from wgkv import model_ops
    print(f"[model_ops] gemv n{n} k{k}", flush=True)
    g = torch.Generator().manual_seed(n + k)
    w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16)
    x = torch.randn(1, 1, k, generator=g).to(torch.bfloat16)
    ref = (x.double().view(1, k) @ w.double().t()).view(-1)
    y = model_ops.linear(x.to(DEV), w.to(DEV)).view(-1).cpu()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    err = ((y.double() - ref).abs() / ulp).max().item()
    assert err <= 1.0, err
    assert torch.equal(model_ops.linear(x.to(DEV), w.to(DEV)).view(-1).cpu(), y)


@pytest.mark.parametrize("n,k", [(14336, 4096), (40, 64)])
def test_gemv_epilogues_equal_the_torch_compositions(n, k):
    """Mode 1 is residual + (W x) and mode 2 silu(W_gate x) * (W_up x) with
    torch's bf16 rounding, bit for bit against the torch ops applied to the
    mode-0 products (each row's sum is computed the same way in every mode);
    rows given as a strided view (weight rows wider than k) and a two-row
    input (torch's GEMM) also work."""
    from wgkv import model_ops
    print(f"[model_ops] gemv epilogues n{n} k{k}", flush=True)
    g = torch.Generator().manual_seed(3 * n + k)
    gu = (torch.randn(2 * n, k, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    x = torch.randn(1, 1, k, generator=g).to(torch.bfloat16).to(DEV)
    r = torch.randn(1, 1, 2 * n, generator=g).to(torch.bfloat16).to(DEV)
    y0 = model_ops.linear(x, gu)
    assert torch.equal(model_ops.linear(x, gu, residual=r), r + y0)
    s = model_ops.swiglu_linear(x, gu)
    assert torch.equal(s, F.silu(y0[..., :n]) * y0[..., n:])
    # a weight whose rows are a strided view (the left k columns of a wider buffer)
    wide = (torch.randn(n, k + 8, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    wv = wide[:, :k]
    assert model_ops.gemv_usable(x, wv)
    assert torch.equal(model_ops.linear(x, wv), model_ops.linear(x, wv.contiguous()))
    # two rows: not a decode step, torch's GEMM
    x2 = torch.randn(1, 2, k, generator=g).to(torch.bfloat16).to(DEV)
    assert not model_ops.gemv_usable(x2, gu)
    assert torch.equal(model_ops.linear(x2, gu), F.linear(x2, gu))


@pytest.mark.parametrize("with_res", [False, True])
@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("H", [4096, 512, 256])
def test_gemv_norm_prologue_equals_rms_norm_then_gemv(with_res, mode, H):
    """The workgroups' own RMSNorm of x (+ residual) gives wgkv_rms_norm's
    bits, so the fused launch equals rms_norm followed by the product (the
    decode step's post-attention norm before the SwiGLU product, and the
    input norm before a q/k/v product without the RoPE epilogue)."""
    from wgkv import model_ops
    print(f"[model_ops] gemv norm prologue H={H} res={with_res} mode={mode}", flush=True)
    g = torch.Generator().manual_seed(5 + mode + int(with_res) + H)
    N = 1024
    x = torch.randn(1, 1, H, generator=g).to(torch.bfloat16).to(DEV)
    r = torch.randn(1, 1, H, generator=g).to(torch.bfloat16).to(DEV) if with_res else None
    nw = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(DEV)
    w = (torch.randn(2 * N if mode == 2 else N, H, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    y, h = model_ops.rms_norm_linear(x, nw, 1e-5, w, residual=r, mode=mode)
    normed, h_ref = model_ops.rms_norm(x, nw, 1e-5, residual=r)
    ref = model_ops.swiglu_linear(normed, w) if mode == 2 else model_ops.linear(normed, w)
    assert torch.equal(y, ref)
    if with_res:
        assert torch.equal(h, h_ref)


@pytest.mark.parametrize("with_norm", [False, True])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (8, 2, 64)])
def test_qkv_rope_equals_product_then_rope(with_norm, Hq, Hkv, D):
    """Mode 3: the q/k/v rows with RoPE applied in the epilogue equal the
    product followed by wgkv_rope_qkv (itself bit-identical to
    apply_rotary_pos_emb), and k_raw is the unrotated k."""
    from wgkv import model_ops
    from wgkv.attention import LlamaRotaryEmbedding
    print(f"[model_ops] qkv_rope Hq{Hq} Hkv{Hkv} D{D} norm={with_norm}", flush=True)
    g = torch.Generator().manual_seed(Hq + D + int(with_norm))
    hidden = 4096 if D == 128 else 512
    n = (Hq + 2 * Hkv) * D
    x = torch.randn(1, 1, hidden, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, hidden, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(DEV) if with_norm else None
    rot = LlamaRotaryEmbedding(D, 500000.0, device=DEV)
    cos, sin = rot(x, torch.tensor([[123457]], device=DEV))
    buf, kraw = model_ops.qkv_rope(x, w, cos, sin, Hq, Hkv, D, nw, 1e-5)
    xin = model_ops.rms_norm(x, nw, 1e-5)[0] if with_norm else x
    qkv = model_ops.linear(xin, w)
    q = qkv[..., :Hq * D].view(1, 1, Hq, D).transpose(1, 2)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(1, 1, Hkv, D).transpose(1, 2)
    v = qkv[..., (Hq + Hkv) * D:].view(1, 1, Hkv, D).transpose(1, 2)
    fq, fk, fv = model_ops.rope_qkv(q, k, v, cos, sin)
    assert torch.equal(buf[:, :, :Hq].transpose(1, 2), fq)
    assert torch.equal(buf[:, :, Hq:Hq + Hkv].transpose(1, 2), fk)
    assert torch.equal(buf[:, :, Hq + Hkv:].transpose(1, 2), fv)
    assert torch.equal(kraw.transpose(1, 2), k)


@pytest.mark.parametrize("ring_full", [False, True])
@pytest.mark.parametrize("Hq,Hkv,D,layer", [(32, 8, 128, 5), (8, 2, 64, 1)])
def test_qkv_ring_write_equals_projection_then_append(ring_full, Hq, Hkv, D, layer):
    """wgkv_qkv_rope_ring_write gives wgkv_gemv_ex mode 3's q/k/v and
    unrotated k, and writes the ring row, pre-RoPE key, attention lengths and
    slot that wgkv_decode_append_ring without a mask, promotion or advance
    writes from them -- bit for bit, every other byte of the pools left as
    it was, the ring pointers unchanged.  Ring not yet full (slot = length)
    and full (slot = the oldest)."""
    from types import SimpleNamespace
    from wgkv import model_ops, ops
    from wgkv.attention import LlamaRotaryEmbedding
    print(f"[model_ops] qkv ring write Hq{Hq} Hkv{Hkv} D{D} layer {layer} full={ring_full}", flush=True)
    g = torch.Generator().manual_seed(31 + D + int(ring_full))
    L, W, page = layer + 2, 64, 16
    hidden = 4096 if D == 128 else 512
    n = (Hq + 2 * Hkv) * D
    x = torch.randn(1, 1, hidden, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, hidden, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(DEV)
    rot = LlamaRotaryEmbedding(D, 500000.0, device=DEV)
    cos, sin = rot(x, torch.tensor([[4321]], device=DEV))
    total_pages = L * Hkv * W // page + 16
    i32 = dict(dtype=torch.int32, device=DEV)

    def cache():
        g2 = torch.Generator().manual_seed(7)
        return SimpleNamespace(
            num_layers=L, num_kv_heads=Hkv, head_dim=D, local_window_size=W, block_size=page,
            max_tokens_per_head=10 ** 6, total_blocks=total_pages, device_ring=True,
            block_pool_k=torch.randn(total_pages * page, D, generator=g2).to(torch.bfloat16).to(DEV),
            block_pool_v=torch.randn(total_pages * page, D, generator=g2).to(torch.bfloat16).to(DEV),
            local_pre_key=torch.randn(L, Hkv, W, D, generator=g2).to(torch.bfloat16).to(DEV),
            global_lengths=torch.randint(0, 5000, (L * Hkv,), generator=g2).to(**i32),
            block_table=torch.zeros(L, Hkv, 4, **i32),
            local_is_global=torch.zeros(L, Hkv, W, dtype=torch.bool, device=DEV),
            next_free_block_dev=torch.zeros(1, **i32), status=torch.zeros(1, **i32),
            ring_state=torch.tensor([37, W, -1] if ring_full else [0, 21, -1], **i32),
            seqlens=torch.full((Hkv,), -5, **i32))

    a, b = cache(), cache()
    buf_a, kraw_a = model_ops.qkv_rope(x, w, cos, sin, Hq, Hkv, D, nw, 1e-5, ring=(a, layer, a.seqlens))
    buf_b, kraw_b = model_ops.qkv_rope(x, w, cos, sin, Hq, Hkv, D, nw, 1e-5)
    ops.decode_append(b, layer, buf_b[0, 0, Hq:Hq + Hkv], buf_b[0, 0, Hq + Hkv:], g_mask=None,
                      pre_key=kraw_b[0, 0], migrate=False, write=True, cache_seqlens=b.seqlens, advance=False)
    torch.cuda.synchronize()
    assert torch.equal(buf_a, buf_b) and torch.equal(kraw_a, kraw_b)
    for name in ("block_pool_k", "block_pool_v", "local_pre_key", "seqlens", "ring_state", "status",
                 "local_is_global", "global_lengths", "block_table"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    slot = 37 if ring_full else 21
    assert a.ring_state.tolist() == ([37, W, slot] if ring_full else [0, 21, slot])
    cur = W if ring_full else 22
    assert a.seqlens.tolist() == (cur + a.global_lengths[layer * Hkv:(layer + 1) * Hkv]).tolist()
    rows = (layer * Hkv + torch.arange(Hkv, device=DEV)) * W + slot
    assert torch.equal(a.block_pool_k[rows], buf_a[0, 0, Hq:Hq + Hkv])
    assert torch.equal(a.local_pre_key[layer, :, slot], kraw_a[0, 0])


@pytest.mark.parametrize("ring_full", [False, True])
@pytest.mark.parametrize("norm", [True, False])
def test_rope_ring_write_equals_rope_then_append(ring_full, norm):
    """wgkv_rope_qkv_norm_ring_write gives wgkv_rope_qkv_norm's outputs for
    one decode row and writes the ring row, pre-RoPE key (normalised with
    the k head norm), attention lengths and slot that
    wgkv_decode_append_ring without a mask, promotion or advance writes from
    them, bit for bit, every other byte of the pools left as it was."""
    from types import SimpleNamespace
    from wgkv import model_ops, ops
    from wgkv.attention import LlamaRotaryEmbedding
    print(f"[model_ops] rope ring write norm={norm} full={ring_full}", flush=True)
    g = torch.Generator().manual_seed(41 + int(norm) + 2 * int(ring_full))
    Hq, Hkv, D, layer, L, W, page = 32, 8, 128, 2, 4, 64, 16
    qkv = torch.randn(1, 1, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16).to(DEV)
    q = qkv[..., :Hq * D].view(1, 1, Hq, D).transpose(1, 2)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(1, 1, Hkv, D).transpose(1, 2)
    v = qkv[..., (Hq + Hkv) * D:].view(1, 1, Hkv, D).transpose(1, 2)
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV) if norm else None
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV) if norm else None
    rot = LlamaRotaryEmbedding(D, 1e6, device=DEV)
    cos, sin = rot(qkv, torch.tensor([[98765]], device=DEV))
    total_pages = L * Hkv * W // page + 16
    i32 = dict(dtype=torch.int32, device=DEV)

    def cache():
        g2 = torch.Generator().manual_seed(9)
        return SimpleNamespace(
            num_layers=L, num_kv_heads=Hkv, head_dim=D, local_window_size=W, block_size=page,
            max_tokens_per_head=10 ** 6, total_blocks=total_pages, device_ring=True,
            block_pool_k=torch.randn(total_pages * page, D, generator=g2).to(torch.bfloat16).to(DEV),
            block_pool_v=torch.randn(total_pages * page, D, generator=g2).to(torch.bfloat16).to(DEV),
            local_pre_key=torch.randn(L, Hkv, W, D, generator=g2).to(torch.bfloat16).to(DEV),
            global_lengths=torch.randint(0, 5000, (L * Hkv,), generator=g2).to(**i32),
            block_table=torch.zeros(L, Hkv, 4, **i32),
            local_is_global=torch.zeros(L, Hkv, W, dtype=torch.bool, device=DEV),
            next_free_block_dev=torch.zeros(1, **i32), status=torch.zeros(1, **i32),
            ring_state=torch.tensor([13, W, -1] if ring_full else [0, 40, -1], **i32),
            seqlens=torch.full((Hkv,), -5, **i32))

    a, b = cache(), cache()
    ra = model_ops.rope_qkv(q, k, v, cos, sin, qn, kn, 1e-6, ring=(a, layer, a.seqlens))
    rb_ = model_ops.rope_qkv(q, k, v, cos, sin, qn, kn, 1e-6)
    pre = rb_[3] if norm else k
    ops.decode_append(b, layer, rb_[1][0, :, 0], rb_[2][0, :, 0], g_mask=None, pre_key=pre[0, :, 0],
                      migrate=False, write=True, cache_seqlens=b.seqlens, advance=False)
    torch.cuda.synchronize()
    for x, y in zip(ra, rb_):
        assert torch.equal(x, y)
    for name in ("block_pool_k", "block_pool_v", "local_pre_key", "seqlens", "ring_state", "status",
                 "local_is_global", "global_lengths", "block_table"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    slot = 13 if ring_full else 40
    assert a.ring_state.tolist()[2] == slot


@pytest.mark.parametrize("S,D", [(1, 128), (300, 128), (77, 64)])
def test_rope_with_qwen3_head_norms_matches_torch(S, D):
    """Qwen3's per-head q_norm / k_norm fused into the RoPE launch against
    HeadRMSNorm followed by wgkv_rope_qkv (itself bit-identical to
    apply_rotary_pos_emb): the only difference allowed is the order of the
    per-head sum of squares, which can move an element by one bf16 unit; the
    normalised, unrotated k equals k_norm(k) to the same bound."""
    from wgkv import model_ops
    from wgkv.attention import HeadRMSNorm, LlamaRotaryEmbedding
    print(f"[model_ops] rope + head norms S{S} D{D}", flush=True)
    g = torch.Generator().manual_seed(S + D)
    B, Hq, Hkv = 1, 8, 2
    qkv = torch.randn(B, S, Hq + 2 * Hkv, D, generator=g).to(torch.bfloat16).to(DEV) * 3
    q, k, v = (qkv[:, :, :Hq].transpose(1, 2), qkv[:, :, Hq:Hq + Hkv].transpose(1, 2),
               qkv[:, :, Hq + Hkv:].transpose(1, 2))
    qn, kn = HeadRMSNorm(D).to(DEV).to(torch.bfloat16), HeadRMSNorm(D).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        qn.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
        kn.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
    rot = LlamaRotaryEmbedding(D, 1e6, device=DEV)
    cos, sin = rot(qkv, torch.arange(1000, 1000 + S, device=DEV)[None])
    fq, fk, fv, fkp = model_ops.rope_qkv(q, k, v, cos, sin, qn.weight, kn.weight, qn.eps)
    with torch.no_grad():
        q2, k2 = qn(q), kn(k)
    rq, rk, rv = model_ops.rope_qkv(q2, k2, v, cos, sin)

    def ulps(a, b):
        a, b = a.float(), b.float()
        ulp = torch.exp2(torch.floor(torch.log2(b.abs().clamp_min(1e-30))) - 7)
        return ((a - b).abs() / ulp)

    for name, x, y in (("q", fq, rq), ("k", fk, rk), ("k_pre", fkp, k2)):
        u = ulps(x, y)
        frac = (u > 0).float().mean().item()
        print(f"   {name}: max {u.max().item():.1f} ulp, {frac:.4%} elements differ", flush=True)
        assert u.max().item() <= 2.0 and frac <= 0.002, name
    assert torch.equal(fv, rv)
