"""The C-ABI library loads (no GPU needed) and exports every symbol that
include/wgkv.h declares, with the ctypes binding covering each of them."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wgkv.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wgkv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "wgkv_paged_decode_attn" in syms
    assert len(syms) >= 4


def test_library_exports_every_declared_symbol():
    from wgkv import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libwgkv.so is not built: run __graft_entry__.build()")
    L = _lib.lib()
    for s in declared_symbols():
        assert hasattr(L, s), f"{s} missing from libwgkv.so"
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert L.wgkv_version() >= 1
    assert _lib.status_string(_lib.ERR_CAPACITY) == "cache capacity exceeded"


def test_decode_rejects_bad_arguments_without_gpu():
    # argument checks run on the host before any HIP call
    from wgkv import _lib
    L = _lib.lib()
    st = L.wgkv_paged_decode_attn(None, 0, 0, None, None, 0, 16, None, 0, None, 0, 0, 0,
                                  None, 0, 0, 1, 4, 1, 128, 1.0, None, 0, None)
    assert st == _lib.ERR_ARG


def test_decode_wrapper_requires_device_tensors():
    import torch
    import wgkv
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    kc = torch.zeros(4, 16, 64, dtype=torch.bfloat16)
    sl = torch.ones(1, 1, dtype=torch.int32)
    bt = torch.zeros(1, 1, 4, dtype=torch.int32)
    with pytest.raises(ValueError):
        wgkv.paged_decode_attn(q, kc, kc, sl, bt, 0.125)
    with pytest.raises(TypeError):
        wgkv.paged_decode_attn(q.float(), kc, kc, sl, bt, 0.125)


def test_snapkv_and_gate_argument_checks_without_gpu():
    """Host-side argument checks of the newer entry points (no HIP call is made)."""
    import ctypes
    from wgkv import _lib
    L = _lib.lib()
    assert L.wgkv_snapkv_workspace_bytes(2, 8, 4, 256, 1024) > 0
    assert L.wgkv_snapkv_workspace_bytes(0, 8, 4, 256, 1024) == -1
    p = ctypes.c_void_p(16)  # never dereferenced: the checks fail first

    def evict(**kw):
        args = dict(L=2, H=2, G=2, D=64, P=16, lb=4, maxp=40, total=200, mtph=640, win=16, ksz=5, ratio=0.3)
        args.update(kw)
        return L.wgkv_snapkv_evict(p, p, p, p, p, p, p, args["L"], args["H"], args["G"], args["D"], args["P"],
                                   args["lb"], args["maxp"], args["total"], args["mtph"], args["win"], args["ksz"],
                                   args["ratio"], 0.125, -1, 1, p, None, None, 0, None)

    assert evict() == _lib.ERR_ARG                      # no workspace
    assert evict(ksz=4) == _lib.ERR_ARG                 # even max-pool kernel (the reference asserts odd)
    assert evict(ratio=0.0) == _lib.ERR_ARG             # ratio in (0, 1]
    assert evict(ratio=1.5) == _lib.ERR_ARG
    assert evict(G=9) == _lib.ERR_ARG
    # gate: precision outside 0..2, and bf16 parameters with fp32 inputs
    assert L.wgkv_gate_packed_bytes(8, 512, 256, 3) == -1
    assert L.wgkv_gate_packed_bytes(8, 512, 256, 1) == 8 * 512 * 256 * 2 + 2 * 2 * 20 * 128 * 2

    def gate(in_dtype, precision):
        return L.wgkv_gate_scores(p, 0, 0, 0, p, 0, 0, 0, None, 0, 0, 0, in_dtype, 3, p, p, None, p, p, p, p,
                                  1, 2, 8, 64, 256, 0, 1, precision, 0.0, 0.1, p, 0, 0, None, 0, 0, None,
                                  None, 0, None, 0, None)

    assert gate(0, 5) == _lib.ERR_ARG
    assert gate(1, 1) == _lib.ERR_UNSUPPORTED


def test_random_admission_argument_checks_without_gpu():
    """wgkv_random_admission rejects bad sizes, a sparsity outside [0, 1] and
    missing buffers on the host, before any launch (the pointers here are
    never dereferenced)."""
    from wgkv import _lib
    L = _lib.lib()
    fake = 0x1000

    def call(flags=fake, stride=8, H=2, n=8, p=0.5, counter=fake):
        return L.wgkv_random_admission(flags, stride, H, n, p, 7, counter, None, 0, None)

    assert call(flags=None) == _lib.ERR_ARG
    assert call(counter=None) == _lib.ERR_ARG
    assert call(n=0) == _lib.ERR_ARG
    assert call(H=0) == _lib.ERR_ARG
    assert call(stride=4) == _lib.ERR_ARG      # rows overlap
    assert call(p=-0.1) == _lib.ERR_ARG
    assert call(p=1.5) == _lib.ERR_ARG
    assert call(p=float("nan")) == _lib.ERR_ARG


def test_ring_write_entry_points_argument_checks_without_gpu():
    """wgkv_qkv_rope_ring_write and wgkv_rope_qkv_norm_ring_write reject
    missing ring buffers, a layer outside the model, an empty window and
    (the q/k/v product) more KV heads than one wave writes lengths for, on
    the host before any launch (the fake pointers are never dereferenced)."""
    from wgkv import _lib
    L = _lib.lib()
    f = 0x1000  # 16-byte aligned, never dereferenced

    def gemv(ring=f, pool=f, layer=1, L_=4, W=64, hkv=8):
        return L.wgkv_qkv_rope_ring_write(f, 4096, 4096, f, f, f, 1e-5, f, f, f, 32, hkv, 128,
                                          layer, L_, W, ring, pool, f, f, f, f, None)

    assert gemv(ring=None) == _lib.ERR_ARG
    assert gemv(pool=None) == _lib.ERR_ARG
    assert gemv(layer=4) == _lib.ERR_ARG
    assert gemv(layer=-1) == _lib.ERR_ARG
    assert gemv(W=0) == _lib.ERR_ARG
    assert gemv(hkv=65) == _lib.ERR_UNSUPPORTED

    def rope(ring=f, v=f, layer=1, W=64, pool=f):
        return L.wgkv_rope_qkv_norm_ring_write(f, 128, f, 128, v, 128, f, f, f, 128, f, 128, f, 128, 32, 8, 128,
                                               f, f, 1e-6, f, 128, layer, 4, W, ring, pool, f, f, f, f, None)

    assert rope(ring=None) == _lib.ERR_ARG
    assert rope(v=None) == _lib.ERR_ARG
    assert rope(layer=4) == _lib.ERR_ARG
    assert rope(W=0) == _lib.ERR_ARG
    assert rope(pool=0x1002) == _lib.ERR_UNSUPPORTED  # ring rows are written 16 bytes at a time
