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
