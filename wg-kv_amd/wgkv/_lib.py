"""ctypes binding of the C ABI in include/wgkv.h.

torch is imported first so that the library binds to the HIP runtime torch
already loaded (both carry the SONAME libamdhip64.so.7); a second runtime in
the process would not share device memory or streams with torch.

There is no fallback: if the library is missing, every operation raises.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede loading libwgkv.so)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwgkv.so")

OK = 0
ERR_ARG = 1
ERR_UNSUPPORTED = 2
ERR_CAPACITY = 3
ERR_WORKSPACE = 4
ERR_HIP = 5

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p
c_f32 = ctypes.c_float
c_f64 = ctypes.c_double
c_size = ctypes.c_size_t

# name -> (restype, argtypes); kept in the order of include/wgkv.h
SIGNATURES = {
    "wgkv_version": (ctypes.c_int, []),
    "wgkv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "wgkv_paged_decode_workspace_bytes": (c_size, [c_i32, c_i32, c_i32]),
    "wgkv_paged_decode_attn": (ctypes.c_int, [
        c_ptr, c_i64, c_i64,
        c_ptr, c_ptr, c_i64, c_i32,
        c_ptr, c_i64,
        c_ptr, c_i64, c_i64, c_i32,
        c_ptr, c_i64, c_i64,
        c_i32, c_i32, c_i32, c_i32,
        c_f32,
        c_ptr, c_size,
        c_ptr]),
    "wgkv_paged_decode_attn_noalloc": (ctypes.c_int, [
        c_ptr, c_i64, c_i64,
        c_ptr, c_ptr, c_i64, c_i32,
        c_ptr, c_i64,
        c_ptr, c_i64, c_i64, c_i32,
        c_ptr, c_i64, c_i64,
        c_i32, c_i32, c_i32, c_i32,
        c_f32,
        c_ptr]),
    "wgkv_build_prefill_meta": (ctypes.c_int, [
        c_ptr, c_i64, c_i64,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_ptr, c_ptr,
        c_ptr, c_ptr, c_i32, c_ptr,
        c_ptr]),
    "wgkv_prefill_admit_workspace_bytes": (c_size, [c_i32, c_i32]),
    "wgkv_prefill_admit": (ctypes.c_int, [
        c_ptr, c_ptr, c_i64, c_i64,
        c_ptr, c_i64, c_i64,
        c_ptr, c_i64,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32, c_i64,
        c_ptr, c_ptr, c_ptr, c_i32,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr,
        c_ptr, c_size, c_ptr]),
    "wgkv_decode_append": (ctypes.c_int, [
        c_ptr, c_ptr, c_i64,
        c_ptr, c_i64,
        c_ptr,
        c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32, c_i64,
        c_i32, c_i32, c_i32, c_i32,
        c_ptr, c_ptr, c_ptr, c_i32,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr, c_ptr, c_ptr,
        c_ptr]),
    "wgkv_decode_append_ring": (ctypes.c_int, [
        c_ptr, c_ptr, c_i64,
        c_ptr, c_i64,
        c_ptr,
        c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32, c_i64,
        c_ptr, c_i32, c_i32, c_i32,
        c_ptr, c_ptr, c_ptr, c_i32,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr, c_ptr, c_ptr,
        c_ptr]),
    "wgkv_random_admission": (ctypes.c_int, [
        c_ptr, c_i64, c_i32, c_i32,
        c_f32, ctypes.c_uint64, c_ptr,
        c_ptr, c_i32, c_ptr]),
    "wgkv_gate_scores": (ctypes.c_int, [
        c_ptr, c_i64, c_i64, c_i64,
        c_ptr, c_i64, c_i64, c_i64,
        c_ptr, c_i64, c_i64, c_i64,
        c_i32, c_i32,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr, c_ptr, c_ptr,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32, c_f32, c_f32,
        c_ptr, c_i64, c_i64,
        c_ptr, c_i64, c_i64,
        c_ptr,
        c_ptr, c_i32,
        c_ptr, c_i64,
        c_ptr]),
    "wgkv_gate_workspace_bytes": (ctypes.c_int64, [c_i32, c_i32, c_i32]),
    "wgkv_gate_packed_bytes": (ctypes.c_int64, [c_i32, c_i32, c_i32, c_i32]),
    "wgkv_gate_pack_weights": (ctypes.c_int, [c_ptr, c_ptr, c_ptr, c_i32, c_i32, c_ptr, c_i32, c_i32, c_i32,
                                              c_i32, c_ptr, c_i64, c_ptr]),
    "wgkv_rms_norm": (ctypes.c_int, [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_ptr, c_i64,
                                     c_i32, c_i32, c_f32, c_ptr]),
    "wgkv_rope_qkv": (ctypes.c_int, [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_i64, c_i64,
                                     c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_i64,
                                     c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_i64, c_i64,
                                     c_ptr, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_ptr]),
    "wgkv_rope_qkv_norm": (ctypes.c_int, [c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_i64, c_i64,
                                          c_ptr, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_i64, c_i64,
                                          c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_i64, c_i64,
                                          c_ptr, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32,
                                          c_ptr, c_ptr, c_f32, c_ptr, c_i64, c_i64, c_i64, c_ptr]),
    "wgkv_silu_mul": (ctypes.c_int, [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_i32, c_ptr]),
    "wgkv_gemv": (ctypes.c_int, [c_ptr, c_i64, c_i32, c_i32, c_ptr, c_ptr, c_i32, c_ptr, c_ptr]),
    "wgkv_gemv_ex": (ctypes.c_int, [c_ptr, c_i64, c_i32, c_i32, c_ptr, c_ptr, c_i32, c_ptr,
                                    c_ptr, c_ptr, c_ptr, c_f32, c_ptr, c_ptr, c_ptr, c_i32, c_i32, c_i32, c_ptr]),
    "wgkv_qkv_rope_ring_write": (ctypes.c_int, [c_ptr, c_i64, c_i32, c_ptr, c_ptr, c_ptr, c_f32, c_ptr, c_ptr, c_ptr,
                                                c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_ptr,
                                                c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "wgkv_rope_qkv_norm_ring_write": (ctypes.c_int, [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_ptr,
                                                     c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64,
                                                     c_i32, c_i32, c_i32, c_ptr, c_ptr, c_f32, c_ptr, c_i64,
                                                     c_i32, c_i32, c_i32, c_ptr, c_ptr, c_ptr, c_ptr,
                                                     c_ptr, c_ptr, c_ptr]),
    "wgkv_sparse_prefill_attn": (ctypes.c_int, [
        c_ptr, c_i64, c_i64, c_i64,
        c_ptr, c_ptr, c_i64, c_i64, c_i64,
        c_ptr, c_i64, c_i64, c_i64,
        c_ptr, c_ptr, c_i32,
        c_ptr, c_ptr, c_i64, c_i64,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_i32, c_f32, c_ptr]),
    "wgkv_quest_update_bounds": (ctypes.c_int, [
        c_ptr, c_ptr, c_i32,
        c_ptr, c_ptr,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_i32, c_ptr, c_ptr, c_ptr]),
    "wgkv_quest_select_workspace_bytes": (c_size, [c_i32, c_i32]),
    "wgkv_quest_select": (ctypes.c_int, [
        c_ptr, c_i64,
        c_ptr, c_i32, c_ptr,
        c_ptr, c_ptr,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_ptr, c_i32, c_ptr,
        c_ptr, c_size, c_ptr]),
    "wgkv_snapkv_workspace_bytes": (c_i64, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "wgkv_snapkv_evict": (ctypes.c_int, [
        c_ptr, c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr, c_ptr,
        c_i32, c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_f64, c_f32, c_i64,
        c_i32, c_ptr, c_ptr,
        c_ptr, c_i64, c_ptr]),
    "wgkv_chunk_admit_workspace_bytes": (c_size, [c_i32, c_i32, c_i32]),
    "wgkv_chunk_cache_update": (ctypes.c_int, [
        c_i32,
        c_ptr, c_ptr, c_i64, c_i64,
        c_ptr, c_i64, c_i64,
        c_ptr, c_i64,
        c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32, c_i64,
        c_ptr, c_ptr, c_ptr, c_i32,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_ptr, c_ptr,
        c_ptr, c_size, c_ptr]),
    "wgkv_chunk_prefill_attn": (ctypes.c_int, [
        c_ptr, c_i64, c_i64,
        c_ptr, c_ptr, c_i64, c_i64,
        c_ptr, c_i64, c_i64,
        c_ptr, c_ptr,
        c_ptr, c_i32,
        c_ptr,
        c_i32, c_i32, c_i32,
        c_i32, c_i32, c_i32,
        c_i32, c_i32, c_f32, c_ptr]),
}

_lib = None


class WGKVError(RuntimeError):
    def __init__(self, status, where):
        self.status = status
        super().__init__(f"{where}: {status_string(status)} (status {status})")


class WGKVCapacityError(WGKVError, AssertionError):
    """Raised for cache overflow; an AssertionError like the reference's asserts."""


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library {LIB_PATH} is not built; run __graft_entry__.build() "
                "(python -c 'import __graft_entry__ as g; g.build()') first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def status_string(status):
    return lib().wgkv_status_string(status).decode()


def check(status, where):
    if status == OK:
        return
    if status == ERR_CAPACITY:
        raise WGKVCapacityError(status, where)
    if status in (ERR_UNSUPPORTED,):
        raise WGKVError(status, where)
    raise WGKVError(status, where)


def stream_handle(device=None):
    """hipStream_t of torch's current stream on ``device``."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
