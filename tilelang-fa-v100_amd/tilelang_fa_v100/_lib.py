"""ctypes binding of libfa355.so (C ABI declared in include/fa355.h).

The structures below mirror the C structs field for field.  The library is
loaded after torch, so its HIP runtime dependency (soname libamdhip64.so.7)
resolves to the runtime torch already loaded and torch's stream handles are
valid inside the library.

There is no fallback: if the shared library is missing every entry point
raises, on CPU and GPU alike.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

LIB_NAME = "libfa355.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 3

FA_OK = 0
FA_E_INVALID = -1
FA_E_UNSUPPORTED = -2
FA_E_HIP = -3
FA_E_WORKSPACE = -4

FA_DTYPE_F16 = 0
FA_DTYPE_BF16 = 1

_i64x3 = ctypes.c_int64 * 3
_i64x2 = ctypes.c_int64 * 2
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp), ("lse", _vp),
        ("q_stride", _i64x3), ("k_stride", _i64x3), ("v_stride", _i64x3),
        ("o_stride", _i64x3),
        ("batch", _i32), ("seqlen_q", _i32), ("seqlen_k", _i32),
        ("num_heads", _i32), ("num_heads_k", _i32), ("head_dim", _i32),
        ("softmax_scale", _f32), ("causal", _i32), ("dtype", _i32),
        ("has_window", _i32), ("window_left", _i32), ("window_right", _i32),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("out", _vp), ("dout", _vp),
        ("lse", _vp), ("dq", _vp), ("dk", _vp), ("dv", _vp),
        ("q_stride", _i64x3), ("k_stride", _i64x3), ("v_stride", _i64x3),
        ("o_stride", _i64x3), ("do_stride", _i64x3), ("dq_stride", _i64x3),
        ("dk_stride", _i64x3), ("dv_stride", _i64x3),
        ("batch", _i32), ("seqlen_q", _i32), ("seqlen_k", _i32),
        ("num_heads", _i32), ("num_heads_k", _i32), ("head_dim", _i32),
        ("softmax_scale", _f32), ("causal", _i32), ("dtype", _i32),
        ("deterministic", _i32), ("has_window", _i32), ("window_left", _i32),
        ("window_right", _i32),
    ]


class PagedArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k_cache", _vp), ("v_cache", _vp), ("out", _vp), ("lse", _vp),
        ("block_table", _vp), ("seq_lens", _vp), ("query_start_loc", _vp),
        ("prefix_kv_lens", _vp),
        ("q_stride", _i64x2), ("o_stride", _i64x2),
        ("k_stride", _i64x3), ("v_stride", _i64x3),
        ("block_table_stride", ctypes.c_int64),
        ("max_blocks", _i32), ("num_tokens", _i32), ("batch", _i32),
        ("num_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("page_size", _i32), ("num_pages", _i32),
        ("softmax_scale", _f32), ("causal", _i32),
        ("window_q", _i32), ("window_k", _i32), ("dtype", _i32),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k_cache", _vp), ("v_cache", _vp), ("out", _vp), ("lse", _vp),
        ("block_table", _vp), ("seq_lens", _vp),
        ("q_stride", _i64x2), ("o_stride", _i64x2),
        ("k_stride", _i64x3), ("v_stride", _i64x3),
        ("block_table_stride", ctypes.c_int64),
        ("max_blocks", _i32), ("max_seq_len", _i32), ("batch", _i32),
        ("num_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("page_size", _i32), ("num_pages", _i32),
        ("softmax_scale", _f32), ("dtype", _i32),
    ]


class CacheWriteArgs(ctypes.Structure):
    _fields_ = [
        ("key", _vp), ("value", _vp), ("k_cache", _vp), ("v_cache", _vp),
        ("slot_mapping", _vp),
        ("key_stride", _i64x2), ("value_stride", _i64x2),
        ("k_stride", _i64x3), ("v_stride", _i64x3),
        ("num_tokens", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
        ("page_size", _i32), ("num_pages", _i32), ("dtype", _i32),
    ]


# Every function the header declares, with its ctypes prototype.
_PROTOTYPES = {
    "fa_abi_version": (ctypes.c_int, []),
    "fa_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "fa_last_error_message": (ctypes.c_char_p, []),
    "fa_fwd": (ctypes.c_int, [ctypes.POINTER(FwdArgs), _vp]),
    "fa_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(BwdArgs)]),
    "fa_bwd_min_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(BwdArgs)]),
    "fa_bwd": (ctypes.c_int, [ctypes.POINTER(BwdArgs), _vp, ctypes.c_size_t, _vp]),
    "fa_paged_prefill": (ctypes.c_int, [ctypes.POINTER(PagedArgs), _vp]),
    "fa_paged_prefill_num_splits": (ctypes.c_int, [ctypes.POINTER(PagedArgs)]),
    "fa_paged_prefill_splitkv_workspace_bytes": (ctypes.c_size_t,
                                                 [ctypes.POINTER(PagedArgs), ctypes.c_int]),
    "fa_paged_prefill_splitkv": (ctypes.c_int, [ctypes.POINTER(PagedArgs), ctypes.c_int, _vp,
                                                ctypes.c_size_t, _vp]),
    "fa_decode_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(DecodeArgs)]),
    "fa_paged_decode": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _vp, ctypes.c_size_t, _vp]),
    "fa_paged_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _vp]),
    "fa_reshape_and_cache": (ctypes.c_int, [ctypes.POINTER(CacheWriteArgs), _vp]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Loads the library once; raises RuntimeError if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_NAME} is not built ({LIB_PATH}); run "
                    "`python tilelang-fa-v100_amd/build.py` (or __graft_entry__.build())")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _PROTOTYPES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            ver = lib.fa_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"{LIB_NAME} ABI version {ver}, expected {ABI_VERSION}")
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Turns a non-zero fa_status into a Python exception."""
    if status == FA_OK:
        return
    lib = load()
    msg = lib.fa_last_error_message().decode(errors="replace")
    text = f"{what}: {lib.fa_strerror(status).decode()}: {msg}"
    if status in (FA_E_INVALID, FA_E_UNSUPPORTED):
        raise ValueError(text)
    raise RuntimeError(text)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return FA_DTYPE_F16
    if dtype == torch.bfloat16:
        return FA_DTYPE_BF16
    raise TypeError(f"unsupported dtype {dtype}; expected torch.float16 or torch.bfloat16")


def stream_handle(device: torch.device) -> int:
    """hipStream_t of `device`'s current stream, as an integer."""
    return torch.cuda.current_stream(device).cuda_stream


def call_on(device: torch.device, fn):
    """Runs fn(stream) with `device` current and its current stream.

    The library launches on the stream it is given and reads the current
    device (CU count); when `device` is already current the device guard
    (a few microseconds per call) is skipped.
    """
    if device.index == torch.cuda.current_device():
        return fn(torch.cuda.current_stream().cuda_stream)
    with torch.cuda.device(device):
        return fn(torch.cuda.current_stream(device).cuda_stream)
