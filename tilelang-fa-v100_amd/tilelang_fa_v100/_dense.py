"""Host drivers of the dense forward / backward kernels.

Replace the host side of tilelang_forward_lse (tilelang_fa_v100/
_kernels_forward.py:188-193, called from interface.py:35-36) and of
tilelang_backward (_kernels_backward.py:200-208).  Tensors stay in the FA2
layout [B, S, H, D]; the kernels address them through strides, so the
reference's permute/contiguous copies (interface.py:19-21,38,51) are gone.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib
from ._checks import HEAD_DIMS, rows_ready, strides


def check_shapes(q, k, v):
    """Validates [B, S, H, D] shapes; returns (B, Sq, Sk, H, Hk, D)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4-D [batch, seqlen, heads, head_dim]")
    B, Sq, H, D = q.shape
    if k.shape != v.shape:
        raise ValueError(f"k shape {tuple(k.shape)} differs from v shape {tuple(v.shape)}")
    if k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"k shape {tuple(k.shape)} incompatible with q shape {tuple(q.shape)}")
    Hk = k.shape[2]
    if Hk == 0 or H % Hk != 0:
        raise ValueError(f"num_heads {H} is not a multiple of num_heads_k {Hk}")
    if D not in HEAD_DIMS:
        raise ValueError(f"head_dim {D} not supported (expected one of {HEAD_DIMS})")
    return B, Sq, k.shape[1], H, Hk, D


def window_bounds(window_size) -> tuple:
    """(left, right) of a FlashAttention-2 window_size; -1 = unbounded."""
    if window_size is None:
        return -1, -1
    try:
        left, right = (int(x) for x in window_size)
    except (TypeError, ValueError):
        raise ValueError(f"window_size must be a pair of ints, got {window_size!r}") from None
    if left < -1 or right < -1:
        raise ValueError(f"window_size entries must be >= -1, got {window_size!r}")
    return left, right


def forward(q, k, v, softmax_scale: float, causal: bool, window=(-1, -1), shapes=None,
            with_lse: bool = True):
    """Returns (out [B,Sq,H,D], lse [B,H,Sq] fp32).  shapes: check_shapes' result
    when the caller has already validated q, k, v.  with_lse=False passes no LSE
    buffer (the kernel skips its store) and returns (out, None): the reference's
    LSE-less tilelang_forward (_kernels_forward.py:9-91,180-185)."""
    B, Sq, Sk, H, Hk, D = shapes if shapes is not None else check_shapes(q, k, v)
    q, k, v = rows_ready(q), rows_ready(k), rows_ready(v)
    # K / V sequence strides must stay below 2^24 elements (fa_fwd).
    k = k.contiguous() if k.stride(1) >= 1 << 24 else k
    v = v.contiguous() if v.stride(1) >= 1 << 24 else v
    out = torch.empty((B, Sq, H, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device) if with_lse else None
    a = _lib.FwdArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.lse = lse.data_ptr() if with_lse else None
    a.q_stride[:] = strides(q, 3)
    a.k_stride[:] = strides(k, 3)
    a.v_stride[:] = strides(v, 3)
    a.o_stride[:] = strides(out, 3)
    a.batch, a.seqlen_q, a.seqlen_k = B, Sq, Sk
    a.num_heads, a.num_heads_k, a.head_dim = H, Hk, D
    a.softmax_scale = float(softmax_scale)
    a.causal = int(bool(causal))
    a.dtype = _lib.dtype_code(q.dtype)
    a.has_window = int(tuple(window) != (-1, -1))
    a.window_left, a.window_right = window
    lib = _lib.load()
    _lib.check(_lib.call_on(q.device, lambda st: lib.fa_fwd(ctypes.byref(a), st)), "fa_fwd")
    return out, lse


def bwd_args(q, k, v, out, dout, lse, dq, dk, dv, softmax_scale, causal, deterministic,
             window=(-1, -1)):
    B, Sq, Sk, H, Hk, D = check_shapes(q, k, v)
    a = _lib.BwdArgs()
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.out, a.dout, a.lse = out.data_ptr(), dout.data_ptr(), lse.data_ptr()
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    for name, t in (("q", q), ("k", k), ("v", v), ("o", out), ("do", dout),
                    ("dq", dq), ("dk", dk), ("dv", dv)):
        getattr(a, f"{name}_stride")[:] = strides(t, 3)
    a.batch, a.seqlen_q, a.seqlen_k = B, Sq, Sk
    a.num_heads, a.num_heads_k, a.head_dim = H, Hk, D
    a.softmax_scale = float(softmax_scale)
    a.causal = int(bool(causal))
    a.dtype = _lib.dtype_code(q.dtype)
    a.deterministic = int(bool(deterministic))
    a.has_window = int(tuple(window) != (-1, -1))
    a.window_left, a.window_right = window
    return a


# ---- backward workspace policy
#
# fa_bwd runs one of two paths, chosen by the workspace it is given:
#  * fa_bwd_min_workspace_bytes: the row statistics only (8 bytes per query
#    row and head); dQ recomputes S and dP, like the reference's dQ kernel.
#    This is the memory footprint of the reference's tilelang_backward
#    (_kernels_backward.py:200-208: row_dot plus its fp32 up-casts).
#  * fa_bwd_workspace_bytes: at head_dim 128 / 256 with causal or full
#    attention, the statistics plus the dS tiles (2 bytes per visible
#    (query, key) pair: 268 MB at [4, 2048, 16, 128], 2.15 GB at
#    [2, 8192, 16, 128]); dQ then costs one product per tile pair instead of
#    three.
# The dS path is taken while its workspace fits the limit below, and the
# recompute path whenever it does not or its allocation fails, so the
# backward never needs more memory than the reference's.

WORKSPACE_LIMIT_ENV = "TILELANG_FA_BWD_WORKSPACE_LIMIT"
# Default limit: this share of the memory the device can still hand out
# (free device memory plus blocks torch holds cached but unused), or all of
# the cached blocks when they alone hold the dS workspace.
FREE_MEMORY_SHARE = 0.5
_workspace_limit = None


def set_backward_workspace_limit(nbytes):
    """Caps the dense backward's workspace at `nbytes` bytes (0: always the
    recompute path); None restores the default.  The environment variable
    TILELANG_FA_BWD_WORKSPACE_LIMIT (bytes) sets it too; this call wins."""
    global _workspace_limit
    if nbytes is not None:
        nbytes = int(nbytes)
        if nbytes < 0:
            raise ValueError(f"workspace limit must be >= 0, got {nbytes}")
    _workspace_limit = nbytes


def workspace_limit(device, want=None) -> int:
    """Bytes the backward's workspace may take on `device` right now.

    want: the dS workspace's size.  When torch already holds at least that
    much cached but unused (the steady state of a training loop, which frees
    the workspace after every backward), the workspace comes from those
    blocks and the device is not queried: torch.cuda.mem_get_info took ~5 us
    on an idle MI355X and a median of ~90 us behind a busy stream."""
    if _workspace_limit is not None:
        return _workspace_limit
    env = os.environ.get(WORKSPACE_LIMIT_ENV)
    if env:
        try:
            return max(int(env), 0)
        except ValueError:
            raise ValueError(f"{WORKSPACE_LIMIT_ENV} must be a byte count, got {env!r}") from None
    cached = max(torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device), 0)
    if want is not None and want <= cached:
        return cached
    free, _ = torch.cuda.mem_get_info(device)
    return int((free + cached) * FREE_MEMORY_SHARE)


def choose_workspace(full: int, minimal: int, limit: int) -> int:
    """Workspace bytes to ask for: `full` (dS path) when it is larger than
    `minimal` and fits `limit`, else `minimal` (recompute path)."""
    return full if minimal < full <= limit else minimal


def _empty_bytes(n: int, device):
    return torch.empty(n, dtype=torch.uint8, device=device)


def alloc_workspace(full: int, minimal: int, device):
    """The backward's workspace tensor: the dS path's when the limit allows
    it, falling back to the recompute path's when that allocation raises
    torch.cuda.OutOfMemoryError."""
    if full <= minimal:
        return _empty_bytes(minimal, device)
    n = choose_workspace(full, minimal, workspace_limit(device, full))
    if n == minimal:
        return _empty_bytes(minimal, device)
    try:
        return _empty_bytes(n, device)
    except torch.cuda.OutOfMemoryError:
        return _empty_bytes(minimal, device)


def backward(q, k, v, out, dout, lse, softmax_scale: float, causal: bool,
             deterministic: bool = False, window=(-1, -1)):
    """Returns (dq, dk, dv), each contiguous [B, S, H, D] in q's dtype."""
    q, k, v, out, dout = (rows_ready(t) for t in (q, k, v, out, dout))
    if dout.dtype != q.dtype:
        dout = dout.to(q.dtype)
    lse = lse.contiguous()
    dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    a = bwd_args(q, k, v, out, dout, lse, dq, dk, dv, softmax_scale, causal, deterministic,
                 window)
    lib = _lib.load()
    full = lib.fa_bwd_workspace_bytes(ctypes.byref(a))
    minimal = lib.fa_bwd_min_workspace_bytes(ctypes.byref(a))
    if full == 0 or minimal == 0:
        _lib.check(_lib.FA_E_INVALID, "fa_bwd_workspace_bytes")
    ws = alloc_workspace(full, minimal, q.device)
    nbytes = ws.numel()
    _lib.check(_lib.call_on(q.device, lambda st: lib.fa_bwd(ctypes.byref(a), ws.data_ptr(),
                                                            nbytes, st)), "fa_bwd")
    return dq, dk, dv
