"""Paged single-token decode: host side of fa_paged_decode.

Mirrors decode_forward (tilelang_fa_v100/_decode_adapter.py:15-47): same
arguments and defaults, returns output [batch, heads, dim] in q's dtype.
Differences: `softmax_scale` is honoured (the reference computes it and then
uses a fixed 1/sqrt(D), :37-38 vs _kernels_paged.py:396; identical at the
default), bf16 is accepted, and the optional `return_lse=True` also returns
the natural-log LSE [batch, heads] fp32 of every query row.

The work is split over fixed-size key chunks (split-KV); the partial results
live in a workspace sized from max_blocks * block_size, allocated here from
torch's caching allocator.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._checks import (PAGED_HEAD_DIMS, as_int32, require_cuda, require_half, require_same,
                      rows_ready, strides)


def _decode_args(q, k_cache, v_cache, block_table, seq_lens, block_size, num_kv_heads,
                 softmax_scale, return_lse):
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        require_half(t, name)
    require_same({"q": q, "k_cache": k_cache, "v_cache": v_cache}, "dtype")
    if q.dim() != 3:
        raise ValueError(f"q must be [batch, num_heads, head_dim], got {tuple(q.shape)}")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache / v_cache must both be [num_pages, page_size, kv_heads, head_dim]")
    batch, num_heads, D = q.shape
    heads_kv = num_kv_heads or k_cache.shape[2]
    num_pages, page_size, cache_heads, cache_d = k_cache.shape
    if block_size != page_size:
        raise ValueError(f"block_size {block_size} != k_cache page size {page_size}")
    if heads_kv != cache_heads:
        raise ValueError(f"num_kv_heads {heads_kv} != k_cache heads {cache_heads}")
    if cache_d != D:
        raise ValueError(f"head_dim mismatch: q {D}, cache {cache_d}")
    if D not in PAGED_HEAD_DIMS:
        raise ValueError(f"head_dim {D} not supported (expected one of {PAGED_HEAD_DIMS})")
    if num_heads % heads_kv != 0:
        raise ValueError(f"num_heads {num_heads} is not a multiple of num_kv_heads {heads_kv}")
    if page_size <= 0 or page_size & (page_size - 1):
        raise ValueError(f"page size {page_size} must be a power of two")
    if block_table.dim() != 2 or block_table.shape[0] != batch:
        raise ValueError(f"block_table must be [{batch}, max_blocks]")
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        require_cuda(t, name)
    require_same({"q": q, "k_cache": k_cache, "v_cache": v_cache}, "device")
    dev = q.device
    bt = as_int32(block_table, dev, "block_table")
    sl = as_int32(seq_lens, dev, "seq_lens")
    if sl.shape != (batch,):
        raise ValueError(f"seq_lens must have shape ({batch},)")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    qr = rows_ready(q)
    kc, vc = rows_ready(k_cache), rows_ready(v_cache)
    out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    lse = torch.empty(q.shape[:2], dtype=torch.float32, device=dev) if return_lse else None

    a = _lib.DecodeArgs()
    a.q, a.k_cache, a.v_cache = qr.data_ptr(), kc.data_ptr(), vc.data_ptr()
    a.out = out.data_ptr()
    a.lse = lse.data_ptr() if lse is not None else None
    a.block_table, a.seq_lens = bt.data_ptr(), sl.data_ptr()
    a.q_stride[:] = strides(qr, 2)
    a.o_stride[:] = strides(out, 2)
    a.k_stride[:] = strides(kc, 3)
    a.v_stride[:] = strides(vc, 3)
    a.block_table_stride = bt.stride(0) if batch > 1 else bt.shape[1]
    a.max_blocks = bt.shape[1]
    a.max_seq_len = bt.shape[1] * page_size
    a.batch, a.num_heads, a.num_kv_heads, a.head_dim = batch, num_heads, heads_kv, D
    a.page_size, a.num_pages = page_size, num_pages
    a.softmax_scale = float(softmax_scale)
    a.dtype = _lib.dtype_code(q.dtype)
    return a, out, lse, (qr, kc, vc, bt, sl)


def decode_forward(q, k_cache, v_cache, block_table, seq_lens,
                   block_size=16, num_kv_heads=None, softmax_scale=None,
                   return_lse=False):
    """Paged decode forward; see the module docstring."""
    a, out, lse, keep = _decode_args(q, k_cache, v_cache, block_table, seq_lens, block_size,
                                     num_kv_heads, softmax_scale, return_lse)
    lib = _lib.load()

    def run(stream):
        # The workspace size depends on the current device (its CU count), so
        # it is queried with the launch's device current.
        nbytes = lib.fa_decode_workspace_bytes(ctypes.byref(a))
        if nbytes == 0:
            _lib.check(_lib.FA_E_INVALID, "fa_decode_workspace_bytes")
        ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
        return lib.fa_paged_decode(ctypes.byref(a), ws.data_ptr(), nbytes, stream)

    _lib.check(_lib.call_on(q.device, run), "fa_paged_decode")
    del keep
    return (out, lse) if return_lse else out
