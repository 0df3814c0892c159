"""Paged (vLLM 4-D cache) varlen attention: host side of fa_paged_prefill.

Mirrors paged_forward (tilelang_fa_v100/_paged_adapter.py:15-52): same
arguments, same defaults (num_kv_heads from k_cache.shape[2], scale 1/sqrt(D),
out allocated when None) and the same return value (out, softmax_lse).
Differences, all on the side of the caller:
  * the kernel writes into `out` directly (no extra copy, :49) and the
    returned `out` is the caller's tensor;
  * softmax_lse [num_heads, num_tokens] fp32 holds the natural-log LSE of
    every query row (the reference returns an uninitialised buffer, :51);
  * fp16 and bf16 are both accepted;
  * shape mistakes raise ValueError before any launch;
  * when the query tiles alone cannot fill the GPU (few new tokens, long
    block tables), the keys are split across workgroups and merged
    (fa_paged_prefill_splitkv; the split count comes from
    fa_paged_prefill_num_splits).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib
from ._checks import (PAGED_HEAD_DIMS, as_int32, require_cuda, require_half, require_same,
                      rows_ready, strides)


def paged_forward(q, k_cache, v_cache, block_table, seq_lens,
                  query_start_loc, prefix_kv_lens, out=None,
                  block_size=16, num_kv_heads=None, softmax_scale=None,
                  causal=True, sliding_window_q=-1, sliding_window_k=-1):
    return paged_forward_splits(q, k_cache, v_cache, block_table, seq_lens, query_start_loc,
                                prefix_kv_lens, out, block_size, num_kv_heads, softmax_scale,
                                causal, sliding_window_q, sliding_window_k)


def paged_forward_splits(q, k_cache, v_cache, block_table, seq_lens,
                         query_start_loc, prefix_kv_lens, out=None,
                         block_size=16, num_kv_heads=None, softmax_scale=None,
                         causal=True, sliding_window_q=-1, sliding_window_k=-1,
                         num_splits=None):
    """paged_forward with an explicit split-KV count (None: the library's)."""
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        require_half(t, name)
    require_same({"q": q, "k_cache": k_cache, "v_cache": v_cache}, "dtype")
    if q.dim() != 3:
        raise ValueError(f"q must be [num_tokens, num_heads, head_dim], got {tuple(q.shape)}")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache / v_cache must both be [num_pages, page_size, kv_heads, head_dim]")
    num_tokens, num_heads, D = q.shape
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
    if block_table.dim() != 2:
        raise ValueError("block_table must be [batch, max_blocks]")
    B = block_table.shape[0]
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        require_cuda(t, name)
    require_same({"q": q, "k_cache": k_cache, "v_cache": v_cache}, "device")
    dev = q.device
    bt = as_int32(block_table, dev, "block_table")
    sl = as_int32(seq_lens, dev, "seq_lens")
    qsl = as_int32(query_start_loc, dev, "query_start_loc")
    pkl = as_int32(prefix_kv_lens, dev, "prefix_kv_lens")
    if sl.shape != (B,) or pkl.shape != (B,):
        raise ValueError(f"seq_lens / prefix_kv_lens must have shape ({B},)")
    if qsl.shape != (B + 1,):
        raise ValueError(f"query_start_loc must have shape ({B + 1},)")

    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != dev:
        raise ValueError("out must match q in shape, dtype and device")
    lse = torch.empty((num_heads, num_tokens), dtype=torch.float32, device=dev)

    qr = rows_ready(q)
    kc, vc = rows_ready(k_cache), rows_ready(v_cache)
    target = rows_ready(out)

    a = _lib.PagedArgs()
    a.q, a.k_cache, a.v_cache = qr.data_ptr(), kc.data_ptr(), vc.data_ptr()
    a.out, a.lse = target.data_ptr(), lse.data_ptr()
    a.block_table, a.seq_lens = bt.data_ptr(), sl.data_ptr()
    a.query_start_loc, a.prefix_kv_lens = qsl.data_ptr(), pkl.data_ptr()
    a.q_stride[:] = strides(qr, 2)
    a.o_stride[:] = strides(target, 2)
    a.k_stride[:] = strides(kc, 3)
    a.v_stride[:] = strides(vc, 3)
    a.block_table_stride = bt.stride(0) if B > 1 else bt.shape[1]
    a.max_blocks = bt.shape[1]
    a.num_tokens, a.batch = num_tokens, B
    a.num_heads, a.num_kv_heads, a.head_dim = num_heads, heads_kv, D
    a.page_size, a.num_pages = page_size, num_pages
    a.softmax_scale = float(softmax_scale)
    a.causal = int(bool(causal))
    a.window_q = int(sliding_window_q)
    a.window_k = int(sliding_window_k)
    a.dtype = _lib.dtype_code(q.dtype)
    lib = _lib.load()

    def run(stream):
        ns = num_splits
        if ns is None:  # chosen from the sizes and the current device's CU count
            ns = lib.fa_paged_prefill_num_splits(ctypes.byref(a))
            _lib.check(min(ns, 0), "fa_paged_prefill_num_splits")
        nbytes = lib.fa_paged_prefill_splitkv_workspace_bytes(ctypes.byref(a), int(ns))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if nbytes else None
        return lib.fa_paged_prefill_splitkv(ctypes.byref(a), int(ns),
                                            ws.data_ptr() if ws is not None else None,
                                            nbytes, stream)

    _lib.check(_lib.call_on(dev, run), "fa_paged_prefill_splitkv")
    if target is not out:
        out.copy_(target)
    return out, lse
