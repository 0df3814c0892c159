"""KV-cache write (vLLM reshape_and_cache): host side of fa_reshape_and_cache.

Writes each new token's K and V rows into the paged cache layout that
tilelang_paged_forward and tilelang_decode_forward read,
[num_pages, page_size, num_kv_heads, head_dim] (the layout of the
reference's caches, tilelang_fa_v100/_kernels_paged.py:198-199).  The
reference has no cache writer; the argument names follow vLLM's
reshape_and_cache(key, value, key_cache, value_cache, slot_mapping).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._checks import require_cuda, require_half, require_same, rows_ready, strides


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping):
    """Copies key/value [T, Hkv, D] into the caches at slot_mapping [T].

    Token t goes to page slot_mapping[t] // page_size, slot
    slot_mapping[t] % page_size of both caches.  A negative entry (padding)
    or one at or beyond num_pages * page_size leaves the caches untouched.
    The caches are modified in place; nothing is returned.
    """
    for name, t in (("key", key), ("value", value), ("key_cache", key_cache),
                    ("value_cache", value_cache)):
        require_half(t, name)
    require_same({"key": key, "value": value, "key_cache": key_cache,
                  "value_cache": value_cache}, "dtype")
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("key / value must both be [num_tokens, num_kv_heads, head_dim]")
    if key_cache.dim() != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("key_cache / value_cache must both be "
                         "[num_pages, page_size, num_kv_heads, head_dim]")
    T, Hkv, D = key.shape
    num_pages, page_size, cache_heads, cache_d = key_cache.shape
    if (cache_heads, cache_d) != (Hkv, D):
        raise ValueError(f"cache rows [{cache_heads}, {cache_d}] do not match key rows [{Hkv}, {D}]")
    if D % 8 != 0 or D > 1024:
        raise ValueError(f"head_dim {D} must be a multiple of 8 and at most 1024")
    if not isinstance(slot_mapping, torch.Tensor):
        raise TypeError("slot_mapping must be a torch.Tensor")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"slot_mapping must be an integer tensor, got {slot_mapping.dtype}")
    if slot_mapping.shape != (T,):
        raise ValueError(f"slot_mapping must have shape ({T},), got {tuple(slot_mapping.shape)}")
    for name, t in (("key", key), ("value", value), ("key_cache", key_cache),
                    ("value_cache", value_cache)):
        require_cuda(t, name)
    require_same({"key": key, "value": value, "key_cache": key_cache,
                  "value_cache": value_cache}, "device")
    dev = key.device
    if T == 0:
        return
    slots = slot_mapping.to(device=dev, dtype=torch.int64).contiguous()
    k, v = rows_ready(key), rows_ready(value)
    kc, vc = rows_ready(key_cache), rows_ready(value_cache)
    if kc is not key_cache or vc is not value_cache:
        raise ValueError("key_cache / value_cache must have a contiguous head_dim, 16-byte "
                         "aligned rows and strides that are multiples of 8 (they are written "
                         "in place)")
    a = _lib.CacheWriteArgs()
    a.key, a.value = k.data_ptr(), v.data_ptr()
    a.k_cache, a.v_cache = kc.data_ptr(), vc.data_ptr()
    a.slot_mapping = slots.data_ptr()
    a.key_stride[:] = strides(k, 2)
    a.value_stride[:] = strides(v, 2)
    a.k_stride[:] = strides(kc, 3)
    a.v_stride[:] = strides(vc, 3)
    a.num_tokens, a.num_kv_heads, a.head_dim = T, Hkv, D
    a.page_size, a.num_pages = page_size, num_pages
    a.dtype = _lib.dtype_code(key.dtype)
    lib = _lib.load()
    _lib.check(_lib.call_on(dev, lambda st: lib.fa_reshape_and_cache(ctypes.byref(a), st)),
               "fa_reshape_and_cache")
