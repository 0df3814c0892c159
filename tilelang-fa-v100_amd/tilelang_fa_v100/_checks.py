"""Argument checks shared by the Python entry points.

Shape and dtype mistakes are reported as ValueError / TypeError before any
device work, mirroring where the reference surfaced TileLang binding errors
(tilelang_fa_v100/_kernels_paged.py:196-206 signatures).
"""
from __future__ import annotations

import torch

_FLOAT16 = (torch.float16, torch.bfloat16)
HEAD_DIMS = (64, 128, 256)             # dense forward / backward
PAGED_HEAD_DIMS = (64, 128, 256, 512)  # paged prefill and decode (_kernels_paged.py:353-364)


def require_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU device, got {t.device}")


def require_half(t: torch.Tensor, name: str) -> None:
    if t.dtype not in _FLOAT16:
        raise TypeError(f"{name} must be float16 or bfloat16, got {t.dtype}")


def require_same(ts: dict, what: str) -> None:
    names = list(ts)
    first = ts[names[0]]
    for n in names[1:]:
        if what == "dtype" and ts[n].dtype != first.dtype:
            raise TypeError(f"{n} dtype {ts[n].dtype} differs from {names[0]} dtype {first.dtype}")
        if what == "device" and ts[n].device != first.device:
            raise ValueError(f"{n} is on {ts[n].device} but {names[0]} is on {first.device}")


def rows_ready(t: torch.Tensor) -> torch.Tensor:
    """Returns t, or a contiguous copy when the kernels cannot address it.

    The kernels read 16-byte vectors along the last dimension, so it must be
    contiguous, every other stride a multiple of 8 elements and the base
    16-byte aligned.
    """
    if t.is_contiguous() and t.data_ptr() % 16 == 0 and t.shape[-1] % 8 == 0:
        return t  # common case: every stride is a multiple of the last dim
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0
    if ok:
        for size, st in zip(t.shape[:-1], t.stride()[:-1]):
            if size > 1 and (st % 8 != 0 or st < 0):
                ok = False
                break
    return t if ok else t.contiguous()


def strides(t: torch.Tensor, n: int) -> tuple:
    """Element strides of the leading n dimensions (0 for size-1 dims)."""
    sh, st = t.shape, t.stride()
    return tuple(0 if sh[i] == 1 else st[i] for i in range(n))


def as_int32(t: torch.Tensor, device: torch.device, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"{name} must be an integer tensor, got {t.dtype}")
    return t.to(device=device, dtype=torch.int32).contiguous()
