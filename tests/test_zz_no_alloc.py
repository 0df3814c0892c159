"""fa_paged_decode_noalloc (static device scratch) against fa_paged_decode.

The allocation-free entry point runs the same validation and kernels as
fa_paged_decode with the split-KV workspace taken from the library's static
per-device scratch array, so on the same inputs its output and LSE must be
bit-identical to the workspace entry point's.  Two calls in a row, the second
with a smaller problem (the array keeps the first call's contents), at
head_dim 128 and at head_dim 256 then 64 (all on the streaming decode
kernel).
"""
import ctypes

import pytest
import torch

from helpers import build_paged, randn
from tilelang_fa_v100 import _lib
from tilelang_fa_v100._decode_adapter import _decode_args, decode_forward

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def problem(seed, lens, Hq, Hkv, D, dtype, page=16):
    g = torch.Generator().manual_seed(seed)
    ks = [randn(g, n, Hkv, D, dtype=dtype) for n in lens]
    vs = [randn(g, n, Hkv, D, dtype=dtype) for n in lens]
    kc, vc, bt = build_paged(g, ks, vs, page, dtype=dtype)
    q = randn(g, len(lens), Hq, D, dtype=dtype)
    return [t.to(DEV) for t in (q, kc, vc, bt)] + [torch.tensor(lens, dtype=torch.int32,
                                                                device=DEV)]


def run_noalloc(q, kc, vc, bt, sl):
    a, out, lse, keep = _decode_args(q, kc, vc, bt, sl, kc.shape[1], None, None, True)
    lib = _lib.load()
    nbytes = lib.fa_decode_workspace_bytes(ctypes.byref(a))
    assert 0 < nbytes <= (64 << 20)
    _lib.check(lib.fa_paged_decode_noalloc(ctypes.byref(a), _lib.stream_handle(q.device)),
               "fa_paged_decode_noalloc")
    torch.cuda.synchronize()
    del keep
    return out, lse


CASES = [
    # first call (larger), second call (smaller)
    ((11, [9000, 3000, 17, 4097, 1, 2500, 8000, 640], 32, 8, 128, torch.float16),
     (12, [300, 5], 32, 8, 128, torch.float16)),
    ((13, [5000, 1200, 33], 16, 2, 256, torch.bfloat16),
     (14, [70], 8, 2, 64, torch.float16)),
]


@pytest.mark.parametrize("first,second", CASES, ids=["d128", "d256_d64"])
def test_noalloc_decode_matches_workspace_entry_point(first, second):
    for seed, lens, Hq, Hkv, D, dt in (first, second):
        args = problem(seed, lens, Hq, Hkv, D, dt)
        out, lse = run_noalloc(*args)
        ref_out, ref_lse = decode_forward(*args, block_size=16, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), f"out differs (seed {seed})"
        assert torch.equal(lse, ref_lse), f"lse differs (seed {seed})"
        assert torch.isfinite(out.float()).all()
