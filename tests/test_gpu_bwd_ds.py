"""GPU parity: the two dq paths of fa_bwd at head_dim 128 and 256.

With the workspace fa_bwd_workspace_bytes asks for, the dK / dV kernel stores
its dS tiles and dq = scale * dS K is formed from them; with
fa_bwd_min_workspace_bytes, a query-stationary kernel recomputes S and dP.
Both are checked against the fp32 CPU oracle (atol 2e-3 / rtol 1e-2, relative
L2 < 1e-2) and for bit-for-bit repeats; dk and dv come from the same kernel
with the same row statistics on both paths, so they must agree exactly.  The
dS workspace is filled with NaN bytes first, so a tile the dq kernel reads
but the dK / dV kernel did not write shows up as NaN.
"""
import ctypes

import pytest
import torch

from helpers import assert_close, randn, rel_l2
from oracle import attention_ref as ref
from tilelang_fa_v100 import _dense, _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

CASES = [
    # (B, Sq, Sk, H, Hk, D, causal, dtype)
    (1, 700, 700, 4, 4, 128, True, torch.float16),
    (1, 300, 500, 4, 2, 128, True, torch.bfloat16),     # Sk > Sq, GQA
    (1, 500, 300, 2, 2, 128, True, torch.float16),      # Sq > Sk: rows that see no key
    (2, 333, 333, 4, 4, 128, False, torch.float16),     # full attention, ragged tiles
    (1, 77, 1030, 2, 1, 128, False, torch.bfloat16),    # MQA, one partial query tile
    (1, 1, 300, 2, 2, 128, True, torch.float16),        # one query row
    (1, 40, 1, 2, 2, 128, False, torch.float16),        # one key
    (1, 2100, 2100, 2, 2, 128, True, torch.float16),    # several 256-row query blocks
    (2, 2080, 2080, 32, 8, 128, True, torch.float16),   # GQA 4:1, 576 dQ workgroups
    (1, 700, 700, 2, 2, 256, True, torch.float16),
    (1, 300, 500, 4, 2, 256, True, torch.bfloat16),     # Sk > Sq, GQA
    (1, 500, 300, 2, 2, 256, True, torch.float16),      # Sq > Sk
    (2, 333, 200, 2, 1, 256, False, torch.float16),     # full attention, MQA
    (1, 1, 90, 2, 2, 256, True, torch.float16),         # one query row
    # dQ-from-dS loop edges: 2, 3 and 4 key steps (the steady loop runs all
    # but the last two; its two-step tail), full and causal.  bf16 only where
    # every row sees many keys: with Sq > Sk a causal row near the top sees
    # one or two keys, dP - rowdot cancels, and the rowdot of the bf16-rounded
    # O alone moves dq by up to 5e-3 (fp64 check), above atol.
    (1, 64, 64, 2, 2, 128, False, torch.float16),
    (1, 96, 96, 2, 2, 128, False, torch.bfloat16),
    (1, 128, 128, 2, 1, 128, True, torch.float16),
    (1, 96, 96, 2, 2, 256, False, torch.float16),
    (1, 128, 100, 2, 2, 256, True, torch.float16),
    (1, 100, 128, 2, 2, 256, True, torch.bfloat16),
]


def _ids(c):
    B, Sq, Sk, H, Hk, D, causal, dt = c
    return f"B{B}-{Sq}x{Sk}-H{H}/{Hk}-D{D}-{'c' if causal else 'nc'}-{str(dt)[6:]}"


def _bwd(q, k, v, out, lse, do, scale, causal, minimal):
    lib = _lib.load()
    dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
    a = _dense.bwd_args(q, k, v, out, do, lse, dq, dk, dv, scale, causal, False)
    full = lib.fa_bwd_workspace_bytes(ctypes.byref(a))
    low = lib.fa_bwd_min_workspace_bytes(ctypes.byref(a))
    assert low > 0 and full > low, "head_dim 128 / 256, causal / full: the dS path applies"
    n = low if minimal else full
    ws = torch.full((n,), 0xFF, dtype=torch.uint8, device=DEV)
    _lib.check(_lib.call_on(q.device, lambda st: lib.fa_bwd(ctypes.byref(a), ws.data_ptr(), n,
                                                            st)), "fa_bwd")
    torch.cuda.synchronize()
    return dq, dk, dv


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_dq_paths_match_oracle_and_each_other(case):
    B, Sq, Sk, H, Hk, D, causal, dt = case
    g = torch.Generator().manual_seed(41)
    q, do = randn(g, B, Sq, H, D, dtype=dt), None
    k, v = randn(g, B, Sk, Hk, D, dtype=dt), randn(g, B, Sk, Hk, D, dtype=dt)
    do = randn(g, B, Sq, H, D, dtype=dt)
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    scale = D ** -0.5
    print(f"case {_ids(case)}", flush=True)
    out, lse = _dense.forward(qd, kd, vd, scale, causal)
    ds_path = _bwd(qd, kd, vd, out, lse, dod, scale, causal, minimal=False)
    ds_again = _bwd(qd, kd, vd, out, lse, dod, scale, causal, minimal=False)
    rc_path = _bwd(qd, kd, vd, out, lse, dod, scale, causal, minimal=True)
    r = ref.dense_attention_backward(q, k, v, do, causal=causal)
    for i, name in enumerate(("dq", "dk", "dv")):
        assert torch.equal(ds_path[i], ds_again[i]), f"{name}: two runs differ"
        if name != "dq":
            assert torch.equal(ds_path[i], rc_path[i]), f"{name}: paths differ"
        for got in (ds_path[i], rc_path[i]):
            assert torch.isfinite(got.float()).all(), name
            assert_close(got, r[i], what=name)
            if r[i].abs().max() > 1e-4:
                assert rel_l2(got, r[i]) < 1e-2, name


def test_public_backward_honours_workspace_limit():
    """tilelang_flash_attn_func's backward takes the dS path by default and
    the recompute path (the reference's memory footprint) when the workspace
    limit is below the dS workspace: its gradients then equal fa_bwd's with
    the minimal workspace bit for bit, and both match the oracle."""
    import tilelang_fa_v100 as fa

    B, S, H, D = 1, 900, 4, 128
    g = torch.Generator().manual_seed(43)
    q, k, v, do = (randn(g, B, S, H, D) for _ in range(4))
    qd, kd, vd, dod = (t.to(DEV) for t in (q, k, v, do))
    scale = D ** -0.5
    out, lse = _dense.forward(qd, kd, vd, scale, True)
    ds_path = _bwd(qd, kd, vd, out, lse, dod, scale, True, minimal=False)
    rc_path = _bwd(qd, kd, vd, out, lse, dod, scale, True, minimal=True)
    r = ref.dense_attention_backward(q, k, v, do, causal=True)
    try:
        for limit, want_path in ((None, ds_path), (0, rc_path), (1 << 40, ds_path)):
            fa.set_backward_workspace_limit(limit)
            qa, ka, va = (t.clone().requires_grad_() for t in (qd, kd, vd))
            fa.tilelang_flash_attn_func(qa, ka, va, causal=True).backward(dod)
            torch.cuda.synchronize()
            for got, want, exact, name in zip((qa.grad, ka.grad, va.grad), r, want_path,
                                              ("dq", "dk", "dv")):
                assert torch.equal(got, exact), f"{name} (limit {limit}): not the chosen path"
                assert_close(got, want, what=name)
    finally:
        fa.set_backward_workspace_limit(None)
