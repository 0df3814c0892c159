"""Shared builders for the GPU parity tests (CPU-side, seeded)."""
from __future__ import annotations

import math

import torch

# outputs / gradients vs fp32, LSE absolute.
ATOL, RTOL, LSE_ATOL = 2e-3, 1e-2, 1e-3


def randn(gen, *shape, dtype=torch.float16, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(dtype)


def build_paged(gen, k_seqs, v_seqs, page, extra_pages=3, sentinel=float("nan"),
                dtype=torch.float16):
    """Scatters per-sequence K/V ([n_b, Hkv, D] each) into a paged cache.

    Pages are a seeded random permutation of the pool; every slot that holds no
    key (unused pool pages, the tail of each last page) is filled with
    `sentinel`, and block-table padding is -1, so a kernel that reads outside
    the visible keys produces NaN or faults in the bounds checks.
    Returns k_cache, v_cache [P, page, Hkv, D] and block_table [B, max_blocks].
    """
    Hkv, D = k_seqs[0].shape[1:]
    npages = [math.ceil(k.shape[0] / page) for k in k_seqs]
    pool = sum(npages) + extra_pages
    perm = torch.randperm(pool, generator=gen)
    kc = torch.full((pool, page, Hkv, D), sentinel, dtype=dtype)
    vc = torch.full((pool, page, Hkv, D), sentinel, dtype=dtype)
    maxb = max(max(npages), 1) + 1
    bt = torch.full((len(k_seqs), maxb), -1, dtype=torch.int32)
    cur = 0
    for b, (k, v) in enumerate(zip(k_seqs, v_seqs)):
        for p in range(npages[b]):
            phys = int(perm[cur])
            cur += 1
            bt[b, p] = phys
            rows = slice(p * page, min((p + 1) * page, k.shape[0]))
            n = rows.stop - rows.start
            kc[phys, :n] = k[rows].to(dtype)
            vc[phys, :n] = v[rows].to(dtype)
    return kc, vc, bt


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what="out"):
    got = got.float().cpu()
    ref = ref.float().cpu()
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    err = (got - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = err > bound
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(
            f"{what}: {int(bad.sum())} elements out of tolerance; max abs err "
            f"{err.max().item():.3e}; first bad {idx}: got {got[tuple(idx)].item():.6f} "
            f"ref {ref[tuple(idx)].item():.6f}")


def rel_l2(got, ref):
    got, ref = got.float().cpu(), ref.float().cpu()
    return ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def assert_lse(got, ref, atol=LSE_ATOL, what="lse"):
    got, ref = got.float().cpu(), ref.float().cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isneginf(got), torch.isneginf(ref)), f"{what}: -inf pattern differs"
    err = (got[fin] - ref[fin]).abs()
    assert err.numel() == 0 or err.max().item() <= atol, f"{what}: max err {err.max().item():.3e}"
