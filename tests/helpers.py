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


def assert_close_as_reference_arithmetic(got, ref, ref_rounded, what="grad", norm=1.0):
    """Gradient check against the exact fp32 gradient `ref` (all three divided
    by `norm`, e.g. a loss scale), element by element: within the north-star
    bound atol + rtol·|ref|, or within twice the largest error of
    `ref_rounded` - the oracle's restatement of the reference's own 16-bit
    roundings (dense_attention_backward(..., round_dtype=...)) - where that
    is larger.  The restatement's errors land on different elements than
    the kernel's (its roundings differ in the last bit here and there), so its
    largest error, not its error at the same element, sets the floor."""
    got = got.float().cpu() / norm
    ref = ref.float().cpu() / norm
    floor = 2 * (ref_rounded.float().cpu() / norm - ref).abs().max().item()
    assert torch.isfinite(got).all(), f"{what}: non-finite values"
    err = (got - ref).abs()
    bound = torch.clamp(ATOL + RTOL * ref.abs(), min=floor)
    bad = err > bound
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(
            f"{what}: {int(bad.sum())} elements out of tolerance; max abs err "
            f"{err.max().item():.3e} (reference arithmetic floor {floor:.3e}); first bad "
            f"{idx}: got {got[tuple(idx)].item():.6f} ref {ref[tuple(idx)].item():.6f}")


def standard_forward_batch(B, H, Sq, D):
    """Batch size (at least B) from which the dense forward of [B', Sq, H, D]
    runs on the row-tile cores rather than the key-split kernel: their grid,
    ceil(Sq / rows) x B' x H workgroups (rows = 128 at head_dim 64, 256 at
    head_dim 128), reaches half the CUs (csrc/fa_tiles.h kFwdSplitMaxFill).
    Head_dim 256 always runs on the row-tile core."""
    if D not in (64, 128):
        return B
    rows = 128 if D == 64 else 256
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    per_batch = math.ceil(Sq / rows) * H
    return max(B, math.ceil(math.ceil(cus / 2) / per_batch))


def rel_l2(got, ref):
    got, ref = got.float().cpu(), ref.float().cpu()
    return ((got - ref).norm() / ref.norm().clamp_min(1e-30)).item()


def assert_lse(got, ref, atol=LSE_ATOL, what="lse"):
    got, ref = got.float().cpu(), ref.float().cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(torch.isneginf(got), torch.isneginf(ref)), f"{what}: -inf pattern differs"
    err = (got[fin] - ref[fin]).abs()
    assert err.numel() == 0 or err.max().item() <= atol, f"{what}: max err {err.max().item():.3e}"


# ------------------------------------------------------------- needle inputs
# Scores that make P one-hot, so the output must equal one V row bit for bit.
# Key j carries the base-16 digits of j in dims 0..3 and q is +/-(1, 16, 256,
# 4096) there and 0 elsewhere, so s = q . k = +/-j exactly (integer products
# and sums below 2^24 are exact in the fp32 accumulators).  With a softmax
# scale whose fp32 product with log2(e) rounds to exactly 128, every score
# is a multiple of 128 in the kernels' base-2 domain: the row maximum gets
# p = exp2(0) = 1 and every other key p <= 2^-128, which vanishes next to it.
# Rising scores (+) put the needle on the LAST visible key of a row (causal
# edge, seq_len boundary, right window edge); falling scores (-) on the FIRST
# (left window edge, key 0).  An off-by-one in a mask or a wrong page then
# returns another V row, which equality detects.

NEEDLE_DIGITS = (1.0, 16.0, 256.0, 4096.0)


def needle_scale() -> float:
    """A float32 scale with fl32(scale * fl32(log2 e)) == 128 exactly."""
    import numpy as np

    log2e = np.float32(1.4426950408889634)
    x = np.float32(128.0) / log2e
    for _ in range(64):
        p = np.float32(x * log2e)
        if p == np.float32(128.0):
            return float(x)
        x = np.nextafter(x, np.float32(np.inf) if p < 128 else np.float32(-np.inf),
                         dtype=np.float32)
    raise AssertionError("no float32 scale maps to 128")


def needle_keys(gen, n, heads, D, dtype=torch.float16):
    """K [n, heads, D]: digits of the key index in dims 0..3, N(0,1) elsewhere."""
    assert n <= 1 << 16
    k = torch.randn(n, heads, D, generator=gen)
    j = torch.arange(n)
    for d in range(4):
        k[:, :, d] = ((j >> (4 * d)) & 15).float().unsqueeze(1)
    return k.to(dtype)


def needle_query(rows, heads, D, sign=1, dtype=torch.float16):
    """q [rows, heads, D] = sign * (1, 16, 256, 4096, 0, ...)."""
    q = torch.zeros(rows, heads, D)
    q[:, :, :4] = torch.tensor(NEEDLE_DIGITS) * sign
    return q.to(dtype)


def needle_expected(v_rows, visible, sign):
    """Per query row the V row of its last (sign > 0) or first visible key.

    v_rows [n, H, D] (already in query-head order), visible [Sq, n] bool.
    Rows with no visible key expect zeros.  Returns [Sq, H, D].
    """
    Sq, n = visible.shape
    if n == 0 or Sq == 0:
        return torch.zeros(Sq, *v_rows.shape[1:], dtype=v_rows.dtype)
    idx = torch.arange(n).expand(Sq, n)
    if sign > 0:
        pick = torch.where(visible, idx, torch.full_like(idx, -1)).max(1).values
    else:
        pick = torch.where(visible, idx, torch.full_like(idx, n)).min(1).values
    out = torch.zeros(Sq, *v_rows.shape[1:], dtype=v_rows.dtype)
    ok = visible.any(1)
    out[ok] = v_rows[pick[ok]]
    return out


def assert_equal_rows(got, want, what="out"):
    """Bit-exact equality; on failure names the first differing row."""
    got = got.cpu()
    want = want.to(got.dtype).cpu()
    same = (got == want) | (torch.isnan(got) & torch.isnan(want))
    if not bool(same.all()):
        bad = (~same).reshape(same.shape[0], -1).any(1).nonzero().flatten()
        raise AssertionError(f"{what}: {bad.numel()} rows differ; first rows {bad[:8].tolist()}")
