"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker or the timed CPU baseline; the
product path (tilelang-fa-v100_amd/) never calls it.

A plain-PyTorch fp32 (or fp64) restatement on the CPU of what the reference
(haohervchb/Tilelang-FA-V100) computes on this path.  Each function cites
the reference lines it follows.  The reference itself cannot run here
(TileLang and CUDA are absent), so the functions are pinned by the checks in
tests/test_oracle.py: brute-force enumeration on tiny inputs
(tests/golden/make_golden.py fixtures), closed forms, invariances, fp64
autograd and finite differences.  Every function below has such a check.

Conventions (all tensors CPU, computed in `dtype`, default float32):
  dense   q [B, Sq, H, D], k/v [B, Sk, Hk, D], H % Hk == 0, query head h uses
          KV head h // (H / Hk) (tests/test_gqa_paged.py:37-38,
          _kernels_paged.py:228);
  LSE     natural log of sum_j exp(scale * s_ij) (_kernels_forward.py:169-170);
  a row with no visible key: out = 0, lse = -inf.
"""
from __future__ import annotations

import math

import torch


def _expand_kv(k: torch.Tensor, heads: int) -> torch.Tensor:
    """[B, S, Hk, D] -> [B, S, H, D] with contiguous head groups."""
    g = heads // k.shape[2]
    return k.repeat_interleave(g, dim=2) if g > 1 else k


def dense_visible(sq: int, sk: int, causal: bool, window=(-1, -1)) -> torch.Tensor:
    """Bool [sq, sk]: key j visible to query i.

    Causal is bottom-right aligned, j <= i + sk - sq: the reference's oracle
    `torch.tril(ones(M, N), diagonal=N - M)` (tests/test_compare_ref.py:21-23)
    and its kernel mask (_kernels_forward.py:135-144).
    window = (left, right) follows FlashAttention-2's window_size, which the
    reference's signature carries (interface.py:59-62) but ignores (:33):
    j >= i + off - left when left >= 0, j <= i + off + right when right >= 0,
    off = sk - sq; causal implies right = 0.
    """
    i = torch.arange(sq).unsqueeze(1)
    j = torch.arange(sk).unsqueeze(0)
    off = sk - sq
    left, right = window
    if causal:
        right = 0
    vis = torch.ones(sq, sk, dtype=torch.bool)
    if right >= 0:
        vis &= j <= i + off + right
    if left >= 0:
        vis &= j >= i + off - left
    return vis


def masked_softmax_attention(q, k, v, visible, scale, dtype=torch.float32):
    """Single-sequence core: q [Sq, H, D], k/v [Sk, H, D], visible [Sq, Sk] or
    [H, Sq, Sk].  Returns out [Sq, H, D] and lse [H, Sq] (natural log)."""
    qf, kf, vf = (t.to(dtype) for t in (q, k, v))
    s = torch.einsum("qhd,khd->hqk", qf, kf) * scale
    vis = visible if visible.dim() == 3 else visible.unsqueeze(0)
    s = s.masked_fill(~vis, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)                       # [H, Sq]
    empty = torch.isneginf(lse)
    p = torch.exp(s - torch.where(empty, torch.zeros_like(lse), lse).unsqueeze(-1))
    p = p.masked_fill(empty.unsqueeze(-1), 0.0)
    out = torch.einsum("hqk,khd->qhd", p, vf)
    return out, lse


def dense_attention(q, k, v, scale=None, causal=False, dtype=torch.float32, window=(-1, -1)):
    """softmax(scale * Q K^T + mask) V and its LSE.

    Follows tests/test_compare_ref.py:15-25 (math) and
    _kernels_forward.py:94-172 (LSE output, :169-170).
    Returns out [B, Sq, H, D] (dtype) and lse [B, H, Sq] (dtype).
    """
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ke, ve = _expand_kv(k, H), _expand_kv(v, H)
    vis = dense_visible(Sq, Sk, causal, window)
    outs, lses = [], []
    for b in range(B):
        o, l = masked_softmax_attention(q[b], ke[b], ve[b], vis, scale, dtype)
        outs.append(o)
        lses.append(l)
    return torch.stack(outs), torch.stack(lses)


def dense_attention_backward(q, k, v, dout, scale=None, causal=False, dtype=torch.float32,
                             window=(-1, -1), round_dtype=None):
    """Gradients of dense_attention w.r.t. q, k, v by the FlashAttention-2
    formulas the reference kernels implement:
      P = exp(scale*S - lse), rowdot = sum_d O*dO   (_kernels_backward.py:203)
      dP = dO V^T, dS = P * (dP - rowdot) * scale  (:55, :72-74, :157-163)
      dV = P^T dO, dK = dS^T Q, dQ = dS K           (:80, :165-170)
    GQA: dK / dV of a KV head sum over its query-head group.
    round_dtype (e.g. torch.float16): also restate the reference's roundings
    to 16 bits - rowdot from the 16-bit forward output (:203 reads out_),
    P rounded before dV (:162-166) and scale*dS rounded before dK and dQ
    (:74-80, :167-170) - with the products still accumulated in `dtype`.
    None (default): no rounding, the exact gradient in `dtype`.
    Returns dq, dk, dv in `dtype`.
    """
    B, Sq, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    g = H // Hk
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    ke, ve = _expand_kv(k, H).to(dtype), _expand_kv(v, H).to(dtype)
    qf, dof = q.to(dtype), dout.to(dtype)
    vis = dense_visible(Sq, Sk, causal, window)
    dq = torch.zeros(B, Sq, H, D, dtype=dtype)
    dke = torch.zeros(B, Sk, H, D, dtype=dtype)
    dve = torch.zeros(B, Sk, H, D, dtype=dtype)
    for b in range(B):
        s = torch.einsum("qhd,khd->hqk", qf[b], ke[b]) * scale
        s = s.masked_fill(~vis.unsqueeze(0), float("-inf"))
        lse = torch.logsumexp(s, dim=-1, keepdim=True)
        lse = torch.where(torch.isneginf(lse), torch.full_like(lse, float("inf")), lse)
        p = torch.exp(s - lse)                                    # [H, Sq, Sk]
        o = torch.einsum("hqk,khd->qhd", p, ve[b])
        if round_dtype is not None:
            o = o.to(round_dtype).to(dtype)
        rowdot = (o * dof[b]).sum(-1).transpose(0, 1).unsqueeze(-1)   # [H, Sq, 1]
        dp = torch.einsum("qhd,khd->hqk", dof[b], ve[b])
        ds = p * (dp - rowdot) * scale
        if round_dtype is not None:
            p = p.to(round_dtype).to(dtype)
            ds = ds.to(round_dtype).to(dtype)
        dve[b] = torch.einsum("hqk,qhd->khd", p, dof[b])
        dke[b] = torch.einsum("hqk,qhd->khd", ds, qf[b])
        dq[b] = torch.einsum("hqk,khd->qhd", ds, ke[b])
    dk = dke.view(B, Sk, Hk, g, D).sum(3)
    dv = dve.view(B, Sk, Hk, g, D).sum(3)
    return dq, dk, dv


# --------------------------------------------------------------------- cache write

def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping):
    """In-place copy of key/value [T, Hkv, D] rows into [P, page, Hkv, D] caches.

    The layout paged_rows reads (_kernels_paged.py:198-199, 265-272): token t
    lands on page slot // page, slot slot % page.  Negative slots (padding)
    and slots at or beyond P * page are skipped.  Written as a per-token loop
    (the definition itself), not as the vectorised scatter the tests compare
    with.
    """
    P, page = k_cache.shape[0], k_cache.shape[1]
    for t in range(key.shape[0]):
        s = int(slot_mapping[t])
        if s < 0 or s >= P * page:
            continue
        k_cache[s // page, s % page] = key[t]
        v_cache[s // page, s % page] = value[t]


# --------------------------------------------------------------------- paged

def paged_rows(cache, block_table_row, n):
    """Rows 0..n-1 of one sequence from a [num_pages, page, Hkv, D] cache.

    Page resolution of _kernels_paged.py:265-272: logical page lp = pos // page,
    slot = pos - lp * page, physical = block_table[b, lp].
    Returns [n, Hkv, D].
    """
    page = cache.shape[1]
    pos = torch.arange(n)
    lp = torch.div(pos, page, rounding_mode="floor")
    phys = block_table_row[lp].long()
    return cache[phys, pos - lp * page]


def paged_visible(q_len, seq_len, prefix, causal, window_q=-1, window_k=-1):
    """Bool [q_len, seq_len]: key n visible to local query token t.

    _kernels_paged.py:274-308: causal  n <= prefix + t  and  n < seq_len;
    non-causal  n < seq_len; when causal and a window is set,
    t < n + window_q (window_q > 0) and n < t + window_k (window_k > 0),
    with t the local query index (:277,283-288).
    """
    t = torch.arange(q_len).unsqueeze(1)
    n = torch.arange(seq_len).unsqueeze(0)
    vis = torch.ones(q_len, seq_len, dtype=torch.bool)
    if causal:
        vis &= n <= prefix + t
        if window_q > 0:
            vis &= t < n + window_q
        if window_k > 0:
            vis &= n < t + window_k
    return vis


def paged_attention(q, k_cache, v_cache, block_table, seq_lens, query_start_loc,
                    prefix_kv_lens, scale=None, causal=True, window_q=-1, window_k=-1,
                    dtype=torch.float32):
    """Varlen paged attention as _kernels_paged.py:193-344 computes it.

    q [T, Hq, D] (T = total query tokens), caches [P, page, Hkv, D].
    Returns out [T, Hq, D] and lse [Hq, T] (the LSE the reference leaves
    uninitialised, _paged_adapter.py:51, defined here by its closed form).
    """
    T, Hq, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.zeros(T, Hq, D, dtype=dtype)
    lse = torch.full((Hq, T), float("-inf"), dtype=dtype)
    B = block_table.shape[0]
    for b in range(B):
        s0, s1 = int(query_start_loc[b]), int(query_start_loc[b + 1])
        n = int(seq_lens[b])
        kb = _expand_kv(paged_rows(k_cache, block_table[b], n).unsqueeze(0), Hq)[0]
        vb = _expand_kv(paged_rows(v_cache, block_table[b], n).unsqueeze(0), Hq)[0]
        vis = paged_visible(s1 - s0, n, int(prefix_kv_lens[b]), causal, window_q, window_k)
        o, l = masked_softmax_attention(q[s0:s1], kb, vb, vis, scale, dtype)
        out[s0:s1] = o
        lse[:, s0:s1] = l
    return out, lse


def decode_attention(q, k_cache, v_cache, block_table, seq_lens, scale=None,
                     dtype=torch.float32):
    """One query token per sequence, mask key < seq_len (_kernels_paged.py:450-451).

    q [B, Hq, D]; returns out [B, Hq, D] and lse [B, Hq].
    """
    B, Hq, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.zeros(B, Hq, D, dtype=dtype)
    lse = torch.full((B, Hq), float("-inf"), dtype=dtype)
    for b in range(B):
        n = int(seq_lens[b])
        kb = _expand_kv(paged_rows(k_cache, block_table[b], n).unsqueeze(0), Hq)[0]
        vb = _expand_kv(paged_rows(v_cache, block_table[b], n).unsqueeze(0), Hq)[0]
        vis = torch.ones(1, n, dtype=torch.bool)
        o, l = masked_softmax_attention(q[b].unsqueeze(0), kb, vb, vis, scale, dtype)
        out[b] = o[0]
        lse[b] = l[:, 0]
    return out, lse


def merge_partials(outs, lses):
    """LSE-weighted merge of attention over disjoint key sets.

    outs [S, ..., D] (each normalised over its own keys), lses [S, ...].
    The merge of the reference's split-KV variant (_kernels_paged.py:175-187).
    """
    m = lses.max(dim=0).values
    m_safe = torch.where(torch.isneginf(m), torch.zeros_like(m), m)
    w = torch.exp(lses - m_safe)
    tot = w.sum(0)
    out = (w.unsqueeze(-1) * outs).sum(0) / torch.where(tot > 0, tot, torch.ones_like(tot)).unsqueeze(-1)
    lse = torch.where(tot > 0, m_safe + torch.log(tot), torch.full_like(tot, float("-inf")))
    return out, lse


# --------------------------------------------------------------------- counts

def dense_pairs(sq: int, sk: int, causal: bool) -> int:
    """Number of visible (query, key) pairs of one head."""
    if not causal:
        return sq * sk
    off = sk - sq
    return sum(max(0, min(i + off + 1, sk)) for i in range(sq))


def paged_pairs(q_lens, seq_lens, prefixes, causal=True) -> int:
    """Visible pairs per query head of a paged batch."""
    total = 0
    for ql, sl, pf in zip(q_lens, seq_lens, prefixes):
        if causal:
            total += sum(min(pf + t + 1, sl) for t in range(ql))
        else:
            total += ql * sl
    return total
