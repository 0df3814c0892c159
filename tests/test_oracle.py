"""Pins the CPU oracle (oracle/attention_ref.py) without the reference.

Each oracle function is checked against something other than its own
formula: brute-force golden vectors (tests/golden/make_golden.py), closed
forms, invariances, fp64 autograd / finite differences, and bit-exact
enumeration for the integer parts.  Planted-mistake tests show that a wrong
mask anchor, a transposed GQA map or a dropped scale would fail them.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention_ref as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def t64(x):
    return torch.from_numpy(np.asarray(x)).to(torch.float64)


# ------------------------------------------------------------------ golden

@pytest.mark.parametrize("name", ["dense_nc", "dense_c_skgt", "dense_c_sqgt"])
def test_dense_matches_golden(gold, name):
    q, k, v = (t64(gold[f"{name}/{x}"]) for x in "qkv")
    out, lse = ref.dense_attention(q, k, v, float(gold[f"{name}/scale"]),
                                   bool(gold[f"{name}/causal"]), dtype=torch.float64)
    torch.testing.assert_close(out, t64(gold[f"{name}/out"]), atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(lse, t64(gold[f"{name}/lse"]), atol=1e-12, rtol=1e-12)


def test_dense_empty_rows_are_zero_and_neg_inf(gold):
    # Sq=6 > Sk=3 causal: rows 0..2 see no key.
    out, lse = ref.dense_attention(t64(gold["dense_c_sqgt/q"]), t64(gold["dense_c_sqgt/k"]),
                                   t64(gold["dense_c_sqgt/v"]), 0.5, True, dtype=torch.float64)
    assert torch.all(out[:, :3] == 0)
    assert torch.all(torch.isneginf(lse[..., :3]))
    assert torch.all(torch.isfinite(lse[..., 3:]))


def test_backward_matches_finite_differences(gold):
    q, k, v, do = (t64(gold[f"bwd/{x}"]) for x in ("q", "k", "v", "dout"))
    dq, dk, dv = ref.dense_attention_backward(q, k, v, do, float(gold["bwd/scale"]), True,
                                              dtype=torch.float64)
    for got, name in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        torch.testing.assert_close(got, t64(gold[f"bwd/{name}"]), atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("tag", ["c", "nc", "win"])
def test_paged_matches_golden(gold, tag):
    g = {k.split("/", 1)[1]: v for k, v in gold.items() if k.startswith("paged/")}
    out, lse = ref.paged_attention(
        t64(g["q"]), t64(g["k_cache"]), t64(g["v_cache"]), torch.from_numpy(g["block_table"]),
        g["seq_lens"], g["query_start_loc"], g["prefix_kv_lens"], float(g["scale"]),
        causal=bool(gold[f"paged_{tag}/causal"]), window_q=int(gold[f"paged_{tag}/wq"]),
        window_k=int(gold[f"paged_{tag}/wk"]), dtype=torch.float64)
    torch.testing.assert_close(out, t64(gold[f"paged_{tag}/out"]), atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(lse, t64(gold[f"paged_{tag}/lse"]), atol=1e-12, rtol=1e-12)


def test_decode_matches_golden(gold):
    g = {k.split("/", 1)[1]: v for k, v in gold.items() if k.startswith("decode/")}
    out, lse = ref.decode_attention(t64(g["q"]), t64(g["k_cache"]), t64(g["v_cache"]),
                                    torch.from_numpy(g["block_table"]), g["seq_lens"],
                                    float(g["scale"]), dtype=torch.float64)
    torch.testing.assert_close(out, t64(g["out"]), atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(lse, t64(g["lse"]), atol=1e-12, rtol=1e-12)


# ------------------------------------------------------------------ closed forms

def test_zero_query_gives_mean_of_visible_values():
    g = torch.Generator().manual_seed(1)
    k = torch.randn(1, 9, 2, 8, generator=g, dtype=torch.float64)
    v = torch.randn(1, 9, 2, 8, generator=g, dtype=torch.float64)
    q = torch.zeros(1, 6, 2, 8, dtype=torch.float64)
    out, lse = ref.dense_attention(q, k, v, 0.3, causal=True, dtype=torch.float64)
    for i in range(6):
        n = i + 9 - 6 + 1  # visible keys of row i
        torch.testing.assert_close(out[0, i], v[0, :n].mean(0), atol=1e-12, rtol=0)
        torch.testing.assert_close(lse[0, :, i], torch.full((2,), math.log(n), dtype=torch.float64),
                                   atol=1e-12, rtol=0)


def test_single_visible_key_returns_that_value_row():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(1, 4, 1, 16, generator=g)
    k = torch.randn(1, 4, 1, 16, generator=g)
    v = torch.randn(1, 4, 1, 16, generator=g)
    out, lse = ref.dense_attention(q, k, v, 0.25, causal=True)
    # causal Sq == Sk: row 0 sees only key 0 -> out is exactly v[0], lse = scale * q.k
    assert torch.equal(out[0, 0, 0], v[0, 0, 0])
    torch.testing.assert_close(lse[0, 0, 0], 0.25 * (q[0, 0, 0] @ k[0, 0, 0]), atol=1e-6, rtol=0)


def test_invariances():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 5, 4, 8, generator=g, dtype=torch.float64)
    k = torch.randn(2, 11, 2, 8, generator=g, dtype=torch.float64)
    v = torch.randn(2, 11, 2, 8, generator=g, dtype=torch.float64)
    out, lse = ref.dense_attention(q, k, v, 0.4, causal=False, dtype=torch.float64)
    perm = torch.randperm(11, generator=g)
    out_p, lse_p = ref.dense_attention(q, k[:, perm], v[:, perm], 0.4, False, dtype=torch.float64)
    torch.testing.assert_close(out_p, out, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(lse_p, lse, atol=1e-12, rtol=1e-12)
    out_s, _ = ref.dense_attention(q, k, 3.0 * v, 0.4, False, dtype=torch.float64)
    torch.testing.assert_close(out_s, 3.0 * out, atol=1e-12, rtol=1e-12)
    # GQA equals MHA with explicitly repeated KV heads
    out_r, _ = ref.dense_attention(q, k.repeat_interleave(2, 2), v.repeat_interleave(2, 2), 0.4,
                                   False, dtype=torch.float64)
    torch.testing.assert_close(out_r, out, atol=0, rtol=0)


def test_backward_matches_autograd_fp64():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(2, 7, 4, 8, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(2, 9, 2, 8, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(2, 9, 2, 8, generator=g, dtype=torch.float64, requires_grad=True)
    do = torch.randn(2, 7, 4, 8, generator=g, dtype=torch.float64)
    for causal in (False, True):
        out, _ = ref.dense_attention(q, k, v, 0.35, causal, dtype=torch.float64)
        gq, gk, gv = torch.autograd.grad(out, (q, k, v), do)
        dq, dk, dv = ref.dense_attention_backward(q.detach(), k.detach(), v.detach(), do, 0.35,
                                                  causal, dtype=torch.float64)
        torch.testing.assert_close(dq, gq, atol=1e-10, rtol=1e-9)
        torch.testing.assert_close(dk, gk, atol=1e-10, rtol=1e-9)
        torch.testing.assert_close(dv, gv, atol=1e-10, rtol=1e-9)


def test_backward_rounding_restatement():
    """round_dtype restates the reference's 16-bit roundings.  Rounding to
    the compute dtype itself changes nothing (so the formula is the pinned
    exact one).  With one query row, head_dim 1, q = 1 and dO = 1, dK[j] is
    the rounded scale*dS[j] and dV[j] the rounded P[j] themselves, so they
    must be fp16 values equal to an independent restatement that rounds
    scale*dS (not dS) and P, with rowdot from the rounded output."""
    g = torch.Generator().manual_seed(12)
    q, k, v, do = (torch.randn(2, 9, 4, 8, generator=g).half() for _ in range(4))
    k, v = k[:, :, :2].contiguous(), v[:, :, :2].contiguous()
    for causal in (False, True):
        exact = ref.dense_attention_backward(q, k, v, do, 0.3, causal)
        same = ref.dense_attention_backward(q, k, v, do, 0.3, causal, round_dtype=torch.float32)
        for a, b in zip(exact, same):
            assert torch.equal(a, b)
    scale = 0.7
    q1 = torch.ones(1, 1, 1, 1)
    k1 = torch.tensor([0.3, -1.2, 2.5, 0.9, -0.4]).view(1, 5, 1, 1)
    v1 = torch.tensor([1.7, -0.6, 0.2, 3.1, -2.2]).view(1, 5, 1, 1)
    do1 = torch.ones(1, 1, 1, 1)
    dq, dk, dv = ref.dense_attention_backward(q1, k1, v1, do1, scale, False,
                                              round_dtype=torch.float16)
    s = k1.view(5) * scale
    p = torch.softmax(s, 0)
    o = (p * v1.view(5)).sum().half().float()
    want_ds = (p * (v1.view(5) - o) * scale).half().float()
    want_p = p.half().float()
    assert torch.equal(dk.view(5), want_ds)
    assert torch.equal(dv.view(5), want_p)
    assert torch.equal(dk.view(5), dk.view(5).half().float())
    # rounding dS before the scale gives different values here
    assert not torch.equal(want_ds, (p * (v1.view(5) - o)).half().float() * scale)


# ------------------------------------------------------------------ integer parts (bit-exact)

def test_paged_rows_resolve_every_slot():
    g = torch.Generator().manual_seed(5)
    for page in (1, 4, 16):
        pool = 13
        cache = torch.randn(pool, page, 3, 8, generator=g)
        perm = torch.randperm(pool, generator=g).to(torch.int32)
        n = min(pool * page, 5 * page + page // 2 + 1)
        rows = ref.paged_rows(cache, perm, n)
        for pos in range(n):
            assert torch.equal(rows[pos], cache[int(perm[pos // page]), pos % page])


def test_paged_visible_matches_enumeration():
    rng = np.random.default_rng(6)
    for _ in range(40):
        ql = int(rng.integers(0, 9))
        pf = int(rng.integers(0, 12))
        sl = pf + ql + int(rng.integers(-2, 3))
        sl = max(sl, 0)
        causal = bool(rng.integers(0, 2))
        wq = int(rng.integers(-1, 5))
        wk = int(rng.integers(-1, 5))
        vis = ref.paged_visible(ql, sl, pf, causal, wq, wk)
        for t in range(ql):
            for n in range(sl):
                exp = (n <= pf + t) if causal else True
                if causal and wq > 0:
                    exp = exp and (t < n + wq)
                if causal and wk > 0:
                    exp = exp and (n < t + wk)
                assert bool(vis[t, n]) == exp


def test_paged_prefill_equals_dense_causal_when_prefix_is_history():
    # seq_len = prefix + q_len makes the prefix-anchored mask bottom-right
    # aligned, i.e. the dense causal convention (tests/test_gqa_paged.py:150-219).
    g = torch.Generator().manual_seed(7)
    page, Hq, Hkv, D = 4, 6, 2, 8
    q_len, total = 5, 13
    k = torch.randn(1, total, Hkv, D, generator=g)
    v = torch.randn(1, total, Hkv, D, generator=g)
    q = torch.randn(1, q_len, Hq, D, generator=g)
    npg = -(-total // page)
    perm = torch.randperm(npg + 3, generator=g)
    kc = torch.full((npg + 3, page, Hkv, D), float("nan"))
    vc = kc.clone()
    for pos in range(total):
        kc[perm[pos // page], pos % page] = k[0, pos]
        vc[perm[pos // page], pos % page] = v[0, pos]
    bt = perm[:npg].to(torch.int32).unsqueeze(0)
    out, lse = ref.paged_attention(q[0], kc, vc, bt, [total], [0, q_len], [total - q_len],
                                   0.3, causal=True)
    d_out, d_lse = ref.dense_attention(q, k, v, 0.3, causal=True)
    torch.testing.assert_close(out, d_out[0], atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(lse, d_lse[0], atol=1e-6, rtol=1e-6)


def test_decode_equals_paged_single_token():
    g = torch.Generator().manual_seed(8)
    kc = torch.randn(9, 4, 2, 8, generator=g)
    vc = torch.randn(9, 4, 2, 8, generator=g)
    bt = torch.randperm(9, generator=g).to(torch.int32).view(3, 3)
    seq = [3, 12, 7]
    q = torch.randn(3, 4, 8, generator=g)
    out, lse = ref.decode_attention(q, kc, vc, bt, seq, 0.5)
    for b in range(3):
        o, l = ref.paged_attention(q[b:b + 1], kc, vc, bt[b:b + 1], [seq[b]], [0, 1],
                                   [seq[b] - 1], 0.5, causal=True)
        torch.testing.assert_close(out[b], o[0], atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(lse[b], l[:, 0], atol=1e-6, rtol=1e-6)


def test_merge_of_split_partials_equals_unsplit():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 1, 3, 16, generator=g, dtype=torch.float64)
    k = torch.randn(1, 50, 3, 16, generator=g, dtype=torch.float64)
    v = torch.randn(1, 50, 3, 16, generator=g, dtype=torch.float64)
    full_o, full_l = ref.dense_attention(q, k, v, 0.25, False, dtype=torch.float64)
    cuts = [0, 7, 8, 31, 50]
    outs, lses = [], []
    for a, b in zip(cuts[:-1], cuts[1:]):
        o, l = ref.dense_attention(q, k[:, a:b], v[:, a:b], 0.25, False, dtype=torch.float64)
        outs.append(o)
        lses.append(l.transpose(1, 2))  # [B, Sq, H]
    mo, ml = ref.merge_partials(torch.stack(outs), torch.stack(lses))
    torch.testing.assert_close(mo, full_o, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(ml, full_l.transpose(1, 2), atol=1e-12, rtol=1e-12)
    # an empty partial (lse = -inf) does not change the merge
    mo2, _ = ref.merge_partials(torch.cat([torch.stack(outs), torch.zeros_like(outs[0])[None]]),
                                torch.cat([torch.stack(lses), torch.full_like(lses[0], -math.inf)[None]]))
    torch.testing.assert_close(mo2, full_o, atol=1e-12, rtol=1e-12)


def test_pair_counts_match_enumeration_and_benchmark_configs():
    for sq, sk, c in ((5, 7, True), (7, 5, True), (6, 6, False), (2048, 2048, True)):
        assert ref.dense_pairs(sq, sk, c) == int(ref.dense_visible(sq, sk, c).sum())
    assert ref.dense_pairs(2048, 2048, True) == 2_098_176
    lens = [2641, 2501, 1405, 3002, 2670, 3056, 3789, 615]
    assert ref.paged_pairs(lens, lens, [0] * 8) == 27_719_186
    pf = [1751, 3120, 3566, 3048, 244, 5664, 6907, 5746, 127, 492, 1652, 980, 5907, 6417, 6694, 2486]
    assert ref.paged_pairs([512] * 16, [p + 512 for p in pf], pf) == 30_159_360


# ------------------------------------------------------------------ planted mistakes

def test_planted_top_left_causal_mask_is_caught(gold, monkeypatch):
    def top_left(sq, sk, causal, window=(-1, -1)):
        i = torch.arange(sq).unsqueeze(1)
        j = torch.arange(sk).unsqueeze(0)
        return j <= i if causal else torch.ones(sq, sk, dtype=torch.bool)

    monkeypatch.setattr(ref, "dense_visible", top_left)
    with pytest.raises(AssertionError):
        test_dense_matches_golden(gold, "dense_c_skgt")


def test_planted_transposed_gqa_map_is_caught(gold, monkeypatch):
    def wrong_expand(k, heads):
        g = heads // k.shape[2]
        return k.repeat(1, 1, g, 1)  # head h -> kv head h % Hk (wrong)

    monkeypatch.setattr(ref, "_expand_kv", wrong_expand)
    with pytest.raises(AssertionError):
        test_paged_matches_golden(gold, "c")


def test_planted_dropped_scale_in_dk_is_caught(gold, monkeypatch):
    orig = ref.dense_attention_backward

    def no_scale_dk(*a, **kw):
        dq, dk, dv = orig(*a, **kw)
        return dq, dk / float(gold["bwd/scale"]), dv

    monkeypatch.setattr(ref, "dense_attention_backward", no_scale_dk)
    with pytest.raises(AssertionError):
        test_backward_matches_finite_differences(gold)


# ------------------------------------------------------------------ cache write (bit-exact)

def _scatter_ref(key, value, kc, vc, slots):
    """Vectorised restatement: flat [P*page] row view indexed by valid slots."""
    P, page = kc.shape[:2]
    keep = (slots >= 0) & (slots < P * page)
    kf, vf = kc.reshape(P * page, *kc.shape[2:]), vc.reshape(P * page, *vc.shape[2:])
    kf[slots[keep]] = key[keep]
    vf[slots[keep]] = value[keep]


def test_reshape_and_cache_matches_flat_scatter():
    g = torch.Generator().manual_seed(9)
    for page in (1, 4, 16):
        P, T, Hkv, D = 7, 11, 3, 8
        key, value = torch.randn(T, Hkv, D, generator=g), torch.randn(T, Hkv, D, generator=g)
        slots = torch.randperm(P * page + 4, generator=g)[:T] - 2  # some < 0, some >= P*page
        a = [torch.full((P, page, Hkv, D), -7.0) for _ in range(2)]
        b = [x.clone() for x in a]
        ref.reshape_and_cache(key, value, a[0], a[1], slots)
        _scatter_ref(key, value, b[0], b[1], slots)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        written = ((slots >= 0) & (slots < P * page)).sum().item()
        assert (a[0] != -7.0).all(-1).all(-1).sum().item() == written


def test_reshape_and_cache_round_trips_through_paged_rows():
    """Writer and reader agree: slots from a block table, read back in order."""
    g = torch.Generator().manual_seed(10)
    for page in (1, 16):
        P, Hkv, D = 9, 2, 8
        n = min(37, P * page)
        key, value = torch.randn(n, Hkv, D, generator=g), torch.randn(n, Hkv, D, generator=g)
        bt = torch.randperm(P, generator=g).to(torch.int32)
        pos = torch.arange(n)
        slots = bt[pos // page].long() * page + pos % page
        kc = torch.zeros(P, page, Hkv, D)
        vc = torch.zeros(P, page, Hkv, D)
        ref.reshape_and_cache(key, value, kc, vc, slots)
        assert torch.equal(ref.paged_rows(kc, bt, n), key)
        assert torch.equal(ref.paged_rows(vc, bt, n), value)


def test_planted_transposed_page_slot_is_caught(monkeypatch):
    """A writer that swaps page and slot fails the round trip above."""
    def bad(key, value, k_cache, v_cache, slot_mapping):
        P, page = k_cache.shape[0], k_cache.shape[1]
        for t in range(key.shape[0]):
            s = int(slot_mapping[t])
            if 0 <= s < P * page:
                k_cache[s % P, s // P] = key[t]
                v_cache[s % P, s // P] = value[t]
    monkeypatch.setattr(ref, "reshape_and_cache", bad)
    with pytest.raises(AssertionError):
        test_reshape_and_cache_round_trips_through_paged_rows()


# ------------------------------------------------------------------ dense sliding window

def test_dense_window_matches_enumeration():
    """FlashAttention-2 window_size semantics, pair by pair."""
    rng = np.random.default_rng(11)
    for _ in range(60):
        sq, sk = int(rng.integers(1, 9)), int(rng.integers(1, 9))
        left, right = int(rng.integers(-1, 5)), int(rng.integers(-1, 5))
        causal = bool(rng.integers(0, 2))
        vis = ref.dense_visible(sq, sk, causal, (left, right))
        off = sk - sq
        r = 0 if causal else right
        for i in range(sq):
            for j in range(sk):
                exp = (r < 0 or j <= i + off + r) and (left < 0 or j >= i + off - left)
                assert bool(vis[i, j]) == exp, (sq, sk, left, right, causal, i, j)


def test_dense_window_closed_forms():
    g = torch.Generator().manual_seed(12)
    q, k, v = (torch.randn(1, 9, 2, 8, generator=g, dtype=torch.float64) for _ in range(3))
    # window (0, 0) with Sq == Sk: query i sees key i only -> out = v[i], lse = scaled score.
    out, lse = ref.dense_attention(q, k, v, causal=False, window=(0, 0), dtype=torch.float64)
    assert torch.equal(out, v)
    s = (q * k).sum(-1).transpose(1, 2) / math.sqrt(8)
    assert torch.allclose(lse, s, atol=1e-12)
    # unbounded window = plain attention; causal ignores the right bound.
    a, _ = ref.dense_attention(q, k, v, causal=True, window=(-1, 5), dtype=torch.float64)
    b, _ = ref.dense_attention(q, k, v, causal=True, dtype=torch.float64)
    assert torch.equal(a, b)
    # left window >= Sk changes nothing.
    a, _ = ref.dense_attention(q, k, v, causal=True, window=(9, -1), dtype=torch.float64)
    assert torch.equal(a, b)


def test_dense_window_backward_matches_autograd():
    g = torch.Generator().manual_seed(13)
    q, k, v, do = (torch.randn(1, 7, 2, 4, generator=g, dtype=torch.float64) for _ in range(4))
    for causal, window in ((True, (2, -1)), (False, (1, 2)), (False, (-1, 0))):
        qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
        out, _ = ref.dense_attention(qa, ka, va, causal=causal, window=window, dtype=torch.float64)
        out.backward(do)
        dq, dk, dv = ref.dense_attention_backward(q, k, v, do, causal=causal, window=window,
                                                  dtype=torch.float64)
        for got, want in ((dq, qa.grad), (dk, ka.grad), (dv, va.grad)):
            assert torch.allclose(got, want, atol=1e-10)
