"""GPU parity: paged varlen prefill (tilelang_paged_forward) vs the CPU oracle.

Caches are built with scattered pages (seeded permutation), NaN in every
slot no visible key occupies and -1 block-table padding; the oracle gathers
the same pages.  Outputs within atol 2e-3 / rtol 1e-2, LSE within 1e-3.
"""
import pytest
import torch

import tilelang_fa_v100 as fa
from helpers import assert_close, assert_lse, build_paged, randn, rel_l2
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def make_case(seed, q_lens, seq_lens, prefixes, Hq, Hkv, D, page=16, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    ks = [randn(g, n, Hkv, D, dtype=dtype) for n in seq_lens]
    vs = [randn(g, n, Hkv, D, dtype=dtype) for n in seq_lens]
    kc, vc, bt = build_paged(g, ks, vs, page, dtype=dtype)
    T = sum(q_lens)
    q = randn(g, T, Hq, D, dtype=dtype)
    qsl = torch.tensor([0] + list(torch.tensor(q_lens).cumsum(0).tolist()), dtype=torch.int32)
    return dict(q=q, k_cache=kc, v_cache=vc, block_table=bt,
                seq_lens=torch.tensor(seq_lens, dtype=torch.int32), query_start_loc=qsl,
                prefix_kv_lens=torch.tensor(prefixes, dtype=torch.int32), page=page)


def run_both(c, causal=True, wq=-1, wk=-1, scale=None):
    Hkv = c["k_cache"].shape[2]
    out, lse = fa.tilelang_paged_forward(
        c["q"].to(DEV), c["k_cache"].to(DEV), c["v_cache"].to(DEV), c["block_table"].to(DEV),
        c["seq_lens"].to(DEV), c["query_start_loc"].to(DEV), c["prefix_kv_lens"].to(DEV),
        block_size=c["page"], num_kv_heads=Hkv, softmax_scale=scale, causal=causal,
        sliding_window_q=wq, sliding_window_k=wk)
    r_out, r_lse = ref.paged_attention(
        c["q"], c["k_cache"], c["v_cache"], c["block_table"], c["seq_lens"],
        c["query_start_loc"], c["prefix_kv_lens"], scale=scale, causal=causal,
        window_q=wq, window_k=wk)
    return out, lse, r_out, r_lse


def check(c, **kw):
    out, lse, r_out, r_lse = run_both(c, **kw)
    assert_close(out, r_out)
    assert_lse(lse, r_lse)
    assert rel_l2(out, r_out) < 1e-2


def test_c3_config_exact():
    # 8 seqs, lens U[512,4096] from seed 0, 32/8 heads, D=128, fp16.
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 4097, (8,), generator=g).tolist()
    assert lens == [2641, 2501, 1405, 3002, 2670, 3056, 3789, 615]
    c = make_case(0, lens, lens, [0] * 8, 32, 8, 128)
    check(c)


@pytest.mark.parametrize("D", [128, 256])
def test_c5_like_chunked_prefill_bf16(D):
    # BASELINE configs[4] shape, fewer sequences: 512 new tokens after a prefix.
    pf = [1751, 3120, 244, 127]
    c = make_case(1, [512] * 4, [p + 512 for p in pf], pf, 64, 8, D, dtype=torch.bfloat16)
    check(c)


# Reference tests/test_gqa_paged.py shapes (pure prefill and chunked).
GQA_ROWS = [
    # (B, Hq, Hkv, q_len, total, D, causal)
    (1, 16, 2, 64, 64, 128, True), (1, 16, 2, 256, 256, 128, True),
    (1, 24, 4, 64, 64, 128, True), (1, 24, 4, 256, 256, 128, True),
    (1, 8, 1, 64, 64, 256, True), (1, 8, 1, 128, 128, 256, True),
    (1, 4, 1, 64, 64, 128, True), (2, 16, 2, 128, 128, 128, True),
    (1, 8, 1, 64, 64, 256, False),
    (1, 16, 2, 32, 128, 128, True), (1, 24, 4, 32, 128, 128, True),
    (1, 8, 1, 16, 64, 256, True),
    (1, 8, 1, 64, 64, 512, True), (1, 4, 1, 32, 160, 512, True),   # D = 512 (two O passes)
    (1, 8, 2, 64, 64, 512, False),
]


@pytest.mark.parametrize("row", GQA_ROWS, ids=[f"B{r[0]}-H{r[1]}/{r[2]}-q{r[3]}-kv{r[4]}-D{r[5]}-{'c' if r[6] else 'nc'}" for r in GQA_ROWS])
def test_reference_gqa_shapes(row):
    B, Hq, Hkv, ql, tot, D, causal = row
    c = make_case(42, [ql] * B, [tot] * B, [tot - ql] * B, Hq, Hkv, D)
    check(c, causal=causal)


def test_mixed_batch_noncausal_and_empty_sequences():
    c = make_case(3, [37, 0, 300, 1, 64], [90, 0, 300, 5, 1000], [53, 0, 0, 4, 936], 8, 2, 128)
    check(c, causal=False)
    check(c, causal=True)


@pytest.mark.parametrize("D", [128, 256])
def test_sliding_windows(D):
    c = make_case(4, [200, 77], [500, 77], [300, 0], 8, 4, D)
    for wq, wk in ((64, -1), (-1, 33), (100, 50), (1, -1)):
        check(c, causal=True, wq=wq, wk=wk)


@pytest.mark.parametrize("page,D", [(32, 64), (1, 128), (32, 128), (128, 128), (64, 256), (16, 512)])
def test_page_sizes_and_head_dims(page, D):
    c = make_case(5, [150, 260], [400, 260], [250, 0], 4, 2, D, page=page)
    check(c, causal=True)


def test_custom_scale_and_out_tensor_is_reused():
    c = make_case(6, [100, 50], [100, 170], [0, 120], 8, 8, 128)
    out = torch.empty(c["q"].shape, dtype=c["q"].dtype, device=DEV)
    res, lse = fa.tilelang_paged_forward(
        c["q"].to(DEV), c["k_cache"].to(DEV), c["v_cache"].to(DEV), c["block_table"].to(DEV),
        c["seq_lens"].to(DEV), c["query_start_loc"].to(DEV), c["prefix_kv_lens"].to(DEV),
        out=out, softmax_scale=0.02)
    assert res is out
    r_out, r_lse = ref.paged_attention(c["q"], c["k_cache"], c["v_cache"], c["block_table"],
                                       c["seq_lens"], c["query_start_loc"],
                                       c["prefix_kv_lens"], scale=0.02)
    assert_close(out, r_out)
    assert_lse(lse, r_lse)


def test_long_odd_length_d256():
    # reference tests/test_bounds.py: M = N = 19665, D = 256, Hq = 2, Hkv = 1, causal.
    n = 19665
    c = make_case(7, [n], [n], [0], 2, 1, 256)
    out, lse = fa.tilelang_paged_forward(
        c["q"].to(DEV), c["k_cache"].to(DEV), c["v_cache"].to(DEV), c["block_table"].to(DEV),
        c["seq_lens"].to(DEV), c["query_start_loc"].to(DEV), c["prefix_kv_lens"].to(DEV))
    out = out.cpu()
    assert torch.isfinite(out.float()).all()
    rows = torch.tensor([0, 1, 2, 127, 128, 1000, 9832, 19000] + list(range(n - 64, n)))
    k = ref.paged_rows(c["k_cache"], c["block_table"][0], n)
    v = ref.paged_rows(c["v_cache"], c["block_table"][0], n)
    vis = torch.arange(n).unsqueeze(0) <= rows.unsqueeze(1)  # causal, prefix 0
    r_out, r_lse = ref.masked_softmax_attention(c["q"][rows], k.repeat_interleave(2, 1),
                                                v.repeat_interleave(2, 1), vis, 256 ** -0.5)
    assert_close(out[rows], r_out)
    assert_lse(lse.cpu()[:, rows], r_lse)


@pytest.mark.parametrize("D", [128, 256])
def test_v_cache_with_its_own_token_stride(D):
    # V cache a column slice of a wider allocation: its token and page strides
    # differ from K's, and the two-phase cores DMA K and V rows each with
    # their own row stride.
    c = make_case(9, [300, 40], [700, 40], [400, 0], 8, 2, D)
    kc, vc = c["k_cache"], c["v_cache"]
    wide = torch.zeros(*vc.shape[:-1], D + 64, dtype=vc.dtype)
    wide[..., :D] = vc
    vd = wide.to(DEV)[..., :D]
    assert vd.stride(1) != kc.stride(1)
    out, lse = fa.tilelang_paged_forward(
        c["q"].to(DEV), kc.to(DEV), vd, c["block_table"].to(DEV), c["seq_lens"].to(DEV),
        c["query_start_loc"].to(DEV), c["prefix_kv_lens"].to(DEV), block_size=c["page"],
        num_kv_heads=2, causal=True)
    r_out, r_lse = ref.paged_attention(c["q"], kc, vc, c["block_table"], c["seq_lens"],
                                       c["query_start_loc"], c["prefix_kv_lens"], causal=True)
    assert_close(out, r_out)
    assert_lse(lse, r_lse)
