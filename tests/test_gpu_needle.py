"""Bit-exact masking and page resolution ("needle" inputs), on the GPU.

Scores rise (or fall) with the key index by 128 in the kernels' base-2
domain (helpers.needle_*), so each row's softmax is one-hot on its last (or
first) visible key and the output must equal that key's V row exactly: an
off-by-one at the causal edge, the seq_len boundary, a window edge or a
split-KV range boundary, or a wrongly resolved page, returns another row.
The expected row comes from the oracle's visibility rules and page
resolution (oracle.attention_ref.dense_visible / paged_visible /
paged_rows, following _kernels_forward.py:135-144 and
_kernels_paged.py:265-308,450-451).  Paged caches hold a decoy key in every
slot past seq_len of a sequence's last page (continuing the rising scores,
so a read of slot seq_len would win the softmax) and NaN in pages no
sequence owns; block-table padding is -1.
"""
import math

import pytest
import torch

import tilelang_fa_v100 as fa
from helpers import (assert_equal_rows, build_paged, needle_expected, needle_keys,
                     needle_query, needle_scale, standard_forward_batch)
from oracle import attention_ref as ref
from tilelang_fa_v100._paged_adapter import paged_forward_splits

DEV = "cuda:0"
F16, BF16 = torch.float16, torch.bfloat16
SIGNS = [1, -1]


def _sid(s):
    return "rise" if s > 0 else "fall"


# --------------------------------------------------------------------- oracle side (CPU)

def test_needle_inputs_make_the_oracle_one_hot():
    """The construction itself, checked on the oracle: its fp32 output equals
    the picked V rows exactly, for both score directions."""
    g = torch.Generator().manual_seed(0)
    Sq, Sk, D = 40, 90, 64
    scale = needle_scale()
    for sign in SIGNS:
        q = needle_query(Sq, 2, D, sign).unsqueeze(0)
        k = needle_keys(g, Sk, 2, D).unsqueeze(0)
        v = torch.randn(1, Sk, 2, D, generator=g).half()
        out, _ = ref.dense_attention(q, k, v, scale=scale, causal=True)
        want = needle_expected(v[0], ref.dense_visible(Sq, Sk, True), sign)
        assert_equal_rows(out[0].half(), want)


# --------------------------------------------------------------------- dense

DENSE = [
    # (B, Sq, Sk, H, Hk, D, causal, window, dtype)
    (2, 300, 300, 4, 2, 128, True, (-1, -1), F16),
    (1, 257, 1000, 4, 2, 128, True, (-1, -1), BF16),    # Sk > Sq
    (1, 1000, 257, 2, 2, 128, True, (-1, -1), F16),     # Sq > Sk: rows without keys
    (1, 700, 700, 2, 2, 128, True, (130, -1), F16),     # causal + left window
    (1, 300, 520, 2, 2, 128, False, (64, 32), BF16),    # two-sided band
    (1, 520, 300, 2, 2, 128, False, (-1, 0), F16),      # right edge only
    (1, 77, 77, 2, 1, 128, False, (-1, -1), F16),       # full attention
    (1, 600, 600, 4, 4, 64, True, (-1, -1), F16),       # D = 64
    (1, 333, 400, 2, 1, 64, False, (40, 17), BF16),
    (1, 129, 129, 2, 2, 256, True, (-1, -1), BF16),     # D = 256
    (1, 300, 400, 2, 2, 256, False, (50, 70), F16),
    (2, 40, 1003, 4, 2, 256, True, (-1, -1), F16),
    (1, 1, 1, 2, 2, 128, True, (-1, -1), F16),          # single query and key
    (1, 64, 1, 2, 1, 128, False, (-1, -1), F16),        # single key
    (1, 64, 1, 2, 2, 256, False, (-1, -1), BF16),
]


def _dids(c):
    B, Sq, Sk, H, Hk, D, causal, w, dt = c
    return f"{Sq}x{Sk}-H{H}/{Hk}-D{D}-{'c' if causal else 'nc'}-w{w[0]}_{w[1]}-{str(dt)[6:]}"


DENSE_RUNS = [(c, "as_given") for c in DENSE] + [(c, "row_tiles") for c in DENSE if c[5] in (64, 128)]


@pytest.mark.gpu
@pytest.mark.parametrize("sign", SIGNS, ids=_sid)
@pytest.mark.parametrize("case,grid", DENSE_RUNS, ids=[f"{_dids(c)}-{g}" for c, g in DENSE_RUNS])
def test_dense_mask_edges_bit_exact(case, grid, sign):
    """grid: the case as listed (at head_dim 64 / 128 these small batches
    leave the row-tile cores too few workgroups, so the key-split kernel runs
    them), or with its batch repeated until the row-tile cores run it."""
    B, Sq, Sk, H, Hk, D, causal, window, dt = case
    if grid == "row_tiles":
        B = standard_forward_batch(B, H, Sq, D)
    g = torch.Generator().manual_seed(11)
    q = needle_query(B * Sq, H, D, sign, dt).view(B, Sq, H, D)
    k = torch.stack([needle_keys(g, Sk, Hk, D, dt) for _ in range(B)])
    v = torch.randn(B, Sk, Hk, D, generator=g).to(dt)
    out = fa.tilelang_flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), causal=causal,
                                      window_size=window, softmax_scale=needle_scale())
    vis = ref.dense_visible(Sq, Sk, causal, window)
    ve = ref._expand_kv(v, H)
    for b in sorted({0, 1, B - 1} & set(range(B))):
        assert_equal_rows(out[b], needle_expected(ve[b], vis, sign), what=f"batch {b}")


# --------------------------------------------------------------------- paged prefill

def needle_paged(seed, q_lens, seq_lens, prefixes, Hq, Hkv, D, page, dtype, sign):
    """Paged case with needle keys; slots past seq_len in a last page hold
    decoys (the key pattern continues there)."""
    g = torch.Generator().manual_seed(seed)
    alloc = [max(page * math.ceil(n / page), 1) for n in seq_lens]
    ks = [needle_keys(g, a, Hkv, D, dtype) for a in alloc]
    vs = [torch.randn(a, Hkv, D, generator=g).to(dtype) for a in alloc]
    kc, vc, bt = build_paged(g, ks, vs, page, dtype=dtype)
    q = needle_query(sum(q_lens), Hq, D, sign, dtype)
    qsl = torch.tensor([0] + torch.tensor(q_lens).cumsum(0).tolist(), dtype=torch.int32)
    return dict(q=q, k_cache=kc, v_cache=vc, block_table=bt,
                seq_lens=torch.tensor(seq_lens, dtype=torch.int32), query_start_loc=qsl,
                prefix_kv_lens=torch.tensor(prefixes, dtype=torch.int32))


def paged_expected(c, sign, causal=True, wq=-1, wk=-1):
    """Picked V rows per token and head, from the oracle's page resolution
    (paged_rows) and mask (paged_visible)."""
    T, Hq, D = c["q"].shape
    want = torch.zeros(T, Hq, D, dtype=c["q"].dtype)
    qsl = c["query_start_loc"]
    for b in range(c["block_table"].shape[0]):
        s0, s1 = int(qsl[b]), int(qsl[b + 1])
        n = int(c["seq_lens"][b])
        vrows = ref._expand_kv(ref.paged_rows(c["v_cache"], c["block_table"][b], n)
                               .unsqueeze(0), Hq)[0]
        vis = ref.paged_visible(s1 - s0, n, int(c["prefix_kv_lens"][b]), causal, wq, wk)
        want[s0:s1] = needle_expected(vrows, vis, sign)
    return want


def run_paged(c, splits=None, causal=True, wq=-1, wk=-1):
    args = [c[n].to(DEV) for n in ("q", "k_cache", "v_cache", "block_table", "seq_lens",
                                     "query_start_loc", "prefix_kv_lens")]
    out, _ = paged_forward_splits(*args, block_size=c["k_cache"].shape[1],
                                  softmax_scale=needle_scale(), causal=causal,
                                  sliding_window_q=wq, sliding_window_k=wk,
                                  num_splits=splits)
    return out


PAGED = [
    # (q_lens, seq_lens, prefixes, Hq, Hkv, D, page, dtype)
    # chunked prefill after a prefix (C5 shape, fewer sequences)
    ([512, 512, 512], [1751 + 512, 244 + 512, 127 + 512], [1751, 244, 127], 64, 8, 128, 16, BF16),
    # pure prefill with ragged lengths (C3 shape)
    ([615, 1405, 33], [615, 1405, 33], [0, 0, 0], 32, 8, 128, 16, F16),
    # seq_len shorter than prefix + q_len: the seq_len bound cuts rows
    ([100, 64], [130, 20], [60, 0], 8, 2, 128, 16, F16),
    # page sizes other than 16 (one-phase core for pages < 16)
    ([77, 200], [300, 200], [223, 0], 8, 1, 128, 1, F16),
    ([77, 200], [300, 211], [223, 11], 8, 2, 128, 8, BF16),
    ([130], [1000], [870], 16, 2, 128, 128, F16),
    # head_dim 64 / 256 / 512
    ([90, 300], [400, 300], [310, 0], 8, 2, 64, 16, F16),
    ([90, 300], [400, 301], [310, 1], 8, 1, 256, 16, BF16),
    ([40, 70], [170, 70], [130, 0], 4, 1, 512, 16, F16),
    # an empty sequence and a sequence without keys
    ([0, 50, 20], [30, 80, 0], [30, 30, 0], 4, 1, 128, 16, F16),
]


def _pids(c):
    q_lens, seq_lens, _, Hq, Hkv, D, page, dt = c
    return f"B{len(q_lens)}-H{Hq}/{Hkv}-D{D}-p{page}-{str(dt)[6:]}"


@pytest.mark.gpu
@pytest.mark.parametrize("sign", SIGNS, ids=_sid)
@pytest.mark.parametrize("case", PAGED, ids=[_pids(c) for c in PAGED])
def test_paged_mask_and_pages_bit_exact(case, sign):
    c = needle_paged(12, *case, sign=sign)
    assert_equal_rows(run_paged(c, splits=1), paged_expected(c, sign))


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [2, 3, 7, 16])
@pytest.mark.parametrize("sign", SIGNS, ids=_sid)
def test_paged_split_kv_range_edges_bit_exact(splits, sign):
    # Long prefixes and few new tokens: the key ranges of the splits end
    # inside sequences; each range's partial is one-hot on its own edge key
    # and the merge must select exactly the row's needle.
    c = needle_paged(13, [64, 17, 128], [4000 + 64, 1234 + 17, 2500], [4000, 1234, 2372],
                     16, 2, 128, 16, F16, sign)
    assert_equal_rows(run_paged(c, splits=splits), paged_expected(c, sign))


WINDOWS = [(1, -1), (37, -1), (-1, 1), (-1, 29), (40, 300), (513, 64)]


@pytest.mark.gpu
@pytest.mark.parametrize("sign", SIGNS, ids=_sid)
@pytest.mark.parametrize("window", WINDOWS, ids=[f"wq{w[0]}_wk{w[1]}" for w in WINDOWS])
def test_paged_window_edges_bit_exact(window, sign):
    wq, wk = window
    c = needle_paged(14, [300, 96], [300, 500], [0, 404], 8, 2, 128, 16, F16, sign)
    want = paged_expected(c, sign, wq=wq, wk=wk)
    assert_equal_rows(run_paged(c, splits=1, wq=wq, wk=wk), want, what="unsplit")
    assert_equal_rows(run_paged(c, splits=3, wq=wq, wk=wk), want, what="3 splits")


@pytest.mark.gpu
@pytest.mark.parametrize("sign", SIGNS, ids=_sid)
def test_paged_non_causal_bit_exact(sign):
    c = needle_paged(15, [100, 40], [333, 1], [0, 0], 8, 2, 128, 16, BF16, sign)
    assert_equal_rows(run_paged(c, splits=1, causal=False),
                      paged_expected(c, sign, causal=False))


# --------------------------------------------------------------------- decode

DECODE = [
    # (seq_lens, Hq, Hkv, D, page, dtype, max_blocks_extra)
    ([1, 15, 16, 17, 1000, 4097], 32, 8, 128, 16, F16, 0),
    ([8191, 33, 2049], 8, 1, 128, 16, BF16, 0),
    ([32768, 20000, 513], 32, 8, 128, 16, F16, 0),     # long: several splits per sequence
    ([300, 5000], 16, 2, 128, 16, F16, 700),           # block table wider than needed
    ([129, 4000], 8, 2, 64, 16, F16, 0),               # head_dim 64 / 256 / 512
    ([129, 4000], 8, 2, 256, 16, BF16, 0),
    ([129, 1500], 4, 1, 512, 16, F16, 0),
    ([100, 700], 8, 2, 128, 1, F16, 0),                # page sizes other than 16
    ([100, 700], 8, 2, 128, 8, F16, 0),
    ([100, 700], 8, 2, 128, 64, BF16, 0),
    ([0, 37], 8, 2, 128, 16, F16, 0),                  # an empty sequence
    # pages under 16 keys on the streaming kernel (one page per DMA instruction)
    ([1, 3, 5, 17, 700, 3000], 8, 2, 128, 4, F16, 0),
    ([129, 4000], 8, 2, 64, 8, BF16, 0),
    ([7, 2500], 8, 2, 256, 2, F16, 0),
    ([1, 1500], 4, 1, 512, 1, F16, 0),
]


def _decids(c):
    lens, Hq, Hkv, D, page, dt, extra = c
    return f"n{max(lens)}-H{Hq}/{Hkv}-D{D}-p{page}-{str(dt)[6:]}" + (f"-w{extra}" if extra else "")


@pytest.mark.gpu
@pytest.mark.parametrize("sign", SIGNS, ids=_sid)
@pytest.mark.parametrize("case", DECODE, ids=[_decids(c) for c in DECODE])
def test_decode_bounds_and_pages_bit_exact(case, sign):
    lens, Hq, Hkv, D, page, dt, extra = case
    c = needle_paged(16, [1] * len(lens), lens, [0] * len(lens), Hq, Hkv, D, page, dt, sign)
    bt = c["block_table"]
    if extra:
        bt = torch.cat([bt, torch.full((bt.shape[0], extra), -1, dtype=bt.dtype)], 1)
    out = fa.tilelang_decode_forward(c["q"].to(DEV), c["k_cache"].to(DEV), c["v_cache"].to(DEV),
                                     bt.to(DEV), c["seq_lens"].to(DEV), block_size=page,
                                     softmax_scale=needle_scale())
    c["block_table"] = bt
    want = paged_expected(c, sign, causal=False)
    assert_equal_rows(out, want)
