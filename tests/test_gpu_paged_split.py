"""GPU parity: split-KV paged prefill (fa_paged_prefill_splitkv) vs the oracle.

Each case forces a split count through paged_forward_splits and compares
with the CPU oracle at the bar of the unsplit path (outputs atol 2e-3 /
rtol 1e-2, LSE within 1e-3).  Cases cover splits that hold no keys of a
sequence, empty sequences, windows, GQA, every head_dim and bf16, and the
automatic choice for a long-prefix, few-token batch.
"""
import ctypes

import pytest
import torch

from helpers import assert_close, assert_lse, rel_l2
from oracle import attention_ref as ref
from test_gpu_paged import make_case
from tilelang_fa_v100 import _lib
from tilelang_fa_v100._paged_adapter import paged_forward_splits

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def run_split(c, num_splits, causal=True, wq=-1, wk=-1):
    Hkv = c["k_cache"].shape[2]
    out, lse = paged_forward_splits(
        c["q"].to(DEV), c["k_cache"].to(DEV), c["v_cache"].to(DEV), c["block_table"].to(DEV),
        c["seq_lens"].to(DEV), c["query_start_loc"].to(DEV), c["prefix_kv_lens"].to(DEV),
        block_size=c["page"], num_kv_heads=Hkv, causal=causal,
        sliding_window_q=wq, sliding_window_k=wk, num_splits=num_splits)
    r_out, r_lse = ref.paged_attention(
        c["q"], c["k_cache"], c["v_cache"], c["block_table"], c["seq_lens"],
        c["query_start_loc"], c["prefix_kv_lens"], causal=causal, window_q=wq, window_k=wk)
    assert_close(out, r_out)
    assert_lse(lse, r_lse)
    assert rel_l2(out, r_out) < 1e-2
    return out, lse


SPLIT_CASES = [
    # (q_lens, seq_lens, prefixes, Hq, Hkv, D, page, dtype, causal, splits)
    ([64], [3000], [2936], 32, 8, 128, 16, torch.float16, True, 2),
    ([64], [3000], [2936], 32, 8, 128, 16, torch.float16, True, 7),
    ([17, 0, 40], [900, 5, 2100], [883, 5, 2060], 16, 4, 128, 32, torch.bfloat16, True, 3),
    ([33, 20], [1500, 20], [1467, 0], 8, 8, 64, 16, torch.float16, True, 4),   # split past 20 keys
    ([50], [1200], [1150], 8, 1, 256, 64, torch.float16, True, 5),
    ([30, 30], [700, 400], [0, 0], 8, 2, 128, 16, torch.float16, False, 6),    # non-causal
    ([128], [4096], [3968], 64, 8, 128, 16, torch.bfloat16, True, 16),         # C5-like head count
    ([40], [1500], [1460], 4, 1, 512, 16, torch.float16, True, 3),             # D = 512
]


def _ids(c):
    ql, sl, pf, Hq, Hkv, D, page, dt, causal, ns = c
    return f"q{sum(ql)}-kv{max(sl)}-H{Hq}/{Hkv}-D{D}-p{page}-{str(dt)[6:]}-{'c' if causal else 'nc'}-s{ns}"


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[_ids(c) for c in SPLIT_CASES])
def test_split_kv_matches_oracle(case):
    ql, sl, pf, Hq, Hkv, D, page, dt, causal, ns = case
    c = make_case(11, ql, sl, pf, Hq, Hkv, D, page=page, dtype=dt)
    run_split(c, ns, causal=causal)


def test_split_kv_with_sliding_window():
    c = make_case(12, [48], [2000], [1952], 16, 4, 128, page=16)
    run_split(c, 4, causal=True, wq=300, wk=40)


def test_split_kv_agrees_with_unsplit_path():
    c = make_case(13, [96, 31], [2500, 1800], [2404, 1769], 32, 8, 128, page=16)
    one, lse1 = run_split(c, 1)
    many, lsem = run_split(c, 9)
    assert (one.float() - many.float()).abs().max().item() < 2e-3
    assert (lse1 - lsem).abs().max().item() < 1e-3


def test_automatic_split_for_long_prefix_few_tokens():
    # 2 sequences x 64 new tokens after 6k-key prefixes: 8 KV heads give 8
    # workgroups unsplit, so the library splits.
    c = make_case(14, [64, 64], [6000, 6100], [5936, 6036], 32, 8, 128, page=16)
    a = _lib.PagedArgs()
    a.num_tokens, a.batch, a.num_heads, a.num_kv_heads, a.head_dim = 128, 2, 32, 8, 128
    a.max_blocks, a.page_size, a.num_pages = c["block_table"].shape[1], 16, 1000
    for n in ("q", "k_cache", "v_cache", "out", "block_table", "seq_lens", "query_start_loc",
              "prefix_kv_lens"):
        setattr(a, n, 0x1000)
    a.q_stride[:] = (32 * 128, 128)
    a.o_stride[:] = (32 * 128, 128)
    a.k_stride[:] = (16 * 8 * 128, 8 * 128, 128)
    a.v_stride[:] = (16 * 8 * 128, 8 * 128, 128)
    a.block_table_stride = a.max_blocks
    assert _lib.load().fa_paged_prefill_num_splits(ctypes.byref(a)) > 1
    run_split(c, None)
