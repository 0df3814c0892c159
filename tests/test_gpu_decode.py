"""GPU parity: paged split-KV decode (tilelang_decode_forward) vs the oracle.

Contexts span one partial chunk up to many chunks (the split-KV + LSE merge
path), with scattered pages, NaN sentinels in unused slots and -1 padding.
"""
import pytest
import torch

import tilelang_fa_v100 as fa
from helpers import assert_close, assert_lse, build_paged, randn, rel_l2
from oracle import attention_ref as ref
from tilelang_fa_v100._decode_adapter import decode_forward

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def make_case(seed, seq_lens, Hq, Hkv, D, page=16, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    ks = [randn(g, n, Hkv, D, dtype=dtype) for n in seq_lens]
    vs = [randn(g, n, Hkv, D, dtype=dtype) for n in seq_lens]
    kc, vc, bt = build_paged(g, ks, vs, page, dtype=dtype)
    q = randn(g, len(seq_lens), Hq, D, dtype=dtype)
    return q, kc, vc, bt, torch.tensor(seq_lens, dtype=torch.int32), page


def check(case, scale=None):
    q, kc, vc, bt, sl, page = case
    out, lse = decode_forward(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), sl.to(DEV),
                              block_size=page, softmax_scale=scale, return_lse=True)
    r_out, r_lse = ref.decode_attention(q, kc, vc, bt, sl, scale=scale)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert_close(out, r_out)
    assert_lse(lse, r_lse)
    assert rel_l2(out, r_out) < 1e-2


def test_c4_like_batch():
    # BASELINE configs[3] shape with a smaller batch: ctx U[1024, 32768], 32/8 heads, D=128.
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(1024, 32769, (6,), generator=g).tolist()
    check(make_case(0, lens, 32, 8, 128))


@pytest.mark.parametrize("lens", [[1, 2, 255, 256, 257], [511, 512, 513, 1000], [0, 3, 0]])
def test_chunk_boundaries_and_empty(lens):
    check(make_case(1, lens, 8, 2, 128))


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (12, 2), (32, 2), (64, 1), (6, 3)])
def test_group_sizes(Hq, Hkv):
    check(make_case(2, [700, 3000, 45], Hq, Hkv, 128))


@pytest.mark.parametrize("D,page,dtype", [(64, 16, torch.float16), (256, 32, torch.float16),
                                          (128, 16, torch.bfloat16), (128, 1, torch.float16),
                                          (512, 16, torch.float16), (512, 32, torch.bfloat16)])
def test_head_dims_pages_dtypes(D, page, dtype):
    check(make_case(3, [900, 17, 4096], 16, 4, D, page=page, dtype=dtype))


def test_scale_and_public_entry_point():
    q, kc, vc, bt, sl, page = make_case(4, [333, 2048], 16, 4, 128)
    check((q, kc, vc, bt, sl, page), scale=0.3)
    out = fa.tilelang_decode_forward(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), sl.to(DEV))
    r_out, _ = ref.decode_attention(q, kc, vc, bt, sl)
    assert_close(out, r_out)


def test_long_context_32k():
    check(make_case(5, [32768, 32768 - 5, 20000], 32, 8, 128))
