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
                                          (512, 16, torch.float16), (512, 32, torch.bfloat16),
                                          # pages under 16 keys on the streaming kernel
                                          (128, 8, torch.float16), (128, 4, torch.bfloat16),
                                          (64, 8, torch.float16), (256, 2, torch.float16),
                                          (512, 1, torch.float16), (512, 8, torch.bfloat16),
                                          # and on the chunked kernel
                                          (64, 4, torch.float16), (128, 2, torch.float16)])
def test_head_dims_pages_dtypes(D, page, dtype):
    check(make_case(3, [900, 17, 4096], 16, 4, D, page=page, dtype=dtype))


@pytest.mark.parametrize("Hq,Hkv,page", [(32, 4, 16), (8, 8, 16), (16, 8, 64)])
def test_head_dim_512_group_sizes(Hq, Hkv, page):
    # Head_dim 512 on the streaming kernel at 8, 1 and 2 query heads per item;
    # lengths end mid-tile and inside the first tile.
    check(make_case(7, [1500, 9, 2048, 31], Hq, Hkv, 512, page=page))


def test_scale_and_public_entry_point():
    q, kc, vc, bt, sl, page = make_case(4, [333, 2048], 16, 4, 128)
    check((q, kc, vc, bt, sl, page), scale=0.3)
    out = fa.tilelang_decode_forward(q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV), sl.to(DEV))
    r_out, _ = ref.decode_attention(q, kc, vc, bt, sl)
    assert_close(out, r_out)


def test_long_context_32k():
    check(make_case(5, [32768, 32768 - 5, 20000], 32, 8, 128))


def _device_paged(lens, Hq, Hkv, D, seed):
    """Scattered-page cache built on the GPU (too large for the CPU oracle)."""
    page = 16
    npg = [(n + page - 1) // page for n in lens]
    pool = sum(npg)
    g = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn(pool, page, Hkv, D, generator=g, device=DEV).half()
    vc = torch.randn(pool, page, Hkv, D, generator=g, device=DEV).half()
    q = torch.randn(len(lens), Hq, D, generator=g, device=DEV).half()
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    bt = torch.full((len(lens), max(npg)), -1, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(npg):
        bt[b, :n] = perm[cur:cur + n]
        cur += n
    return q, kc, vc, bt.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV)


@pytest.mark.parametrize("lens_kind", ["uniform32k_b64", "skewed_b64", "uniform32k_b16", "d512_4k_b64"])
def test_long_splits_agree_with_paged_prefill(lens_kind):
    # Batches large enough for 1024- to 4096-key splits (64 x 32k keys: the
    # kernel doubles the launcher's 2048 to 4096; the skewed batch keeps
    # 2048; 16 x 32k takes 1024).  Too large for the CPU oracle, so the
    # decode output is checked against the paged prefill kernel (checked
    # against the oracle above and in test_gpu_paged.py) run as one query
    # token per sequence with prefix = len - 1: the same attention.
    D = 128
    if lens_kind == "skewed_b64":
        lens = torch.randint(1024, 32769, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    elif lens_kind == "d512_4k_b64":
        lens, D = [4096 - 7 * i for i in range(64)], 512
    else:
        lens = [32768] * (64 if lens_kind == "uniform32k_b64" else 16)
    q, kc, vc, bt, sl = _device_paged(lens, 32, 8, D, seed=11)
    out = fa.tilelang_decode_forward(q, kc, vc, bt, sl)
    B = len(lens)
    qsl = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    pfx = (sl - 1).to(torch.int32)
    ref_out, _ = fa.tilelang_paged_forward(q, kc, vc, bt, sl, qsl, pfx, causal=True)
    assert_close(out, ref_out.view(B, 32, D).float().cpu())
    assert rel_l2(out, ref_out.view(B, 32, D).float().cpu()) < 1e-2


def test_v_cache_with_its_own_token_stride():
    q, kc, vc, bt, sl, page = make_case(12, [700, 3000, 45], 32, 8, 128)
    wide = torch.zeros(*vc.shape[:-1], 192, dtype=vc.dtype)
    wide[..., :128] = vc
    vd = wide.to(DEV)[..., :128]
    assert vd.stride(1) != kc.stride(1)
    out = fa.tilelang_decode_forward(q.to(DEV), kc.to(DEV), vd, bt.to(DEV), sl.to(DEV),
                                     block_size=page)
    r_out, _ = ref.decode_attention(q, kc, vc, bt, sl)
    assert_close(out, r_out)
