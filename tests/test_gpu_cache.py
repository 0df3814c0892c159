"""GPU parity: reshape_and_cache (KV-cache write) vs the CPU oracle, bit-exact.

Caches start filled with a sentinel, so a write to a wrong slot, a missed
write or a write for a padding / out-of-range slot all show up.  The
end-to-end test writes the K/V of several sequences through the kernel into
scattered pages and runs tilelang_paged_forward on the result.
"""
import pytest
import torch

import tilelang_fa_v100 as fa
from helpers import assert_close, assert_lse, randn
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("page,D,dtype", [(16, 128, torch.float16), (1, 64, torch.bfloat16),
                                          (64, 256, torch.float16), (16, 8, torch.bfloat16)])
def test_matches_oracle_bit_exact(page, D, dtype):
    g = torch.Generator().manual_seed(page + D)
    P, Hkv = 13, 4
    T = min(P * page, 150)
    key, value = randn(g, T, Hkv, D, dtype=dtype), randn(g, T, Hkv, D, dtype=dtype)
    slots = torch.randperm(P * page + 6, generator=g)[:T].long() - 3
    slots[::7] = -1  # padding tokens
    kc = torch.full((P, page, Hkv, D), 3.5, dtype=dtype)
    vc = torch.full((P, page, Hkv, D), -2.5, dtype=dtype)
    kd, vd = kc.to(DEV), vc.to(DEV)
    fa.reshape_and_cache(key.to(DEV), value.to(DEV), kd, vd, slots.to(DEV))
    ref.reshape_and_cache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), kc)
    assert torch.equal(vd.cpu(), vc)


def test_strided_key_value_and_int32_slots():
    """key / value as head slices of a fused qkv tensor (token stride 3*Hkv*D)."""
    g = torch.Generator().manual_seed(3)
    T, Hkv, D, P, page = 40, 2, 128, 8, 16
    qkv = randn(g, T, 3 * Hkv, D)
    key, value = qkv[:, Hkv:2 * Hkv], qkv[:, 2 * Hkv:]
    slots = torch.randperm(P * page, generator=g)[:T].to(torch.int32)
    kc = torch.zeros(P, page, Hkv, D, dtype=torch.float16)
    vc = torch.zeros(P, page, Hkv, D, dtype=torch.float16)
    kd, vd = kc.to(DEV), vc.to(DEV)
    qkv_d = qkv.to(DEV)
    fa.reshape_and_cache(qkv_d[:, Hkv:2 * Hkv], qkv_d[:, 2 * Hkv:], kd, vd, slots.to(DEV))
    ref.reshape_and_cache(key, value, kc, vc, slots.long())
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu(), kc) and torch.equal(vd.cpu(), vc)


def test_write_then_paged_prefill_end_to_end():
    g = torch.Generator().manual_seed(4)
    lens, Hq, Hkv, D, page = [300, 17, 129], 8, 2, 128, 16
    npages = [(n + page - 1) // page for n in lens]
    P = sum(npages) + 2
    perm = torch.randperm(P, generator=g)
    bt = torch.full((len(lens), max(npages)), -1, dtype=torch.int32)
    cur, slot_list = 0, []
    for b, n in enumerate(lens):
        bt[b, :npages[b]] = perm[cur:cur + npages[b]].to(torch.int32)
        cur += npages[b]
        pos = torch.arange(n)
        slot_list.append(bt[b, pos // page].long() * page + pos % page)
    slots = torch.cat(slot_list)
    T = sum(lens)
    key, value = randn(g, T, Hkv, D), randn(g, T, Hkv, D)
    q = randn(g, T, Hq, D)
    kd = torch.full((P, page, Hkv, D), float("nan"), dtype=torch.float16, device=DEV)
    vd = torch.full((P, page, Hkv, D), float("nan"), dtype=torch.float16, device=DEV)
    fa.reshape_and_cache(key.to(DEV), value.to(DEV), kd, vd, slots.to(DEV))
    qsl = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    sl = torch.tensor(lens, dtype=torch.int32)
    pkl = torch.zeros(len(lens), dtype=torch.int32)
    out, lse = fa.tilelang_paged_forward(q.to(DEV), kd, vd, bt.to(DEV), sl.to(DEV), qsl.to(DEV),
                                         pkl.to(DEV), block_size=page, num_kv_heads=Hkv)
    kc, vc = kd.cpu(), vd.cpu()
    r_out, r_lse = ref.paged_attention(q, kc, vc, bt, sl, qsl, pkl)
    assert_close(out, r_out)
    assert_lse(lse, r_lse)
