"""GPU parity at the full BASELINE sizes, checked against the CPU oracle.

* C5: 16 sequences, prefix_kv_lens from
  randint(0, 8193, (16,)) with seed 0, 512 new tokens each, 64 / 8 heads,
  D = 128, bf16, scattered pages (the convention of
  tests/test_gqa_paged.py:150-219 in the reference: prefix = total - q_len).
* C4 and T2 (C4 with every context at 32768): 64 sequences,
  32 / 8 heads, D = 128, fp16; the caches (2-4 GB each) are drawn on the
  GPU, copied to the host and the oracle gathers every sequence's pages
  itself.
* T1 (dense causal, B = 2, S = 8192, H = 16, D = 128, fp16): forward and
  backward on the GPU; sampled (batch, head) slices against the oracle.  The
  same at head_dim 256 (H = 8, the bench's T1-shape D = 256 point): its
  backward runs ~2000 query tiles per key tile, far more than the small
  shapes of test_gpu_dense.py (a build whose register allocator spilled
  the dV accumulators got dV wrong only at this size).

The GPU runs once per workload (module-scoped fixtures); the oracle checks
are split into chunks of sequences / heads so that each test stays short.
Tolerances: outputs and gradients atol 2e-3 / rtol 1e-2, LSE 1e-3, plus a
relative L2 bound.
"""
import math

import pytest
import torch

import tilelang_fa_v100 as fa
from tilelang_fa_v100._decode_adapter import decode_forward
from helpers import assert_close, assert_lse, build_paged, randn, rel_l2
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


# --------------------------------------------------------------------- C5

C5_PREFIX = [1751, 3120, 3566, 3048, 244, 5664, 6907, 5746, 127, 492, 1652, 980, 5907, 6417,
             6694, 2486]


@pytest.fixture(scope="module")
def c5():
    g = torch.Generator().manual_seed(0)
    pf = torch.randint(0, 8193, (16,), generator=g).tolist()
    assert pf == C5_PREFIX
    lens = [p + 512 for p in pf]
    dt = torch.bfloat16
    ks = [randn(g, n, 8, 128, dtype=dt) for n in lens]
    vs = [randn(g, n, 8, 128, dtype=dt) for n in lens]
    kc, vc, bt = build_paged(g, ks, vs, 16, dtype=dt)
    q = randn(g, 16 * 512, 64, 128, dtype=dt)
    qsl = torch.arange(0, 16 * 512 + 1, 512, dtype=torch.int32)
    c = dict(q=q, k_cache=kc, v_cache=vc, block_table=bt,
             seq_lens=torch.tensor(lens, dtype=torch.int32), query_start_loc=qsl,
             prefix_kv_lens=torch.tensor(pf, dtype=torch.int32))
    out, lse = fa.tilelang_paged_forward(*(c[n].to(DEV) for n in (
        "q", "k_cache", "v_cache", "block_table", "seq_lens", "query_start_loc",
        "prefix_kv_lens")), num_kv_heads=8)
    torch.cuda.synchronize()
    return c, out.cpu(), lse.cpu()


@pytest.mark.parametrize("chunk", range(4))
def test_c5_full_batch_vs_oracle(c5, chunk):
    c, out, lse = c5
    seqs = range(4 * chunk, 4 * chunk + 4)
    for b in seqs:
        s0, s1 = 512 * b, 512 * (b + 1)
        one = dict(c)
        one["block_table"] = c["block_table"][b:b + 1]
        one["seq_lens"] = c["seq_lens"][b:b + 1]
        one["prefix_kv_lens"] = c["prefix_kv_lens"][b:b + 1]
        one["query_start_loc"] = torch.tensor([0, 512], dtype=torch.int32)
        r_out, r_lse = ref.paged_attention(
            c["q"][s0:s1], one["k_cache"], one["v_cache"], one["block_table"],
            one["seq_lens"], one["query_start_loc"], one["prefix_kv_lens"])
        assert_close(out[s0:s1], r_out, what=f"seq {b} out")
        assert_lse(lse[:, s0:s1], r_lse, what=f"seq {b} lse")
        assert rel_l2(out[s0:s1], r_out) < 1e-2


# --------------------------------------------------------------------- C4 / T2

def decode_workload(lens, seed=0):
    """Scattered-page caches drawn on the GPU; NaN in the slots past each
    sequence's length; block-table padding -1.  Returns host copies too."""
    g = torch.Generator().manual_seed(seed)
    B, Hq, Hkv, D, page = len(lens), 32, 8, 128, 16
    npg = [math.ceil(n / page) for n in lens]
    pool = sum(npg)
    perm = torch.randperm(pool, generator=g)
    bt = torch.full((B, max(npg) + 1), -1, dtype=torch.int32)
    cur = 0
    for b, n in enumerate(npg):
        bt[b, :n] = perm[cur:cur + n].to(torch.int32)
        cur += n
    q = randn(g, B, Hq, D)
    gd = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn(pool, page, Hkv, D, generator=gd, device=DEV).half()
    vc = torch.randn(pool, page, Hkv, D, generator=gd, device=DEV).half()
    for b, n in enumerate(lens):
        if n % page:
            last = int(bt[b, npg[b] - 1])
            kc[last, n % page:] = float("nan")
            vc[last, n % page:] = float("nan")
    sl = torch.tensor(lens, dtype=torch.int32)
    out, lse = decode_forward(q.to(DEV), kc, vc, bt.to(DEV), sl.to(DEV), return_lse=True)
    torch.cuda.synchronize()
    return dict(q=q, k_cache=kc.cpu(), v_cache=vc.cpu(), block_table=bt, seq_lens=sl,
                out=out.cpu(), lse=lse.cpu())


@pytest.fixture(scope="module")
def c4():
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(1024, 32769, (64,), generator=g).tolist()
    return decode_workload(lens)


@pytest.fixture(scope="module")
def t2():
    return decode_workload([32768] * 64)


def check_decode(w, seqs):
    for b in seqs:
        r_out, r_lse = ref.decode_attention(w["q"][b:b + 1], w["k_cache"], w["v_cache"],
                                            w["block_table"][b:b + 1], w["seq_lens"][b:b + 1])
        assert_close(w["out"][b:b + 1], r_out, what=f"seq {b} out")
        assert_lse(w["lse"][b:b + 1], r_lse, what=f"seq {b} lse")
        assert rel_l2(w["out"][b:b + 1], r_out) < 1e-2


@pytest.mark.parametrize("chunk", range(4))
def test_c4_full_batch_vs_oracle(c4, chunk):
    check_decode(c4, range(16 * chunk, 16 * chunk + 16))


@pytest.mark.parametrize("chunk", range(4))
def test_t2_full_batch_vs_oracle(t2, chunk):
    check_decode(t2, range(16 * chunk, 16 * chunk + 16))


# --------------------------------------------------------------------- T1

@pytest.fixture(scope="module")
def t1():
    B, S, H, D = 2, 8192, 16, 128
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (randn(g, B, S, H, D) for _ in range(4))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out, lse, _ = fa.tilelang_flash_attn_func(qd, kd, vd, causal=True, return_attn_probs=True)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    got = dict(out=out.detach().cpu(), lse=lse.cpu(), dq=qd.grad.cpu(), dk=kd.grad.cpu(),
               dv=vd.grad.cpu())
    return (q, k, v, do), got


T1_SLICES = [(1, 0), (1, 7), (1, 15), (0, 3)]


@pytest.mark.parametrize("bh", T1_SLICES, ids=[f"b{b}h{h}" for b, h in T1_SLICES])
def test_t1_slices_vs_oracle(t1, bh):
    (q, k, v, do), got = t1
    b, h = bh
    sl = lambda t: t[b:b + 1, :, h:h + 1]  # noqa: E731
    r_out, r_lse = ref.dense_attention(sl(q), sl(k), sl(v), causal=True)
    assert_close(sl(got["out"]), r_out, what="out")
    assert_lse(got["lse"][b:b + 1, h:h + 1], r_lse)
    r_dq, r_dk, r_dv = ref.dense_attention_backward(sl(q), sl(k), sl(v), sl(do), causal=True)
    for name, want in (("dq", r_dq), ("dk", r_dk), ("dv", r_dv)):
        assert_close(sl(got[name]), want, what=name)
        assert rel_l2(sl(got[name]), want) < 1e-2, name


@pytest.fixture(scope="module")
def t1_d256():
    B, S, H, D = 2, 8192, 8, 256
    g = torch.Generator().manual_seed(1)
    q, k, v, do = (randn(g, B, S, H, D) for _ in range(4))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = fa.tilelang_flash_attn_func(qd, kd, vd, causal=True)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    got = dict(out=out.detach().cpu(), dq=qd.grad.cpu(), dk=kd.grad.cpu(), dv=vd.grad.cpu())
    return (q, k, v, do), got


T1_D256_SLICES = [(0, 0), (1, 7)]


@pytest.mark.parametrize("bh", T1_D256_SLICES, ids=[f"b{b}h{h}" for b, h in T1_D256_SLICES])
def test_t1_shape_d256_slices_vs_oracle(t1_d256, bh):
    (q, k, v, do), got = t1_d256
    b, h = bh
    sl = lambda t: t[b:b + 1, :, h:h + 1]  # noqa: E731
    r_out, _ = ref.dense_attention(sl(q), sl(k), sl(v), causal=True)
    assert_close(sl(got["out"]), r_out, what="out")
    r_dq, r_dk, r_dv = ref.dense_attention_backward(sl(q), sl(k), sl(v), sl(do), causal=True)
    for name, want in (("dq", r_dq), ("dk", r_dk), ("dv", r_dv)):
        assert_close(sl(got[name]), want, what=name)
        assert rel_l2(sl(got[name]), want) < 1e-2, name
