"""CPU tests of the drop-in boundary: the C ABI library and the Python API.

No GPU is needed: the library loads in a CPU-only process and every argument
check runs before any HIP call, so rejected calls are observable here.
"""
import ctypes
import os
import re
import subprocess

import pytest
import torch

import tilelang_fa_v100 as fa
from tilelang_fa_v100 import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "fa355.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\*?\s+\*?(fa_\w+)\s*\(", text, re.M)))


def test_library_exports_every_header_function():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib._PROTOTYPES), "ctypes prototypes out of sync with header"


def test_abi_version_and_strerror():
    lib = _lib.load()
    assert lib.fa_abi_version() == _lib.ABI_VERSION
    for code in (_lib.FA_OK, _lib.FA_E_INVALID, _lib.FA_E_UNSUPPORTED, _lib.FA_E_HIP,
                 _lib.FA_E_WORKSPACE):
        assert lib.fa_strerror(code)
    assert lib.fa_strerror(-99) == b"unknown status"


STRUCTS = {"fa_fwd_args": _lib.FwdArgs, "fa_bwd_args": _lib.BwdArgs,
           "fa_paged_args": _lib.PagedArgs, "fa_decode_args": _lib.DecodeArgs,
           "fa_cache_write_args": _lib.CacheWriteArgs}


def test_ctypes_structs_match_c_layout(tmp_path):
    """Compiles a C program against the header and compares sizeof/offsetof."""
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "fa355.h"', "int main(void){"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{os.path.dirname(HEADER)}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    for line in out.splitlines():
        cname, field, val = line.split()
        py = STRUCTS[cname]
        if field == "size":
            assert ctypes.sizeof(py) == int(val), cname
        else:
            assert getattr(py, field).offset == int(val), (cname, field)


def fwd_args(**over):
    a = _lib.FwdArgs()
    a.q = a.k = a.v = a.out = 0x1000
    a.lse = 0
    for s in (a.q_stride, a.k_stride, a.v_stride, a.o_stride):
        s[:] = (512 * 16 * 128, 16 * 128, 128)
    a.batch, a.seqlen_q, a.seqlen_k, a.num_heads, a.num_heads_k, a.head_dim = 1, 512, 512, 16, 16, 128
    a.softmax_scale, a.causal, a.dtype = 0.088, 1, 0
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,status", [
    (dict(q=None), _lib.FA_E_INVALID),
    (dict(dtype=7), _lib.FA_E_UNSUPPORTED),
    (dict(head_dim=96), _lib.FA_E_UNSUPPORTED),
    (dict(num_heads_k=5), _lib.FA_E_INVALID),
    (dict(seqlen_q=-1), _lib.FA_E_INVALID),
    (dict(q=0x1008), _lib.FA_E_UNSUPPORTED),  # not 16-byte aligned
])
def test_fwd_rejects_bad_arguments(over, status):
    lib = _lib.load()
    assert lib.fa_fwd(ctypes.byref(fwd_args(**over)), None) == status
    assert lib.fa_last_error_message()


def test_fwd_rejects_unaligned_stride():
    a = fwd_args()
    a.k_stride[1] = 130
    assert _lib.load().fa_fwd(ctypes.byref(a), None) == _lib.FA_E_UNSUPPORTED


@pytest.mark.parametrize("name", ["k_stride", "v_stride"])
def test_fwd_rejects_kv_sequence_stride_beyond_2_pow_24(name):
    a = fwd_args()
    getattr(a, name)[1] = 1 << 24
    assert _lib.load().fa_fwd(ctypes.byref(a), None) == _lib.FA_E_UNSUPPORTED
    assert b"2^24" in _lib.load().fa_last_error_message()


def bwd_args(**over):
    a = _lib.BwdArgs()
    for n in ("q", "k", "v", "out", "dout", "lse", "dq", "dk", "dv"):
        setattr(a, n, 0x2000)
    for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
        getattr(a, f"{n}_stride")[:] = (2048 * 16 * 128, 16 * 128, 128)
    a.batch, a.seqlen_q, a.seqlen_k, a.num_heads, a.num_heads_k, a.head_dim = 4, 2048, 2048, 16, 16, 128
    a.softmax_scale, a.causal, a.dtype = 0.088, 1, 0
    for k, v in over.items():
        setattr(a, k, v)
    return a


def test_bwd_workspace_size_and_checks():
    lib = _lib.load()
    a = bwd_args()
    rows = 4 * 2048 * 16
    stats = 2 * rows * 4 + 256
    # the row statistics (no dQ accumulator), whatever head_dim / `deterministic`;
    # at head_dim 128 / 256 also the dS tiles (causal: 64 * 65 / 2 tiles per head)
    for hd in (64, 128, 256):
        for det in (0, 1):
            ad = bwd_args(head_dim=hd, deterministic=det)
            assert lib.fa_bwd_min_workspace_bytes(ctypes.byref(ad)) == stats
            ds = 2048 * 4 * 16 * (64 * 65 // 2) if hd in (128, 256) else 0
            assert lib.fa_bwd_workspace_bytes(ctypes.byref(ad)) == (stats + ds if ds else stats)
    # workspace missing / too small is rejected before any launch
    assert lib.fa_bwd(ctypes.byref(a), None, 0, None) == _lib.FA_E_WORKSPACE
    assert lib.fa_bwd(ctypes.byref(a), 0x4000, 16, None) == _lib.FA_E_WORKSPACE
    assert lib.fa_bwd(ctypes.byref(bwd_args(head_dim=96)), 0x4000, 1 << 40, None) == \
        _lib.FA_E_UNSUPPORTED
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(bwd_args(lse=None))) == 0
    assert lib.fa_bwd_min_workspace_bytes(ctypes.byref(bwd_args(lse=None))) == 0
    assert lib.fa_bwd_min_workspace_bytes(None) == 0
    # Every grid is one-dimensional: 65536 (batch, head) pairs are accepted,
    # as fa_fwd accepts them, so a training step cannot pass its forward and
    # fail in its backward (tests/test_gpu_dense.py runs such a problem) ...
    big = bwd_args(batch=4096, num_heads=16, num_heads_k=16, seqlen_q=16, seqlen_k=16)
    for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
        getattr(big, f"{n}_stride")[:] = (16 * 16 * 128, 16 * 128, 128)
    stats = 2 * 4096 * 16 * 16 * 4 + 256
    assert lib.fa_bwd_min_workspace_bytes(ctypes.byref(big)) == stats
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(big)) == \
        (stats + 255) // 256 * 256 + 2048 * 4096 * 16
    # ... while grids beyond 32-bit workgroup counts are refused, not truncated
    huge = bwd_args(batch=1 << 20, num_heads=4096, num_heads_k=4096, seqlen_q=1, seqlen_k=1)
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(huge)) == 0
    assert b"too large" in lib.fa_last_error_message()


def _ds_tiles_brute(sq, sk, causal):
    """(query tile, key block) pairs of 32 x 32 that a causal (j <= i + sk - sq)
    or full mask reaches: the dS tiles the dK / dV kernel stores."""
    nq, nk = -(-sq // 32), -(-sk // 32)
    if not causal:
        return nq * nk
    return sum(1 for qt in range(nq) for kb in range(nk) if 32 * kb <= 32 * qt + 31 + sk - sq)


@pytest.mark.parametrize("sq,sk", [(1, 1), (31, 33), (33, 31), (64, 4096), (4096, 64),
                                   (2048, 2048), (1000, 777), (777, 1000), (96, 97), (5, 300),
                                   (300, 5)])
@pytest.mark.parametrize("causal", [0, 1])
def test_bwd_ds_tile_count(sq, sk, causal):
    """The dS workspace holds exactly one 2 KB tile per reachable 32 x 32 pair
    (closed-form prefix sums of the kernels against a brute-force count)."""
    lib = _lib.load()
    a = bwd_args(batch=3, num_heads=5, num_heads_k=5, seqlen_q=sq, seqlen_k=sk, causal=causal)
    for n in ("q", "o", "do", "dq"):
        getattr(a, f"{n}_stride")[:] = (sq * 5 * 128, 5 * 128, 128)
    for n in ("k", "v", "dk", "dv"):
        getattr(a, f"{n}_stride")[:] = (sk * 5 * 128, 5 * 128, 128)
    stats = 2 * 3 * 5 * sq * 4 + 256
    assert lib.fa_bwd_min_workspace_bytes(ctypes.byref(a)) == stats
    off = -(-stats // 256) * 256
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(a)) == \
        off + 2048 * 15 * _ds_tiles_brute(sq, sk, causal)
    # a window band keeps the recompute path (statistics only)
    a.has_window, a.window_left, a.window_right = 1, 40, 0
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(a)) == stats


def test_bwd_ds_workspace_cap():
    """dS tiles beyond 4 GiB: the workspace falls back to the statistics."""
    lib = _lib.load()
    s = 32768
    a = bwd_args(batch=1, num_heads=8, num_heads_k=8, seqlen_q=s, seqlen_k=s, causal=1)
    for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
        getattr(a, f"{n}_stride")[:] = (s * 8 * 128, 8 * 128, 128)
    stats = 2 * 8 * s * 4 + 256
    per_head = 1024 * 1025 // 2  # 1.07 GB of dS per head
    assert 2048 * 8 * per_head > 4 << 30
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(a)) == stats
    a.num_heads = a.num_heads_k = 3  # 3.2 GB: under it
    for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
        getattr(a, f"{n}_stride")[:] = (s * 3 * 128, 3 * 128, 128)
    stats = 2 * 3 * s * 4 + 256
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(a)) == stats + 2048 * 3 * per_head
    # Exactly 4 GiB (one query tile reaching 2^21 key blocks): a wave's dS
    # reads use one buffer resource of count * 2 KB bytes, a 32-bit size that
    # would wrap to zero, so the cap is strict.
    for causal in (0, 1):
        a = bwd_args(batch=1, num_heads=1, num_heads_k=1, seqlen_q=32, seqlen_k=1 << 26,
                     causal=causal)
        for n in ("q", "k", "v", "o", "do", "dq", "dk", "dv"):
            getattr(a, f"{n}_stride")[:] = (a.seqlen_q * 128 if n in ("q", "o", "do", "dq")
                                            else (1 << 26) * 128, 128, 128)
        stats = 2 * 32 * 4 + 256
        assert lib.fa_bwd_min_workspace_bytes(ctypes.byref(a)) == stats
        assert lib.fa_bwd_workspace_bytes(ctypes.byref(a)) == stats
        a.seqlen_k = (1 << 26) - 32  # one key block fewer: under the cap
        assert lib.fa_bwd_workspace_bytes(ctypes.byref(a)) == \
            (stats + 255) // 256 * 256 + 2048 * ((1 << 21) - 1)


def paged_args(**over):
    a = _lib.PagedArgs()
    for n in ("q", "k_cache", "v_cache", "out", "block_table", "seq_lens", "query_start_loc",
              "prefix_kv_lens"):
        setattr(a, n, 0x3000)
    a.q_stride[:] = (32 * 128, 128)
    a.o_stride[:] = (32 * 128, 128)
    a.k_stride[:] = (16 * 8 * 128, 8 * 128, 128)
    a.v_stride[:] = (16 * 8 * 128, 8 * 128, 128)
    a.block_table_stride, a.max_blocks = 300, 237
    a.num_tokens, a.batch, a.num_heads, a.num_kv_heads, a.head_dim = 19679, 8, 32, 8, 128
    a.page_size, a.num_pages, a.softmax_scale, a.causal = 16, 1233, 0.088, 1
    a.window_q = a.window_k = -1
    for k, v in over.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,status", [
    (dict(block_table=None), _lib.FA_E_INVALID),
    (dict(page_size=24), _lib.FA_E_UNSUPPORTED),
    (dict(num_kv_heads=7), _lib.FA_E_INVALID),
    (dict(block_table_stride=100), _lib.FA_E_INVALID),
    (dict(head_dim=80), _lib.FA_E_UNSUPPORTED),
])
def test_paged_rejects_bad_arguments(over, status):
    assert _lib.load().fa_paged_prefill(ctypes.byref(paged_args(**over)), None) == status


def decode_args(**over):
    a = _lib.DecodeArgs()
    for n in ("q", "k_cache", "v_cache", "out", "block_table", "seq_lens"):
        setattr(a, n, 0x5000)
    a.q_stride[:] = (32 * 128, 128)
    a.o_stride[:] = (32 * 128, 128)
    a.k_stride[:] = (16 * 8 * 128, 8 * 128, 128)
    a.v_stride[:] = (16 * 8 * 128, 8 * 128, 128)
    a.block_table_stride, a.max_blocks, a.max_seq_len = 2048, 2048, 32768
    a.batch, a.num_heads, a.num_kv_heads, a.head_dim = 64, 32, 8, 128
    a.page_size, a.num_pages, a.softmax_scale = 16, 131072, 0.088
    for k, v in over.items():
        setattr(a, k, v)
    return a


def test_decode_workspace_and_checks():
    lib = _lib.load()
    a = decode_args()
    # D=128, page >= 16: the streaming kernel; 64 x 16 x 8 items of 2048 keys are
    # >= 2 per resident wave (256 CUs x 8 waves without a GPU): 2048-key splits
    rows = 64 * 32 * (32768 // 2048)
    assert lib.fa_decode_workspace_bytes(ctypes.byref(a)) == rows * 128 * 4 + rows * 4 + 256
    # batch 8: 8 x 64 x 8 items of 512 keys are the first to reach 4096
    b8 = decode_args(batch=8)
    rows8 = 8 * 32 * (32768 // 512)
    assert lib.fa_decode_workspace_bytes(ctypes.byref(b8)) == rows8 * 128 * 4 + rows8 * 4 + 256
    assert lib.fa_paged_decode(ctypes.byref(a), None, 0, None) == _lib.FA_E_WORKSPACE
    assert lib.fa_paged_decode(ctypes.byref(decode_args(max_seq_len=100)), 0x6000, 1 << 40,
                               None) == _lib.FA_E_INVALID
    assert lib.fa_paged_decode(ctypes.byref(decode_args(page_size=3)), 0x6000, 1 << 40,
                               None) == _lib.FA_E_UNSUPPORTED


def test_decode_noalloc_rejects_before_launch():
    """The allocation-free decode validates like fa_paged_decode and refuses
    problems whose split-KV workspace exceeds its static scratch."""
    lib = _lib.load()
    limit = 64 << 20
    big = decode_args(batch=256, num_heads=64)
    assert lib.fa_decode_workspace_bytes(ctypes.byref(big)) > limit
    assert lib.fa_paged_decode_noalloc(ctypes.byref(big), None) == _lib.FA_E_WORKSPACE
    assert b"static buffer" in lib.fa_last_error_message()
    assert lib.fa_paged_decode_noalloc(None, None) == _lib.FA_E_INVALID
    assert lib.fa_paged_decode_noalloc(ctypes.byref(decode_args(page_size=3)),
                                       None) == _lib.FA_E_UNSUPPORTED
    assert lib.fa_paged_decode_noalloc(ctypes.byref(decode_args(max_seq_len=100)),
                                       None) == _lib.FA_E_INVALID
    # The C4 / T2 shapes (64 sequences, 32 / 8 heads, 32k keys) fit.
    assert lib.fa_decode_workspace_bytes(ctypes.byref(decode_args())) <= limit


# ------------------------------------------------------------------ Python API

def _qkv(dtype=torch.float16, shape=(1, 8, 2, 64)):
    return (torch.zeros(shape, dtype=dtype) for _ in range(3))


@pytest.mark.parametrize("kw", [dict(dropout_p=0.1), dict(alibi_slopes=torch.zeros(2)),
                                dict(softcap=1.0)])
def test_unsupported_features_raise_not_implemented(kw):
    q, k, v = _qkv()
    with pytest.raises(NotImplementedError):
        fa.tilelang_flash_attn_func(q, k, v, **kw)


def test_dense_validation_errors():
    q, k, v = _qkv()
    with pytest.raises(TypeError):
        fa.tilelang_flash_attn_func(q.float(), k.float(), v.float())
    with pytest.raises(TypeError):
        fa.tilelang_flash_attn_func(q, k.bfloat16(), v)
    with pytest.raises(ValueError, match="head_dim"):
        fa.tilelang_flash_attn_func(*_qkv(shape=(1, 8, 2, 96)))
    with pytest.raises(ValueError, match="multiple"):
        fa.tilelang_flash_attn_func(torch.zeros(1, 8, 3, 64, dtype=torch.float16), k, v)
    with pytest.raises(ValueError, match="GPU"):
        fa.tilelang_flash_attn_func(q, k, v)
    assert fa.tilelang_flash_attn_gpu is fa.tilelang_flash_attn_func


def test_paged_validation_errors():
    q = torch.zeros(10, 8, 128, dtype=torch.float16)
    kc = torch.zeros(4, 16, 2, 128, dtype=torch.float16)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    sl = torch.tensor([5, 5], dtype=torch.int32)
    qsl = torch.tensor([0, 5, 10], dtype=torch.int32)
    pkl = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="block_size"):
        fa.tilelang_paged_forward(q, kc, kc, bt, sl, qsl, pkl, block_size=32)
    with pytest.raises(ValueError, match="num_kv_heads"):
        fa.tilelang_paged_forward(q, kc, kc, bt, sl, qsl, pkl, num_kv_heads=4)
    with pytest.raises(ValueError, match="multiple"):
        fa.tilelang_paged_forward(torch.zeros(10, 7, 128, dtype=torch.float16),
                                  kc, kc, bt, sl, qsl, pkl)
    with pytest.raises(TypeError):
        fa.tilelang_paged_forward(q, kc.bfloat16(), kc, bt, sl, qsl, pkl)
    with pytest.raises(ValueError, match="GPU"):
        fa.tilelang_paged_forward(q, kc, kc, bt, sl, qsl, pkl)


def test_decode_validation_errors():
    q = torch.zeros(2, 8, 128, dtype=torch.float16)
    kc = torch.zeros(4, 16, 2, 128, dtype=torch.float16)
    bt = torch.zeros(2, 2, dtype=torch.int32)
    sl = torch.tensor([5, 5], dtype=torch.int32)
    with pytest.raises(ValueError, match="block_size"):
        fa.tilelang_decode_forward(q, kc, kc, bt, sl, block_size=8)
    with pytest.raises(ValueError, match="block_table"):
        fa.tilelang_decode_forward(q, kc, kc, bt[:1], sl)
    with pytest.raises(ValueError, match="GPU"):
        fa.tilelang_decode_forward(q, kc, kc, bt, sl)


def test_paged_splitkv_workspace_and_checks():
    lib = _lib.load()
    a = paged_args()
    rows_per_split = a.num_heads * a.num_tokens
    assert lib.fa_paged_prefill_splitkv_workspace_bytes(ctypes.byref(a), 1) == 0
    assert lib.fa_paged_prefill_splitkv_workspace_bytes(ctypes.byref(a), 4) == \
        4 * rows_per_split * (a.head_dim * 4 + 4) + 256
    assert lib.fa_paged_prefill_splitkv_workspace_bytes(ctypes.byref(a), 0) == 0
    assert lib.fa_paged_prefill_splitkv_workspace_bytes(ctypes.byref(a), 65) == 0
    for ns in (0, 65, -2):
        assert lib.fa_paged_prefill_splitkv(ctypes.byref(a), ns, None, 0, None) == \
            _lib.FA_E_INVALID
    # missing / short / unaligned workspace is rejected before any launch
    need = lib.fa_paged_prefill_splitkv_workspace_bytes(ctypes.byref(a), 4)
    assert lib.fa_paged_prefill_splitkv(ctypes.byref(a), 4, None, 0, None) == _lib.FA_E_WORKSPACE
    assert lib.fa_paged_prefill_splitkv(ctypes.byref(a), 4, 0x4000, need - 1, None) == \
        _lib.FA_E_WORKSPACE
    assert lib.fa_paged_prefill_splitkv(ctypes.byref(a), 4, 0x4008, need, None) == \
        _lib.FA_E_WORKSPACE
    assert lib.fa_paged_prefill_num_splits(ctypes.byref(paged_args(q=None))) == _lib.FA_E_INVALID


def test_paged_and_decode_accept_head_dim_512_dense_does_not():
    lib = _lib.load()
    # validation only (the rejected cases never launch)
    assert lib.fa_paged_prefill(ctypes.byref(paged_args(head_dim=384)), None) == \
        _lib.FA_E_UNSUPPORTED
    assert lib.fa_paged_prefill_num_splits(ctypes.byref(paged_args(head_dim=512))) >= 1
    assert lib.fa_fwd(ctypes.byref(fwd_args(head_dim=512)), None) == _lib.FA_E_UNSUPPORTED
    assert lib.fa_bwd(ctypes.byref(bwd_args(head_dim=512)), 0x4000, 1 << 40, None) == \
        _lib.FA_E_UNSUPPORTED


def test_paged_num_splits_heuristic():
    lib = _lib.load()
    # C3-sized batch: enough query tiles to fill the GPU -> no split
    assert lib.fa_paged_prefill_num_splits(ctypes.byref(paged_args())) == 1
    # 64 tokens, 8 KV heads (8 workgroups), 32k-key block table -> split:
    # about one workgroup per CU (256 CUs without a GPU), ranges of 1024-8192 keys
    few = paged_args(num_tokens=64, batch=1, max_blocks=2048, block_table_stride=2048)
    ns = lib.fa_paged_prefill_num_splits(ctypes.byref(few))
    assert ns == 32
    # 256 tokens x 4 heads per KV head = 4 row tiles, x 8 KV heads = 32 workgroups;
    # 8k-key table: max(256 / 32, 1) = 8 ranges of 1024 keys
    mid = paged_args(num_tokens=256, batch=1, max_blocks=512, block_table_stride=512)
    assert lib.fa_paged_prefill_num_splits(ctypes.byref(mid)) == 8
    # 64k-key table: max(8, 8) = 8; 128k keys: max(8, 16) = 16 (ranges of at most 8192 keys)
    big = paged_args(num_tokens=256, batch=1, max_blocks=8192, block_table_stride=8192)
    assert lib.fa_paged_prefill_num_splits(ctypes.byref(big)) == 16
    # same tokens, short block table (< 4096 keys) -> no split
    short = paged_args(num_tokens=64, batch=1, max_blocks=128, block_table_stride=128)
    assert lib.fa_paged_prefill_num_splits(ctypes.byref(short)) == 1


def test_public_api_matches_reference_signatures():
    import inspect
    sig = inspect.signature(fa.tilelang_flash_attn_func)
    assert list(sig.parameters) == ["q", "k", "v", "dropout_p", "softmax_scale", "causal",
                                    "window_size", "softcap", "alibi_slopes", "deterministic",
                                    "return_attn_probs"]
    assert sig.parameters["causal"].default is False
    sig = inspect.signature(fa.tilelang_paged_forward)
    assert list(sig.parameters) == ["q", "k_cache", "v_cache", "block_table", "seq_lens",
                                    "query_start_loc", "prefix_kv_lens", "out", "block_size",
                                    "num_kv_heads", "softmax_scale", "causal",
                                    "sliding_window_q", "sliding_window_k"]
    assert sig.parameters["causal"].default is True
    assert sig.parameters["block_size"].default == 16
    sig = inspect.signature(fa.tilelang_decode_forward)
    assert list(sig.parameters) == ["q", "k_cache", "v_cache", "block_table", "seq_lens",
                                    "block_size", "num_kv_heads", "softmax_scale"]
    assert fa.__all__ == ["tilelang_flash_attn_func", "tilelang_flash_attn_gpu",
                          "tilelang_paged_forward", "tilelang_decode_forward"]
    # The cache writer (no reference counterpart) follows vLLM's argument order.
    sig = inspect.signature(fa.reshape_and_cache)
    assert list(sig.parameters) == ["key", "value", "key_cache", "value_cache", "slot_mapping"]


def test_reshape_and_cache_rejects_bad_arguments_before_launch():
    k = torch.zeros(4, 2, 64, dtype=torch.float16)
    kc = torch.zeros(3, 16, 2, 64, dtype=torch.float16)
    slots = torch.arange(4)
    with pytest.raises(TypeError):
        fa.reshape_and_cache(k.float(), k, kc, kc, slots)
    with pytest.raises(TypeError):
        fa.reshape_and_cache(k, k, kc, kc, slots.float())
    with pytest.raises(ValueError):
        fa.reshape_and_cache(k, k[:, :1], kc, kc, slots)
    with pytest.raises(ValueError):
        fa.reshape_and_cache(k, k, kc[:, :, :1], kc[:, :, :1], slots)
    with pytest.raises(ValueError):
        fa.reshape_and_cache(k, k, kc, kc, slots[:3])
    with pytest.raises(ValueError):  # CPU tensors: a GPU is required
        fa.reshape_and_cache(k, k, kc, kc, slots)


def test_cache_write_abi_rejects_bad_arguments():
    lib = _lib.load()
    a = _lib.CacheWriteArgs()
    a.key = a.value = a.k_cache = a.v_cache = 0x1000
    a.slot_mapping = 0x2000
    a.key_stride[:] = (256, 128)
    a.value_stride[:] = (256, 128)
    a.k_stride[:] = (16 * 256, 256, 128)
    a.v_stride[:] = (16 * 256, 256, 128)
    a.num_tokens, a.num_kv_heads, a.head_dim, a.page_size, a.num_pages, a.dtype = 4, 2, 128, 16, 3, 0
    bad = [("head_dim", 100), ("dtype", 7), ("page_size", 0), ("num_kv_heads", 0)]
    for field, val in bad:
        old = getattr(a, field)
        setattr(a, field, val)
        assert lib.fa_reshape_and_cache(ctypes.byref(a), None) != 0, field
        setattr(a, field, old)
    a.key = 0x1008  # misaligned
    assert lib.fa_reshape_and_cache(ctypes.byref(a), None) == _lib.FA_E_UNSUPPORTED
    a.key = 0
    assert lib.fa_reshape_and_cache(ctypes.byref(a), None) == _lib.FA_E_INVALID


def test_window_size_is_validated_before_launch():
    q = torch.zeros(1, 4, 2, 64, dtype=torch.float16)
    with pytest.raises(ValueError):
        fa.tilelang_flash_attn_func(q, q, q, window_size=(-2, 0))
    with pytest.raises(ValueError):
        fa.tilelang_flash_attn_func(q, q, q, window_size=(3,))
    lib = _lib.load()
    a = fwd_args(has_window=1, window_left=-5)
    assert lib.fa_fwd(ctypes.byref(a), None) == _lib.FA_E_INVALID
