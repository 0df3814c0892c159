"""The GPU path runs the in-tree HIP library on the one HIP runtime torch uses."""
import os

import pytest
import torch

import tilelang_fa_v100 as fa
from tilelang_fa_v100 import _lib

pytestmark = pytest.mark.gpu


def test_in_tree_library_and_single_hip_runtime():
    q = torch.randn(1, 128, 2, 64, device="cuda:0", dtype=torch.float16)
    fa.tilelang_flash_attn_func(q, q, q)
    torch.cuda.synchronize()
    maps = open("/proc/self/maps").read()
    libs = {line.split()[-1] for line in maps.splitlines() if line.strip().endswith(".so") or ".so." in line}
    ours = [p for p in libs if p.endswith(_lib.LIB_NAME)]
    assert ours == [os.path.realpath(_lib.LIB_PATH)] or ours == [_lib.LIB_PATH], ours
    hip = sorted({p for p in libs if "libamdhip64" in os.path.basename(p)})
    assert len(hip) == 1, f"more than one HIP runtime mapped: {hip}"
