"""Builds libfa355.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: python tilelang-fa-v100_amd/build.py [-v]

Every source in csrc/ is compiled to an object under _build/ (in parallel),
then linked into tilelang_fa_v100/libfa355.so next to the Python package that
loads it.  The library links the HIP runtime by soname (libamdhip64.so.7);
inside a process that has imported torch that resolves to torch's own copy,
so the library and torch share one runtime and one set of streams.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(REPO, "_build")
LIB = os.path.join(HERE, "tilelang_fa_v100", "libfa355.so")

SOURCES = ["fa_fwd.hip", "fa_bwd.hip", "fa_decode.hip", "fa_cache.hip", "fa_scratch.hip",
           "fa_capi.cpp"]
ARCH = "gfx950"

# Per-source flags: MFMA results in VGPRs (the "VGPR form"; AGPRs then hold
# what does not fit).  fa_bwd.hip: its head_dim 256 dK / dV kernel holds
# dK / dV in the 256 accumulator registers; with the default heuristic the
# S / dP accumulators were placed there too and 32 of them spilled to scratch
# every tile (T1-shape head_dim 256 backward 3.54 ms, 2.41 ms in this form).
# fa_fwd.hip: the generic core at head_dim 512 spilled 35 VGPRs (none in this
# form; paged prefill 3.96 -> 3.60 ms) and at head_dim 256 with small pages
# ran 9% faster.  Every head_dim 64 / 128 kernel, and the head_dim 256 cores
# that keep their accumulators in VGPRs anyway, compile to the same code
# either way.
_VGPR_FORM = ["-mllvm", "--amdgpu-mfma-vgpr-form"]
SOURCE_FLAGS = {"fa_bwd.hip": _VGPR_FORM, "fa_fwd.hip": _VGPR_FORM}

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # The process's HIP runtime is the one bundled with torch (ROCm 7.0);
    # code-object v5 is loadable by it.
    "-mcode-object-version=5",
    # Packed FP32 instructions are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n"
                           f"{res.stdout}\n{res.stderr}")
    if verbose and (res.stdout or res.stderr):
        print(res.stdout + res.stderr, flush=True)


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> str:
    """Compiles every source and links the shared library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    flags = COMMON_FLAGS + list(extra_flags or [])
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([cc, *flags, *SOURCE_FLAGS.get(src, []), "-x", "hip", "-c",
                     os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 4)) as ex:
        for fut in [ex.submit(_run, c, verbose) for c in cmds]:
            fut.result()
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
