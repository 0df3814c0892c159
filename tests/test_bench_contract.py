"""CPU checks of bench.py's contract that need no GPU."""
import os
import re
import subprocess
import sys

from tilelang_fa_v100 import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_uses_only_existing_library_helpers():
    src = open(os.path.join(REPO, "bench.py")).read()
    names = set(re.findall(r"\b_lib\.(\w+)", src))
    assert names, "bench.py no longer calls the library helpers?"
    missing = sorted(n for n in names if not hasattr(_lib, n))
    assert not missing, f"bench.py uses missing _lib attributes: {missing}"


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "1 GPU" in (r.stdout + r.stderr)
