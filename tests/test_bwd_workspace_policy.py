"""CPU tests of the dense backward's workspace choice (tilelang_fa_v100._dense).

fa_bwd takes either the dS-path workspace (statistics + dS tiles) or the
minimal one (statistics only, dQ recomputed as in the reference's
_kernels_backward.py:10-85).  The Python layer takes the dS path only while it
fits the limit (a caller-set value, the environment variable, or a share of
the device memory still available) and falls back to the minimal workspace
when that allocation runs out of memory.  No GPU is touched here: device
memory queries and the allocator are replaced.
"""
import pytest
import torch

from tilelang_fa_v100 import _dense, set_backward_workspace_limit

FULL, MIN = 2_150_000_000, 1_048_832


@pytest.fixture(autouse=True)
def _reset(monkeypatch):
    monkeypatch.delenv(_dense.WORKSPACE_LIMIT_ENV, raising=False)
    set_backward_workspace_limit(None)
    yield
    set_backward_workspace_limit(None)


def test_choose_workspace():
    assert _dense.choose_workspace(FULL, MIN, FULL) == FULL        # fits exactly
    assert _dense.choose_workspace(FULL, MIN, FULL - 1) == MIN     # one byte short
    assert _dense.choose_workspace(FULL, MIN, 0) == MIN
    assert _dense.choose_workspace(MIN, MIN, 1 << 60) == MIN       # no dS path (D = 64, windows)


def test_limit_sources(monkeypatch):
    calls = []

    def mem_get_info(device):
        calls.append(device)
        return 10_000, 80_000

    monkeypatch.setattr(torch.cuda, "mem_get_info", mem_get_info)
    monkeypatch.setattr(torch.cuda, "memory_reserved", lambda device: 3_000)
    monkeypatch.setattr(torch.cuda, "memory_allocated", lambda device: 1_000)
    # default: half of (free + cached-but-unused)
    assert _dense.workspace_limit("cuda:0") == (10_000 + 2_000) // 2
    assert _dense.workspace_limit("cuda:0", want=2_001) == (10_000 + 2_000) // 2
    assert calls == ["cuda:0", "cuda:0"]
    # a dS workspace that fits torch's cached blocks is taken from them, and
    # the device is not queried
    assert _dense.workspace_limit("cuda:0", want=2_000) == 2_000
    assert len(calls) == 2
    # the environment variable overrides the default ...
    monkeypatch.setenv(_dense.WORKSPACE_LIMIT_ENV, "12345")
    assert _dense.workspace_limit("cuda:0") == 12345
    # ... and the setter overrides both, without querying the device
    set_backward_workspace_limit(0)
    assert _dense.workspace_limit("cuda:0") == 0
    assert len(calls) == 2
    monkeypatch.setenv(_dense.WORKSPACE_LIMIT_ENV, "lots")
    set_backward_workspace_limit(None)
    with pytest.raises(ValueError):
        _dense.workspace_limit("cuda:0")
    with pytest.raises(ValueError):
        set_backward_workspace_limit(-1)


def test_alloc_falls_back_on_out_of_memory(monkeypatch):
    asked = []

    def empty(n, device):
        asked.append(n)
        if n > MIN:
            raise torch.cuda.OutOfMemoryError("HIP out of memory (test)")
        return torch.empty(n, dtype=torch.uint8)

    monkeypatch.setattr(_dense, "_empty_bytes", empty)
    set_backward_workspace_limit(1 << 40)
    ws = _dense.alloc_workspace(FULL, MIN, "cuda:0")
    assert ws.numel() == MIN and asked == [FULL, MIN]


def test_alloc_respects_limit_without_trying_the_large_size(monkeypatch):
    asked = []
    monkeypatch.setattr(_dense, "_empty_bytes",
                        lambda n, device: asked.append(n) or torch.empty(n, dtype=torch.uint8))
    set_backward_workspace_limit(FULL - 1)
    assert _dense.alloc_workspace(FULL, MIN, "cuda:0").numel() == MIN
    set_backward_workspace_limit(FULL)
    assert _dense.alloc_workspace(FULL, MIN, "cuda:0").numel() == FULL
    assert asked == [MIN, FULL]


def test_minimal_allocation_failure_propagates(monkeypatch):
    def empty(n, device):
        raise torch.cuda.OutOfMemoryError("HIP out of memory (test)")

    monkeypatch.setattr(_dense, "_empty_bytes", empty)
    set_backward_workspace_limit(1 << 40)
    with pytest.raises(torch.cuda.OutOfMemoryError):
        _dense.alloc_workspace(FULL, MIN, "cuda:0")
    with pytest.raises(torch.cuda.OutOfMemoryError):
        _dense.alloc_workspace(MIN, MIN, "cuda:0")
