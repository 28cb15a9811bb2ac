"""Workspace cache rules of the compiled drop-in module (host logic, no GPU)."""

import pytest
import torch

from vllm_exl3_amd import vllm_exl3_c as C


@pytest.fixture
def fresh_cache():
    C._C._reset_workspaces_for_tests()
    yield
    C._C._assume_capturing_for_tests(-1)
    C._C._reset_workspaces_for_tests()


def test_growth_keeps_superseded_buffers(fresh_cache):
    cpu = torch.device("cpu")
    a = C.workspace(cpu, "t", 1000)
    assert C.workspace(cpu, "t", 900) is a          # no growth: same buffer
    b = C.workspace(cpu, "t", 1001)
    assert b is not a and b.numel() >= 1500          # grows by at least half
    retired = C.retired_workspaces()
    assert len(retired) == 1 and retired[0] is a     # never freed (graphs may hold it)


def test_growth_during_capture_is_refused(fresh_cache):
    cpu = torch.device("cpu")
    a = C.workspace(cpu, "t", 4096)
    C._C._assume_capturing_for_tests(1)
    assert C.workspace(cpu, "t", 4096) is a          # fits: fine under capture
    with pytest.raises(RuntimeError, match="graph capture"):
        C.workspace(cpu, "t", 8192)
    with pytest.raises(RuntimeError, match="graph capture"):
        C.workspace(cpu, "other", 16)


def test_reserve_workspace_sizes_ahead(fresh_cache):
    cpu = torch.device("cpu")
    ws = C.reserve_workspace(cpu, "reserve_test", 1 << 16)
    assert C.workspace(cpu, "reserve_test", 1 << 15) is ws
