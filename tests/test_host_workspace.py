"""Workspace cache rules of the drop-in module (host logic, no GPU)."""

import pytest
import torch

from vllm_exl3_amd import vllm_exl3_c as C


def test_growth_keeps_superseded_buffers(monkeypatch):
    monkeypatch.setattr(C, "_WORKSPACES", {})
    monkeypatch.setattr(C, "_RETIRED", [])
    cpu = torch.device("cpu")
    a = C.workspace(cpu, "t", 1000)
    assert C.workspace(cpu, "t", 900) is a          # no growth: same buffer
    b = C.workspace(cpu, "t", 1001)
    assert b is not a and b.numel() >= 1500          # grows by at least half
    assert C._RETIRED == [a]                         # never freed (graphs may hold it)


def test_growth_during_capture_is_refused(monkeypatch):
    monkeypatch.setattr(C, "_WORKSPACES", {})
    monkeypatch.setattr(C, "_RETIRED", [])
    cpu = torch.device("cpu")
    a = C.workspace(cpu, "t", 4096)
    monkeypatch.setattr(C, "_capturing", lambda dev: True)
    assert C.workspace(cpu, "t", 4096) is a          # fits: fine under capture
    with pytest.raises(RuntimeError, match="graph capture"):
        C.workspace(cpu, "t", 8192)
    with pytest.raises(RuntimeError, match="graph capture"):
        C.workspace(cpu, "other", 16)


def test_reserve_workspace_sizes_ahead():
    cpu = torch.device("cpu")
    ws = C.reserve_workspace(cpu, "reserve_test", 1 << 16)
    assert C.workspace(cpu, "reserve_test", 1 << 15) is ws
