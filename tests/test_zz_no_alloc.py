"""exl3_moe_forward_noalloc (the decode MoE step on the library's own scratch
array, no caller workspace) against exl3_moe_forward (caller workspace), both
called through the C ABI: bit-identical outputs on two calls in a row, the
second with a smaller batch, and the size limit rejected before any launch."""

import ctypes

import numpy as np
import pytest
import torch

from vllm_exl3_amd import _lib
from vllm_exl3_amd import synthetic as S

pytestmark = pytest.mark.gpu
NAMES = ("gate_trellis", "gate_suh", "gate_svh", "up_trellis", "up_suh", "up_svh",
         "down_trellis", "down_suh", "down_svh")


def _args(layer, x, ids, w, T, H, I, E, topk, out):
    tabs = [layer[n].data_ptr() for n in NAMES]
    kt = [t.data_ptr() for t in layer["k_tables"]]
    return ([x.data_ptr(), 1, T, H, I] + tabs +
            [E, kt[0], kt[1], kt[2], 4, 4, 4, 1, 0, 0, 0.0, ids.data_ptr(), 1, w.data_ptr(), 2, topk,
             None, out.data_ptr(), 2])


def test_noalloc_matches_workspace_entry(gpu):
    lib = _lib.load()
    E, H, I, topk = 16, 1024, 512, 8
    ks = S.mixed_k(5, E)
    layer = S.moe_layer_device(5, E, H, I, ks, gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for T in (16, 3):  # the second call is smaller: stale scratch contents must not leak
        x = torch.from_numpy(S.activations(50 + T, T, H)).to(gpu).bfloat16()
        ids_np, w_np = S.softmax_topk(60 + T, T, E, topk)
        ids = torch.from_numpy(ids_np).to(gpu)
        w = torch.from_numpy(w_np).to(gpu)
        need = lib.exl3_moe_workspace_size(T, topk, E, H, I, 0)
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        out_ws = torch.full((T, H), float("nan"), device=gpu)
        out_na = torch.full((T, H), float("nan"), device=gpu)
        rc = lib.exl3_moe_forward(*_args(layer, x, ids, w, T, H, I, E, topk, out_ws), ws.data_ptr(),
                                  need, stream)
        assert rc == 0, _lib.last_error()
        rc = lib.exl3_moe_forward_noalloc(*_args(layer, x, ids, w, T, H, I, E, topk, out_na), stream)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(out_ws).all()
        assert torch.equal(out_ws, out_na), f"T={T}: noalloc result differs"


def test_noalloc_rejects_oversized_calls(gpu):
    lib = _lib.load()
    # T*topk large enough that the workspace exceeds the 64 MiB scratch array
    T, topk, E, H, I = 4096, 8, 64, 4096, 2048
    assert lib.exl3_moe_workspace_size(T, topk, E, H, I, 0) > 64 << 20
    dummy = torch.zeros(16, dtype=torch.int64, device=gpu)
    p = dummy.data_ptr()
    rc = lib.exl3_moe_forward_noalloc(p, 1, T, H, I, *([p] * 9), E, None, None, None, 4, 4, 4, 1, 0,
                                      0, 0.0, p, 1, p, 2, topk, None, p, 2,
                                      torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == -1
    assert "scratch" in _lib.last_error()
