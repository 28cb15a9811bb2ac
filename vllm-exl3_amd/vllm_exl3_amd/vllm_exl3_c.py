"""Drop-in for the reference's native module ``vllm_exl3_c``.

Same function names, keyword names, argument meaning and error behaviour as
the pybind exports of ``csrc/bindings.cpp:197-266``; every call validates its
tensors here (raising ``RuntimeError`` with the reference's message), then
hands raw device pointers to the C ABI of ``libexl3_mi355x.so`` on the current
HIP stream.  There is no CPU compute path: a missing library or a machine
without a GPU raises.
"""

from __future__ import annotations

import math

import torch

from . import _lib

# Module attributes the plugin gates on (csrc/bindings.cpp:243-257).
P2B_MOE_ABI_VERSION = 4
P2B_MOE_MIXED_K = True
P2B_MOE_PADDED = True

CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def codebook_id(mcg: bool, mul1: bool = False, codebook: int | None = None) -> int:
    """Map the reference's (mcg, mul1) flags to a codebook id; `codebook`
    (0 = 3INST, 1 = MCG, 2 = mul1) overrides them."""
    if codebook is not None:
        _check(codebook in (0, 1, 2), "codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)")
        return int(codebook)
    if mcg and mul1:
        raise RuntimeError("a tensor cannot carry both the mcg and the mul1 codebook marker")
    return CB_MCG if mcg else (CB_MUL1 if mul1 else CB_3INST)


def _gpu_device(t: torch.Tensor) -> torch.device:
    if t.is_cuda:
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("vllm_exl3_amd needs a HIP device; there is no CPU compute path")
    return torch.device("cuda", torch.cuda.current_device())


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dequant_trellis(trellis: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor, K: int,
                    mcg: bool, *, mul1: bool = False, codebook: int | None = None) -> torch.Tensor:
    """Decode a trellis into fp16 W[in, out]; result on trellis' device.

    csrc/bindings.cpp:117-132.  Runs on the GPU even for host tensors (they
    are staged through the current device)."""
    K = int(K)
    _check(K in (2, 3, 4, 8), "K must be one of 2, 3, 4, or 8")
    _check(trellis.dim() == 3 and trellis.dtype == torch.int16,
           "trellis must be int16 [rows/16, cols/16, 16*K]")
    _check(trellis.size(2) == 16 * K, "trellis last dimension must be 16*K")
    _check(trellis.size(0) > 0 and trellis.size(1) > 0, "trellis dimensions must be positive")
    _check(suh.dtype == torch.float16 and svh.dtype == torch.float16, "suh and svh must be float16")
    _check(suh.numel() >= trellis.size(0) * 16 and svh.numel() >= trellis.size(1) * 16,
           "suh/svh are too short")
    rows, cols = trellis.size(0) * 16, trellis.size(1) * 16
    _check(rows % 128 == 0 and cols % 128 == 0,
           "trellis dimensions must reconstruct whole 128-element Hadamard blocks")
    cb = codebook_id(mcg, mul1, codebook)
    dev = _gpu_device(trellis)
    t = trellis.to(dev).contiguous()
    su = suh.to(dev).reshape(-1)[:rows].contiguous()
    sv = svh.to(dev).reshape(-1)[:cols].contiguous()
    out = torch.empty((rows, cols), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("exl3_dequant_trellis", t.data_ptr(), t.size(0), t.size(1), K, cb,
                  su.data_ptr(), sv.data_ptr(), out.data_ptr(), stream_of(dev))
    return out if trellis.is_cuda else out.to(trellis.device)


def decode_tiles(trellis: torch.Tensor, K: int, mcg: bool, *, mul1: bool = False,
                 codebook: int | None = None) -> torch.Tensor:
    """Codebook values at tile positions, no rotation (ExLlamaV3 `reconstruct`
    as used at src/vllm_exl3/exl3.py:3130-3156)."""
    K = int(K)
    _check(1 <= K <= 8, "K must be in 1..8")
    _check(trellis.dim() == 3 and trellis.dtype == torch.int16 and trellis.size(2) == 16 * K,
           "trellis must be int16 [rows/16, cols/16, 16*K]")
    cb = codebook_id(mcg, mul1, codebook)
    dev = _gpu_device(trellis)
    t = trellis.to(dev).contiguous()
    out = torch.empty((t.size(0) * 16, t.size(1) * 16), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("exl3_decode_tiles", t.data_ptr(), t.size(0), t.size(1), K, cb,
                  out.data_ptr(), stream_of(dev))
    return out if trellis.is_cuda else out.to(trellis.device)
