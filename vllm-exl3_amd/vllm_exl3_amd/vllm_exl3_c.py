"""Drop-in for the reference's native module ``vllm_exl3_c``.

The functions are those of the compiled PyTorch-ROCm extension ``_C``
(``csrc/torch_ext.cpp``): the pybind exports of ``csrc/bindings.cpp:197-266``
with the same names, keyword names, argument meaning and error behaviour
(``RuntimeError`` with the reference's message), plus this build's executor
entries.  Each validates its tensors in C++ and hands raw device pointers to
the C ABI of ``libexl3_mi355x.so`` on the current HIP stream.  There is no
CPU compute path: importing this module without the built extension raises.

Exports:
  dequant_trellis, exl3_gemv, exl3_gemm, p2b_gemv_batched, p2b_fused_moe,
  p2b_fused_moe_mk, p2b_fused_moe_padded, exl3_fat_gemm, exl3_fat_gemm_scatter
      -- the reference module's functions (keyword extensions: ``codebook``,
         ``mul1``; ``exl3_gemm``'s ``out_dtype`` and ``bias``;
         ``p2b_gemv_batched``'s ``out_features``);
  moe_forward, moe_prefill -- the routed-expert decode and prefill executors
      (``x`` [T, hidden], ``ids`` / ``weights`` [T, topk], ``tables`` the nine
      int64 pointer tables by name, K tables optional, ``n_valid`` optional);
  decode_tiles, ngram_dequant_rows, ngram_words_per_row;
  workspace, reserve_workspace -- the per-(device, kind) scratch cache shared
      by every entry point (grown on demand, never freed, growth refused
      during graph capture).
"""

from __future__ import annotations

import torch

from . import _C
from ._C import (  # noqa: F401
    NGRAM_ROW_DIM,
    P2B_MOE_ABI_VERSION,
    P2B_MOE_MIXED_K,
    P2B_MOE_PADDED,
    decode_tiles,
    dequant_trellis,
    exl3_fat_gemm,
    exl3_fat_gemm_scatter,
    exl3_gemm,
    exl3_gemv,
    moe_forward,
    moe_prefill,
    ngram_dequant_rows,
    ngram_words_per_row,
    p2b_fused_moe,
    p2b_fused_moe_mk,
    p2b_fused_moe_padded,
    p2b_gemv_batched,
    reserve_workspace,
    retired_workspaces,
    workspace,
)

CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
ACT_SILU, ACT_RELU2, ACT_SWIGLU_OAI = 0, 2, 3

# dtype ids of the C ABI (fp16 / bf16 / fp32), for the modules that call the
# C ABI directly (the KV caches, whose reference host code is Python)
_DTYPE_ID = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def codebook_id(mcg: bool, mul1: bool = False, codebook: int | None = None) -> int:
    """Map the reference's (mcg, mul1) flags to a codebook id; `codebook`
    (0 = 3INST, 1 = MCG, 2 = mul1) overrides them."""
    if codebook is not None:
        if codebook not in (0, 1, 2):
            raise RuntimeError("codebook must be 0 (3INST), 1 (MCG) or 2 (mul1)")
        return int(codebook)
    if mcg and mul1:
        raise RuntimeError("a tensor cannot carry both the mcg and the mul1 codebook marker")
    return CB_MCG if mcg else (CB_MUL1 if mul1 else CB_3INST)


def stream_of(device: torch.device) -> int:
    """The current HIP stream of `device` as an integer handle."""
    return torch.cuda.current_stream(device).cuda_stream


__all__ = [
    "P2B_MOE_ABI_VERSION", "P2B_MOE_MIXED_K", "P2B_MOE_PADDED", "NGRAM_ROW_DIM",
    "CB_3INST", "CB_MCG", "CB_MUL1", "ACT_SILU", "ACT_RELU2", "ACT_SWIGLU_OAI",
    "dequant_trellis", "decode_tiles", "exl3_gemv", "exl3_gemm", "p2b_gemv_batched",
    "moe_forward", "moe_prefill", "exl3_fat_gemm", "exl3_fat_gemm_scatter", "p2b_fused_moe",
    "p2b_fused_moe_mk", "p2b_fused_moe_padded", "ngram_words_per_row", "ngram_dequant_rows",
    "workspace", "reserve_workspace", "retired_workspaces", "codebook_id", "stream_of", "_C",
]
