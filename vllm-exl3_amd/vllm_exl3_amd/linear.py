"""Dense EXL3 linear layers: the host side of the reference's
``Exl3LinearMethod.apply`` (src/vllm_exl3/exl3.py:6641-6739) over the HIP
linear (``vllm_exl3_c.exl3_gemm``).

A layer holds one or more output shards (fused q/k/v or gate/up
projections): each EXL3 shard is an :class:`~vllm_exl3_amd.dispatch.Exl3Linear`
run on the fp16-cast input with fp32 output (the reference's
``_dense_forward``, exl3.py:5797-5819: its row-count switch to
reconstruct + hgemm above 16 rows lives inside ``exl3_gemm`` here, which
decodes on MFMA from 128 rows); bf16 shards are plain ``F.linear`` slices of
``_exl3_bf16_weight``.  Shard outputs are concatenated along the output
dimension, padded columns trimmed, the result cast to x's dtype and reshaped
to x's leading dimensions, and the bias added last, as the reference does.

Layer attributes read (the reference's names): ``_exl3_linears``,
``_exl3_linear_output_partition_sizes``, ``_exl3_linear_bf16_shards``,
``_exl3_bf16_weight``, ``_exl3_linear_padded``,
``_exl3_linear_input_size_per_partition``, ``_exl3_linear_true_out``.
"""

from __future__ import annotations

from typing import Any

import torch
import torch.nn.functional as F


def apply_exl3_linear(layer: Any, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    linears = getattr(layer, "_exl3_linears", None)
    if not linears:
        raise RuntimeError("EXL3 linear layers were not built after weight load")
    orig_shape = x.shape
    x_2d = x.reshape(-1, orig_shape[-1])
    x_fp16 = x_2d.to(torch.float16).contiguous()
    if getattr(layer, "_exl3_linear_padded", False):
        pad_in = int(layer._exl3_linear_input_size_per_partition) - int(x_fp16.shape[1])
        if pad_in > 0:
            x_fp16 = F.pad(x_fp16, (0, pad_in))
    bf16_shards = list(getattr(layer, "_exl3_linear_bf16_shards", []))
    bf16_weight = getattr(layer, "_exl3_bf16_weight", None)
    sizes = list(getattr(layer, "_exl3_linear_output_partition_sizes", []))
    # a single EXL3 shard takes the bias into its output pass
    fused_bias = bias is not None and len(linears) == 1 and not bf16_shards \
        and not getattr(layer, "_exl3_linear_padded", False) and x.dtype == torch.float32
    outputs = []
    for i, linear in enumerate(linears):
        if i in bf16_shards:
            if bf16_weight is None:
                raise RuntimeError(f"EXL3 bf16 shard {i} but _exl3_bf16_weight is missing")
            j = bf16_shards.index(i)
            start = sum(sizes[s] for s in bf16_shards[:j])
            outputs.append(F.linear(x_2d, bf16_weight[start:start + sizes[i]]).to(torch.float32))
        else:
            if linear is None:
                raise RuntimeError(f"EXL3 linear shard {i} is None")
            outputs.append(linear.forward(x_fp16, {}, out_dtype=torch.float32,
                                          **({"bias": bias} if fused_bias else {})))
    y = torch.cat(outputs, dim=1) if len(outputs) > 1 else outputs[0]
    if getattr(layer, "_exl3_linear_padded", False):
        y = y[:, : sum(layer._exl3_linear_true_out)]
    y = y.to(dtype=x.dtype)
    if len(orig_shape) > 2:
        y = y.reshape(*orig_shape[:-1], y.shape[-1])
    if bias is not None and not fused_bias:
        y = y + bias
    return y
