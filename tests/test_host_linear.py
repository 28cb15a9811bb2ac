"""Host logic of vllm_exl3_amd.linear.apply_exl3_linear on the CPU with
stand-in projections: shard order, padding trim, dtype cast, reshape and the
bias, as the reference's Exl3LinearMethod.apply/_apply_impl
(src/vllm_exl3/exl3.py:6641-6739)."""

from types import SimpleNamespace

import pytest
import torch

from vllm_exl3_amd.linear import apply_exl3_linear


class _Scale:
    """Stand-in EXL3 shard: y = x[:, :n] * s (fp32 out), records its input."""

    def __init__(self, n, s):
        self.n, self.s, self.seen = n, s, []

    def forward(self, x, _params, *, out_dtype, bias=None):
        self.seen.append(x)
        y = x[:, : self.n].to(out_dtype) * self.s
        return y if bias is None else y + bias


def test_shards_concat_cast_reshape_bias():
    a, b = _Scale(3, 2.0), _Scale(2, -1.0)
    layer = SimpleNamespace(_exl3_linears=[a, b], _exl3_linear_output_partition_sizes=[3, 2])
    x = torch.arange(24, dtype=torch.bfloat16).reshape(2, 3, 4)
    bias = torch.tensor([1, 2, 3, 4, 5], dtype=torch.bfloat16)
    y = apply_exl3_linear(layer, x, bias)
    assert y.shape == (2, 3, 5) and y.dtype == torch.bfloat16
    x2 = x.reshape(6, 4).float()
    want = (torch.cat([x2[:, :3] * 2.0, -x2[:, :2]], 1).to(torch.bfloat16) + bias)
    assert torch.equal(y.reshape(6, 5), want)
    assert a.seen[0].dtype == torch.float16  # shards see the fp16-cast input


def test_padding_trim_and_pad_in():
    a = _Scale(6, 1.0)
    layer = SimpleNamespace(_exl3_linears=[a], _exl3_linear_output_partition_sizes=[6],
                            _exl3_linear_padded=True, _exl3_linear_input_size_per_partition=6,
                            _exl3_linear_true_out=[4])
    x = torch.ones(2, 4)
    y = apply_exl3_linear(layer, x)
    assert y.shape == (2, 4) and a.seen[0].shape == (2, 6)
    assert torch.equal(a.seen[0][:, 4:], torch.zeros(2, 2, dtype=torch.float16))


def test_fp32_single_shard_fuses_bias():
    a = _Scale(2, 1.0)
    layer = SimpleNamespace(_exl3_linears=[a], _exl3_linear_output_partition_sizes=[2])
    y = apply_exl3_linear(layer, torch.ones(1, 2), torch.tensor([0.5, 1.5]))
    assert torch.equal(y, torch.tensor([[1.5, 2.5]]))


def test_missing_shards_raise():
    with pytest.raises(RuntimeError, match="not built"):
        apply_exl3_linear(SimpleNamespace(), torch.ones(1, 2))
    layer = SimpleNamespace(_exl3_linears=[None], _exl3_linear_output_partition_sizes=[2])
    with pytest.raises(RuntimeError, match="is None"):
        apply_exl3_linear(layer, torch.ones(1, 2))
