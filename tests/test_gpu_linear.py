"""GPU parity of the dense EXL3 linear at large m (the fat path: rotate,
MFMA GEMM over the decoded weights, output pass with optional bias) and of the
host linear method (vllm_exl3_amd.linear.apply_exl3_linear), against the
oracle's dequant + fp32 matmul.  Relative L2 <= 2e-3."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import rel_l2
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C
from vllm_exl3_amd.dispatch import Exl3Linear
from vllm_exl3_amd.linear import apply_exl3_linear

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _dev(lin, gpu):
    return [torch.from_numpy(lin[k]).to(gpu) for k in ("trellis", "suh", "svh")]


@pytest.mark.parametrize("K,cb", [(2, 1), (3, 0), (4, 2), (4, 1)])
@pytest.mark.parametrize("m", [127, 128, 300, 2048])
def test_linear_large_m_vs_oracle(gpu, K, cb, m):
    in_f, out_f = 512, 384
    lin = S.linear(5000 + 10 * K + cb + m, in_f, out_f, K)
    x = S.activations(9 + m, m, in_f)
    bias = (np.random.default_rng(m).standard_normal(out_f) * 0.1).astype(np.float16)
    want = O.gemv(x, O.dequant(lin["trellis"], lin["suh"], lin["svh"], K, cb)) + bias.astype(np.float32)
    t, su, sv = _dev(lin, gpu)
    got = C.exl3_gemm(torch.from_numpy(x).to(gpu).bfloat16(), t, su, sv, K, cb == 1, codebook=cb,
                      out_dtype=torch.float32, bias=torch.from_numpy(bias).to(gpu))
    assert rel_l2(got, want) <= TOL
    got16 = C.exl3_gemm(torch.from_numpy(x).to(gpu).bfloat16(), t, su, sv, K, cb == 1, codebook=cb)
    assert got16.dtype == torch.float16
    assert rel_l2(got16, want - bias.astype(np.float32)) <= TOL


def test_linear_config0_prefill_2048(gpu):
    """C0's weights (2048 x 2048, K4 MCG) at a 2048-row prefill."""
    lin = S.linear(0, 2048, 2048, 4)
    x = S.activations(21, 2048, 2048)
    want = O.gemv(x, O.dequant(lin["trellis"], lin["suh"], lin["svh"], 4, 1))
    t, su, sv = _dev(lin, gpu)
    got = C.exl3_gemm(torch.from_numpy(x).to(gpu).bfloat16(), t, su, sv, 4, True, out_dtype=torch.float32)
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("m", [4, 200])
def test_apply_exl3_linear_shards_bias(gpu, m):
    """Two EXL3 shards and a bf16 shard, concatenated along the output, cast
    to x's dtype, reshaped to x's leading dimensions, bias added last."""
    in_f = 256
    a, b = S.linear(61, in_f, 256, 3), S.linear(62, in_f, 128, 4)
    wb = torch.randn(128, in_f, device=gpu).bfloat16()
    layer = SimpleNamespace(
        _exl3_linears=[Exl3Linear(*_dev(a, gpu), 3, 1), Exl3Linear(*_dev(b, gpu), 4, 1), None],
        _exl3_linear_output_partition_sizes=[256, 128, 128], _exl3_linear_bf16_shards=[2],
        _exl3_bf16_weight=wb)
    x = torch.from_numpy(S.activations(63, m, in_f)).to(gpu).bfloat16().view(2, m // 2, in_f)
    bias = torch.randn(512, device=gpu).bfloat16()
    y = apply_exl3_linear(layer, x, bias)
    assert y.shape == (2, m // 2, 512) and y.dtype == torch.bfloat16
    x2 = x.reshape(m, in_f).float().cpu().numpy()
    want = np.concatenate([O.gemv(x2, O.dequant(a["trellis"], a["suh"], a["svh"], 3, 1)),
                           O.gemv(x2, O.dequant(b["trellis"], b["suh"], b["svh"], 4, 1)),
                           (x.reshape(m, in_f).float() @ wb.float().t()).cpu().numpy()], axis=1)
    want = want + bias.float().cpu().numpy()
    assert rel_l2(y.reshape(m, 512).float(), want) <= TOL + 4e-3  # bf16 output rounding
