"""GPU parity of the streaming decode GEMV/GEMM against dequant + fp32 matmul.

Tolerance: relative L2 <= 2e-3 (the target's floating-point bar)."""

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import rel_l2
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _run(lin, x, cb, gpu, out_dtype=torch.float16):
    return C.exl3_gemm(torch.from_numpy(x).to(gpu).to(torch.bfloat16),
                       torch.from_numpy(lin["trellis"]).to(gpu),
                       torch.from_numpy(lin["suh"]).to(gpu),
                       torch.from_numpy(lin["svh"]).to(gpu), lin["K"], cb == 1, codebook=cb,
                       out_dtype=out_dtype)


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("m", [1, 3, 16, 21])
def test_gemm_small_vs_oracle(gpu, K, cb, m):
    lin = S.linear(3000 + 100 * K + 10 * cb + m, 384, 256, K)
    x = S.activations(7 + m, m, 384)
    w = O.dequant(lin["trellis"], lin["suh"], lin["svh"], K, cb)
    want = O.gemv(x, w)
    got = _run(lin, x, cb, gpu, torch.float32)
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("m", [1, 16])
def test_gemm_config0_full_size(gpu, m):
    # in=out=2048, K4, MCG, bf16 activations, m in {1, 16}
    lin = S.linear(0, 2048, 2048, 4)
    x = S.activations(1, m, 2048)
    w = O.dequant(lin["trellis"], lin["suh"], lin["svh"], 4, 1)
    want = O.gemv(x, w)
    got = _run(lin, x, 1, gpu, torch.float32)
    assert rel_l2(got, want) <= TOL
    # fp16 output path agrees with the fp32 one to fp16 rounding
    got16 = _run(lin, x, 1, gpu, torch.float16)
    assert rel_l2(got16, want) <= TOL


def test_exl3_gemv_contract(gpu):
    lin = S.linear(11, 256, 256, 3)
    x = torch.from_numpy(S.activations(2, 4, 256)).to(gpu).half()
    t = torch.from_numpy(lin["trellis"]).to(gpu)
    su, sv = torch.from_numpy(lin["suh"]).to(gpu), torch.from_numpy(lin["svh"]).to(gpu)
    y = C.exl3_gemv(x, t, su, sv, 3, True)
    assert y.dtype == torch.float16 and y.shape == (4, 256)
    w = O.dequant(lin["trellis"], lin["suh"], lin["svh"], 3, 1)
    assert rel_l2(y, O.gemv(x.float().cpu().numpy(), w)) <= TOL
    with pytest.raises(RuntimeError, match="1 <= m <= 8"):
        C.exl3_gemv(x.repeat(3, 1), t, su, sv, 3, True)
    with pytest.raises(RuntimeError, match="does not match trellis"):
        C.exl3_gemv(x[:, :128], t, su, sv, 3, True)


def test_gemm_deterministic(gpu):
    lin = S.linear(12, 1024, 512, 2)
    x = S.activations(3, 2, 1024)
    a = _run(lin, x, 1, gpu, torch.float32)
    b = _run(lin, x, 1, gpu, torch.float32)
    assert torch.equal(a, b)
