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
def test_gemm_small_vs_oracle(gpu, gemv_policy, K, cb, m):
    lin = S.linear(3000 + 100 * K + 10 * cb + m, 384, 256, K)
    x = S.activations(7 + m, m, 384)
    w = O.dequant(lin["trellis"], lin["suh"], lin["svh"], K, cb)
    want = O.gemv(x, w)
    got = _run(lin, x, cb, gpu, torch.float32)
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("m", [1, 16])
def test_gemm_config0_full_size(gpu, gemv_policy, m):
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


@pytest.mark.parametrize("m,xdt", [(1, torch.bfloat16), (3, torch.float16), (4, torch.float32),
                                    (5, torch.bfloat16)])
def test_linear_raw_rows_vs_rotation_launch(gpu, gemv_policy, monkeypatch, m, xdt):
    """Up to 4 rows the linear GEMV rotates its own input blocks while staging
    them; EXL3_LINEAR_RAW=0 keeps the rotation launch.  Both against the
    oracle and each other, with a bias (5 rows always take the launch)."""
    in_f, out_f = 2048, 640
    lin = S.linear(4100 + m, in_f, out_f, 3)
    x = S.activations(9 + m, m, in_f)
    bias = np.random.default_rng(m).standard_normal(out_f).astype(np.float16)
    w = O.dequant(lin["trellis"], lin["suh"], lin["svh"], 3, 0)
    want = O.gemv(x, w) + bias.astype(np.float32)
    args = (torch.from_numpy(x).to(gpu).to(xdt), torch.from_numpy(lin["trellis"]).to(gpu),
            torch.from_numpy(lin["suh"]).to(gpu), torch.from_numpy(lin["svh"]).to(gpu), 3, False)
    b = torch.from_numpy(bias).to(gpu)
    raw = C.exl3_gemm(*args, codebook=0, out_dtype=torch.float32, bias=b)
    monkeypatch.setenv("EXL3_LINEAR_RAW", "0")
    img = C.exl3_gemm(*args, codebook=0, out_dtype=torch.float32, bias=b)
    torch.cuda.synchronize()
    assert rel_l2(raw, want) <= TOL and rel_l2(img, want) <= TOL
    assert rel_l2(raw, img.cpu().numpy()) <= TOL


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


def _batched_layer(gpu, seed, n, in_f, out_f, K):
    packs = [S.linear(seed + e, in_f, out_f, K) for e in range(n)]
    dev = [{k: torch.from_numpy(p[k]).to(gpu) for k in ("trellis", "suh", "svh")} for p in packs]
    tabs = [torch.tensor([d[k].data_ptr() for d in dev], dtype=torch.int64, device=gpu)
            for k in ("trellis", "suh", "svh")]
    return packs, dev, tabs


@pytest.mark.parametrize("K,cb,m", [(2, 1, 1), (3, 0, 5), (4, 2, 3)])
def test_gemv_batched_vs_oracle_and_sequential(gpu, gemv_policy, K, cb, m):
    # p2b_gemv_batched: entry i == exl3_gemv(x, W[idx_i]); repeated ids, and an
    # id outside the tables gives zeros (csrc/p2b_batched.cu:341-368)
    packs, dev, tabs = _batched_layer(gpu, 4000 + 10 * K + cb, 4, 512, 256, K)
    x = S.activations(40 + m, m, 512)
    xt = torch.from_numpy(x).to(gpu).half()
    idx = torch.tensor([3, 0, 3, 9, 1], dtype=torch.int32, device=gpu)
    got = C.p2b_gemv_batched(xt, *tabs, idx, K, cb == 1, codebook=cb, out_features=256)
    assert got.shape == (5, m, 256) and got.dtype == torch.float16
    assert torch.count_nonzero(got[3]) == 0
    for i, e in enumerate([3, 0, 3, None, 1]):
        if e is None:
            continue
        w = O.dequant(packs[e]["trellis"], packs[e]["suh"], packs[e]["svh"], K, cb)
        assert rel_l2(got[i], O.gemv(xt.float().cpu().numpy(), w)) <= TOL
        seq = C.exl3_gemm(xt, dev[e]["trellis"], dev[e]["suh"], dev[e]["svh"], K, cb == 1, codebook=cb)
        assert (got[i].float() - seq.float()).abs().max().item() <= 1e-3


def test_gemv_batched_reference_shape_and_split_path(gpu, gemv_policy):
    # the reference's test shape: 8 experts, K2 MCG, 4096 -> 2048, m = 1
    # (long input dimension: the split-K finisher path)
    packs, dev, tabs = _batched_layer(gpu, 5000, 8, 4096, 2048, 2)
    x = S.activations(50, 1, 4096)
    xt = torch.from_numpy(x).to(gpu).half()
    idx = torch.arange(8, dtype=torch.int64, device=gpu)
    got = C.p2b_gemv_batched(xt, *tabs, idx, 2, True)
    assert got.shape == (8, 1, 2048)
    for e in (0, 5, 7):
        w = O.dequant(packs[e]["trellis"], packs[e]["suh"], packs[e]["svh"], 2, 1)
        assert rel_l2(got[e], O.gemv(x, w)) <= TOL
    # graph replay with new activations matches eager launches
    out = torch.empty_like(got)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out.copy_(C.p2b_gemv_batched(xt, *tabs, idx, 2, True))
    for seed in (51, 52):
        xt.copy_(torch.from_numpy(S.activations(seed, 1, 4096)))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, C.p2b_gemv_batched(xt, *tabs, idx, 2, True))
