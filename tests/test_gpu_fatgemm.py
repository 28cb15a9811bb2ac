"""GPU parity of the prefill fat GEMM against the oracle's decoded tiles.

Reference semantics (csrc/exl3_fat_gemm.cu:65-197 of the reference):
out = had128(a @ Wq) * svh in fp32, a already input-rotated.  The check is a
float64 product over the oracle's decoded tiles; tolerance relative L2 <= 2e-3
(fp16 a and weights are exact inputs, so the error is fp32 accumulation only)."""

import numpy as np
import pytest
import torch

import oracle as O
from moe_util import rel_l2
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _want(a16: np.ndarray, lin: dict, cb: int) -> np.ndarray:
    wq = O.decode_tiles(lin["trellis"], lin["K"], cb).astype(np.float64)
    z = a16.astype(np.float64) @ wq
    return O.block_hadamard(z, axis=-1) * lin["svh"].astype(np.float64)


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("cb", [0, 1, 2])
@pytest.mark.parametrize("M,kin,n", [(1, 256, 128), (17, 384, 384), (256, 256, 256), (300, 128, 512)])
def test_fat_gemm_vs_oracle(gpu, K, cb, M, kin, n):
    lin = S.linear(500 + 7 * K + cb + M, kin, n, K)
    a16 = S.activations(M + K, M, kin).astype(np.float16)
    want = _want(a16, lin, cb)
    out = torch.full((M, n), float("nan"), dtype=torch.float32, device=gpu)
    C.exl3_fat_gemm(torch.from_numpy(a16).to(gpu), torch.from_numpy(lin["trellis"]).to(gpu), out,
                    torch.from_numpy(lin["svh"]).to(gpu), K, cb == 1, cb == 2)
    assert rel_l2(out, want) <= TOL


def test_fat_gemm_large_m_deterministic(gpu):
    # several row tiles and both column-tile shapes
    lin = S.linear(77, 512, 640, 4)
    a16 = S.activations(3, 700, 512).astype(np.float16)
    want = _want(a16, lin, 1)
    a = torch.from_numpy(a16).to(gpu)
    t = torch.from_numpy(lin["trellis"]).to(gpu)
    sv = torch.from_numpy(lin["svh"]).to(gpu)
    out1 = torch.empty((700, 640), dtype=torch.float32, device=gpu)
    out2 = torch.empty_like(out1)
    C.exl3_fat_gemm(a, t, out1, sv, 4, True, False)
    C.exl3_fat_gemm(a, t, out2, sv, 4, True, False)
    assert torch.equal(out1, out2)
    assert rel_l2(out1, want) <= TOL


@pytest.mark.parametrize("K,cb", [(2, 0), (3, 1), (4, 2)])
def test_fat_gemm_helper_waves_bit_exact(gpu, monkeypatch, K, cb):
    """Row tiles of at most 128 rows let the second row half's MFMA waves
    decode half of each B tile (EXL3_FAT_HELPERS=0: the producers decode it
    all); the decoded values, and so the outputs, are the same bit for bit.
    700 rows: two full tiles, one of 188 rows and a last tile of 0..128-row
    sizes across the grid of column tiles."""
    M, kin, n = 700, 384, 640
    lin = S.linear(90 + K, kin, n, K)
    a16 = S.activations(6, M, kin).astype(np.float16)
    a = torch.from_numpy(a16).to(gpu)
    t = torch.from_numpy(lin["trellis"]).to(gpu)
    sv = torch.from_numpy(lin["svh"]).to(gpu)
    outs = []
    for helpers in ("1", "0"):
        monkeypatch.setenv("EXL3_FAT_HELPERS", helpers)
        for m in (700, 100, 33):
            o = torch.empty((m, n), dtype=torch.float32, device=gpu)
            C.exl3_fat_gemm(a[:m].contiguous(), t, o, sv, K, cb == 1, cb == 2)
            outs.append(o)
    torch.cuda.synchronize()
    for x, y in zip(outs[:3], outs[3:]):
        assert torch.equal(x, y)
    assert rel_l2(outs[0], _want(a16, lin, cb)) <= TOL


def test_fat_gemm_scatter(gpu):
    M, kin, n, T = 40, 256, 256, 64
    lin = S.linear(88, kin, n, 3)
    a16 = S.activations(4, M, kin).astype(np.float16)
    g = np.random.default_rng(5)
    tok = g.permutation(T)[:M].astype(np.int64)
    rw = g.uniform(0.1, 1.0, M).astype(np.float16)
    base = g.standard_normal((T, n)).astype(np.float32)
    want = base.astype(np.float64).copy()
    want[tok] += rw.astype(np.float64)[:, None] * _want(a16, lin, 1)
    out = torch.from_numpy(base).to(gpu)
    C.exl3_fat_gemm_scatter(torch.from_numpy(a16).to(gpu), torch.from_numpy(lin["trellis"]).to(gpu),
                            out, torch.from_numpy(lin["svh"]).to(gpu),
                            torch.from_numpy(tok).to(gpu), torch.from_numpy(rw).to(gpu), 3, True, False)
    assert rel_l2(out, want) <= 1e-4 + TOL * 0.1


def test_fat_gemm_is_the_dequant_product(gpu):
    # a = had(x * suh) makes the fat GEMM equal x @ dequant(W) (the reference's
    # prefill path applies had_r_128 to x before exl3_fat_gemm)
    lin = S.linear(99, 256, 256, 4)
    x = S.activations(6, 8, 256)
    xr = O.block_hadamard(x.astype(np.float16).astype(np.float64) * lin["suh"].astype(np.float64))
    a16 = xr.astype(np.float16)
    out = torch.empty((8, 256), dtype=torch.float32, device=gpu)
    C.exl3_fat_gemm(torch.from_numpy(a16).to(gpu), torch.from_numpy(lin["trellis"]).to(gpu), out,
                    torch.from_numpy(lin["svh"]).to(gpu), 4, True, False)
    want = O.gemv(x, O.dequant(lin["trellis"], lin["suh"], lin["svh"], 4, 1))
    assert rel_l2(out, want) <= TOL


@pytest.mark.parametrize("bad,match", [("K", "K in"), ("dtype", "float16"), ("width", "divisible by 128"),
                                       ("out", "float32")])
def test_fat_gemm_rejects_bad_arguments(gpu, bad, match):
    a = torch.zeros((4, 256), dtype=torch.float16, device=gpu)
    t = torch.zeros((16, 16, 64), dtype=torch.int16, device=gpu)
    sv = torch.ones(256, dtype=torch.float16, device=gpu)
    out = torch.zeros((4, 256), dtype=torch.float32, device=gpu)
    K = 4
    if bad == "K":
        K = 5
    elif bad == "dtype":
        a = a.float()
    elif bad == "width":
        t = torch.zeros((16, 5, 64), dtype=torch.int16, device=gpu)
        sv = torch.ones(80, dtype=torch.float16, device=gpu)
        out = torch.zeros((4, 80), dtype=torch.float32, device=gpu)
    else:
        out = out.half()
    with pytest.raises(RuntimeError, match=match):
        C.exl3_fat_gemm(a, t, out, sv, K, True, False)
