"""GPU parity: the HIP trellis decode / dequant is bit-exact with the oracle."""

import numpy as np
import pytest
import torch

import oracle as O
from vllm_exl3_amd import synthetic as S
from vllm_exl3_amd import vllm_exl3_c as C

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("K", [2, 3, 4, 8])
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_dequant_bit_exact(gpu, K, cb):
    lin = S.linear(1000 + 10 * K + cb, 256, 384, K)
    want = O.dequant(lin["trellis"], lin["suh"], lin["svh"], K, cb)
    t = torch.from_numpy(lin["trellis"]).to(gpu)
    su = torch.from_numpy(lin["suh"]).to(gpu)
    sv = torch.from_numpy(lin["svh"]).to(gpu)
    got = C.dequant_trellis(t, su, sv, K, cb == 1, codebook=cb)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_decode_tiles_bit_exact(gpu, K, cb):
    lin = S.linear(2000 + 10 * K + cb, 64, 96, K)
    want = O.decode_tiles(lin["trellis"], K, cb).astype(np.float16)
    got = C.decode_tiles(torch.from_numpy(lin["trellis"]).to(gpu), K, cb == 1, codebook=cb)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))


def test_dequant_config0_full_size(gpu):
    # 2048x2048, K4, MCG
    lin = S.linear(0, 2048, 2048, 4)
    want = O.dequant(lin["trellis"], lin["suh"], lin["svh"], 4, 1)
    got = C.dequant_trellis(torch.from_numpy(lin["trellis"]).to(gpu),
                            torch.from_numpy(lin["suh"]).to(gpu),
                            torch.from_numpy(lin["svh"]).to(gpu), 4, True)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))


def test_dequant_host_tensors_round_trip_through_device(gpu):
    lin = S.linear(5, 128, 128, 3)
    got = C.dequant_trellis(torch.from_numpy(lin["trellis"]), torch.from_numpy(lin["suh"]),
                            torch.from_numpy(lin["svh"]), 3, True)
    assert got.device.type == "cpu"
    want = O.dequant(lin["trellis"], lin["suh"], lin["svh"], 3, 1)
    assert np.array_equal(got.numpy().view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("bad,match", [
    ("K", "K must be one of"), ("dtype", "trellis must be int16"), ("last", "16\\*K"),
    ("scale_dtype", "float16"), ("short", "too short")])
def test_dequant_rejects_bad_arguments(gpu, bad, match):
    t = torch.zeros((8, 8, 64), dtype=torch.int16, device=gpu)
    su = torch.ones(128, dtype=torch.float16, device=gpu)
    sv = torch.ones(128, dtype=torch.float16, device=gpu)
    K = 4
    if bad == "K":
        K = 5
    elif bad == "dtype":
        t = t.to(torch.int32)
    elif bad == "last":
        t = torch.zeros((8, 8, 48), dtype=torch.int16, device=gpu)
    elif bad == "scale_dtype":
        su = su.float()
    else:
        su = su[:64]
    with pytest.raises(RuntimeError, match=match):
        C.dequant_trellis(t, su, sv, K, True)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_ngram_rows_bit_exact(gpu, bits):
    g = np.random.default_rng(40 + bits)
    n, words = 257, O.ngram_words_per_row(bits)
    packed = g.integers(-32768, 32768, (n, words + 3)).astype(np.int16)  # padded row stride
    packed[:, 0] = g.uniform(-2, 2, n).astype(np.float16).view(np.int16)
    hb = g.standard_normal((5, 160)).astype(np.float16)
    heads = g.integers(0, 5, n)
    want = O.ngram_dequant_rows(packed[:, :words], bits, heads, hb)
    got = C.ngram_dequant_rows(torch.from_numpy(packed).to(gpu)[:, :], bits,
                               torch.from_numpy(heads).to(gpu), torch.from_numpy(hb).to(gpu))
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))
