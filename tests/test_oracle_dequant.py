"""CPU checks that pin the dequant oracle (oracle/exl3_oracle.c).

Pins: the reference's own golden vectors (tests/test_dequant_parity.py of the
reference), the reference's compiled primitives (oracle/_ref, built from
csrc/exl3_dequant.cuh where it lies) and its whole dequant_cpu
(csrc/bindings.cpp:15-100, compiled in place by oracle/ref_dequant_harness.cpp),
numpy's IEEE casts, and closed forms of the Hadamard composition.
"""

import ctypes
import math
import pathlib

import numpy as np
import pytest

import oracle as O

ROOT = pathlib.Path(__file__).resolve().parent.parent
REF_SO = ROOT / "oracle" / "_ref" / "libexl3_ref.so"


@pytest.fixture(scope="module")
def ref():
    if not REF_SO.exists():
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    lib = ctypes.CDLL(str(REF_SO))
    lib.ref_decode_codebook_bits.restype = ctypes.c_uint16
    lib.ref_decode_codebook_bits.argtypes = [ctypes.c_uint16, ctypes.c_int]
    lib.ref_read_window.restype = ctypes.c_uint16
    lib.ref_read_window.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t]
    lib.ref_hadamard.restype = None
    lib.ref_hadamard.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.ref_float_to_half_bits.restype = ctypes.c_uint16
    lib.ref_float_to_half_bits.argtypes = [ctypes.c_float]
    return lib


# Reference golden vectors: tests/test_dequant_parity.py:18-35
@pytest.mark.parametrize(("value", "expected"), [
    (2**-15, 0x0200), (1.00075, 0x3C01), (-1.00075, 0xBC01), (2**-24, 0x0001),
    (2**-25, 0x0000), (1.0 + 2**-11, 0x3C00), (1.0 + 3 * 2**-11, 0x3C02),
    (65504.0, 0x7BFF), (65520.0, 0x7C00), (0.0, 0x0000), (-0.0, 0x8000),
    (math.inf, 0x7C00), (-math.inf, 0xFC00)])
def test_f32_to_f16_golden(value, expected):
    assert O.lib().oc_f32_to_f16(value) == expected


def test_f32_to_f16_nan_is_quiet():
    b = O.lib().oc_f32_to_f16(float("nan"))
    assert (b & 0x7C00) == 0x7C00 and (b & 0x3FF)


def test_f16_roundtrip_all_patterns_vs_numpy():
    L = O.lib()
    pats = np.arange(65536, dtype=np.uint32)
    ref = pats.astype(np.uint16).view(np.float16).astype(np.float32)
    mine = np.array([L.oc_f16_to_f32(int(p)) for p in pats], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(mine[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(mine[~finite & np.isnan(ref)]).all()


def test_f32_to_f16_random_vs_numpy():
    L = O.lib()
    g = np.random.default_rng(1)
    # values across the binary16 range incl. subnormals, ties and overflow
    v = np.concatenate([
        g.standard_normal(4000).astype(np.float32) * np.float32(2.0) ** g.integers(-26, 17, 4000).astype(np.float32),
        (np.arange(0, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),  # subnormal ties
        np.float32(1.0) + (np.arange(0, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10),  # normal ties
    ]).astype(np.float32)
    mine = np.array([L.oc_f32_to_f16(float(x)) for x in v], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(mine, want)


# Reference golden vectors: tests/test_dequant_parity.py:84-104
@pytest.mark.parametrize(("window", "mcg_bits", "mul1_bits"), [
    (0x0000, 0x3F60, 0xC2E8), (0x0001, 0x304E, 0x3921), (0x1234, 0x3E0F, 0xB89E),
    (0x7FFF, 0x4172, 0x3FCA), (0xFFFF, 0x3ACD, 0xB936)])
def test_codebook_golden(window, mcg_bits, mul1_bits):
    assert O.decode_codebook(window, 1) == mcg_bits
    assert O.decode_codebook(window, 2) == mul1_bits


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_all_windows_vs_reference(ref, cb):
    mine = O.decode_codebook_table(cb)
    theirs = np.array([ref.ref_decode_codebook_bits(w, cb) for w in range(65536)], dtype=np.uint16)
    assert np.array_equal(mine, theirs)


def test_codebook_closed_form_3inst():
    # 3INST from its definition in float64: each masked half has exponent
    # 12..15, so the fp32 sum is exact and one fp16 rounding gives the weight.
    for w in range(0, 65536, 97):
        x = (w * 89226354 + 64248484) & 0xFFFFFFFF
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        lo = np.array([x & 0xFFFF], dtype=np.uint16).view(np.float16)[0]
        hi = np.array([x >> 16], dtype=np.uint16).view(np.float16)[0]
        want = np.float16(float(lo) + float(hi)).view(np.uint16)
        assert O.decode_codebook(w, 0) == want


@pytest.mark.parametrize("K", [2, 3, 4, 8])
def test_read_window_all_positions_vs_reference(ref, K):
    g = np.random.default_rng(K)
    tile = g.integers(0, 65536, size=16 * K, dtype=np.uint16)
    for bit in range(256 * K):
        assert O.read_window(tile, K, bit) == ref.ref_read_window(tile.ctypes.data, 16 * K, bit)


@pytest.mark.parametrize("K", [2, 3, 4])
def test_read_window_brute_force_bits(K):
    # Independent spelling: list the stream bits MSB-first per uint32 word.
    g = np.random.default_rng(10 + K)
    tile = g.integers(0, 65536, size=16 * K, dtype=np.uint16)
    words = tile[0::2].astype(np.uint64) | (tile[1::2].astype(np.uint64) << 16)
    stream = [(int(w) >> (31 - b)) & 1 for w in words for b in range(32)]
    n = len(stream)
    for bit in range(0, n, 7):
        want = 0
        for j in range(16):
            want = (want << 1) | stream[(bit + j) % n]
        assert O.read_window(tile, K, bit) == want


def test_tile_positions_bijective_and_match_swizzle_loop():
    r1, c1 = O.tile_positions()
    r2, c2 = O.tile_positions_loop()
    assert np.array_equal(r1, r2) and np.array_equal(c1, c2)
    assert len(set(zip(r1.tolist(), c1.tolist()))) == 256


def test_hadamard_vs_reference_and_closed_form(ref):
    g = np.random.default_rng(3)
    for _ in range(20):
        v = g.standard_normal(128).astype(np.float32)
        a = O.hadamard_f32(v)
        b = v.copy()
        ref.ref_hadamard(b.ctypes.data, 128)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        np.testing.assert_allclose(a, O.hadamard_matrix(128) @ v.astype(np.float64), rtol=1e-5, atol=1e-4)
    h = O.hadamard_matrix(128)
    assert np.array_equal(h @ h, 128 * np.eye(128))


REF_DEQUANT_SO = ROOT / "oracle" / "_ref" / "libref_dequant.so"


@pytest.fixture(scope="module")
def ref_dequant():
    """The reference's own dequant_cpu (csrc/bindings.cpp:15-100), compiled in
    place by oracle/Makefile (oracle/ref_dequant_harness.cpp)."""
    if not REF_DEQUANT_SO.exists():
        pytest.skip("oracle/_ref/libref_dequant.so not built (reference checkout absent)")
    import os

    import torch  # noqa: F401  (the harness links libtorch)

    lib = ctypes.CDLL(str(REF_DEQUANT_SO), mode=os.RTLD_LAZY)
    fn = lib.ref_dequant_cpu
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                   ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return fn


@pytest.mark.parametrize("K,cb", [(2, 1), (3, 2), (4, 1), (4, 2), (8, 1), (1, 2)])
def test_dequant_bit_exact_vs_reference_dequant_cpu(ref_dequant, K, cb):
    """The whole composition (window read, codebook, swizzle, both Hadamard
    passes, suh/svh, fp16 rounding) against the reference's own dequant_cpu:
    bit for bit (MCG and mul1, the codebooks its mcg flag reaches)."""
    g = np.random.default_rng(200 + K * 3 + cb)
    tk, tn = 16, 24  # 256 x 384
    t = g.integers(0, 65536, size=(tk, tn, 16 * K), dtype=np.uint16).view(np.int16)
    su = np.where(g.random(tk * 16) < 0.5, -1.0, 1.0).astype(np.float16)
    sv = (np.where(g.random(tn * 16) < 0.5, -1.0, 1.0) * g.uniform(0.005, 0.02, tn * 16)).astype(np.float16)
    out = np.zeros((tk * 16, tn * 16), np.uint16)
    assert ref_dequant(t.ctypes.data, tk, tn, su.ctypes.data, sv.ctypes.data, K, 1 if cb == 1 else 0,
                       out.ctypes.data) == 0
    w = O.dequant(t, su, sv, K, cb)
    assert np.array_equal(out, np.asarray(w, np.float16).view(np.uint16))


def test_reference_dequant_catches_a_reordered_composition(ref_dequant):
    """A plausible mistake -- the scales applied before the second Hadamard
    pass instead of after -- stays within an ulp of the float64 form but is
    not bit-identical to the reference."""
    g = np.random.default_rng(9)
    t = g.integers(0, 65536, size=(8, 8, 64), dtype=np.uint16).view(np.int16)
    su = (np.where(g.random(128) < 0.5, -1.0, 1.0) * g.uniform(0.5, 2.0, 128)).astype(np.float16)
    sv = (np.where(g.random(128) < 0.5, -1.0, 1.0) * g.uniform(0.005, 0.02, 128)).astype(np.float16)
    out = np.zeros((128, 128), np.uint16)
    ref_dequant(t.ctypes.data, 8, 8, su.ctypes.data, sv.ctypes.data, 4, 1, out.ctypes.data)
    q = O.decode_tiles(t, 4, 1).astype(np.float32)
    norm = np.float32(0.088388347648)
    a = O.block_hadamard(q * su.astype(np.float32)[:, None], axis=1).astype(np.float32) * norm
    wrong = (O.block_hadamard(a, axis=0).astype(np.float32) * norm * sv.astype(np.float32)[None, :])
    assert not np.array_equal(out, wrong.astype(np.float16).view(np.uint16))
    assert np.array_equal(out, np.asarray(O.dequant(t, su, sv, 4, 1), np.float16).view(np.uint16))


@pytest.mark.parametrize("K,cb", [(2, 1), (3, 0), (4, 1), (4, 2), (8, 1)])
def test_dequant_matches_float64_composition(K, cb):
    g = np.random.default_rng(100 + K * 3 + cb)
    tk, tn = 16, 16  # 256 x 256
    t = g.integers(0, 65536, size=(tk, tn, 16 * K), dtype=np.uint16).view(np.int16)
    su = np.where(g.random(256) < 0.5, -1.0, 1.0).astype(np.float16)
    sv = (np.where(g.random(256) < 0.5, -1.0, 1.0) * g.uniform(0.005, 0.02, 256)).astype(np.float16)
    w = O.dequant(t, su, sv, K, cb).astype(np.float64)
    q = O.decode_tiles(t, K, cb).astype(np.float64)
    # W = diag(suh) H Wq H diag(svh) / 128, blockwise
    want = O.block_hadamard(O.block_hadamard(q, axis=1), axis=0)
    want = want * su.astype(np.float64)[:, None] * sv.astype(np.float64)[None, :]
    ulp = np.abs(want.astype(np.float16).astype(np.float64) - np.nextafter(
        want.astype(np.float16), np.float16(np.inf)).astype(np.float64))
    assert (np.abs(w - want) <= ulp + 1e-12).all()


def test_dequant_unit_scales_round_trip():
    # With suh = svh = 1: H W H / 128 applied twice returns Wq (within fp16).
    g = np.random.default_rng(7)
    t = g.integers(0, 65536, size=(8, 8, 64), dtype=np.uint16).view(np.int16)
    ones = np.ones(128, dtype=np.float16)
    w = O.dequant(t, ones, ones, 4, 1).astype(np.float64)
    back = O.block_hadamard(O.block_hadamard(w, axis=1), axis=0)
    q = O.decode_tiles(t, 4, 1).astype(np.float64)
    np.testing.assert_allclose(back, q, atol=2e-2, rtol=0)
    assert np.abs(back - q).mean() < 2e-3


def test_dequant_constant_tile_is_single_spike():
    # All-zero trellis decodes every weight to codebook(window 0): a constant
    # block, whose 2-D Hadamard is one non-zero entry per 128x128 block.
    t = np.zeros((8, 8, 16 * 4), dtype=np.int16)
    ones = np.ones(128, dtype=np.float16)
    w = O.dequant(t, ones, ones, 4, 1).astype(np.float64)
    c = float(np.array([O.decode_codebook(0, 1)], dtype=np.uint16).view(np.float16)[0])
    assert np.count_nonzero(w) == 1
    assert w[0, 0] == pytest.approx(c * 128.0 * 128.0 / 128.0, rel=1e-3)


# ---------------------------------------------------------------------------
# n-gram embedding rows (mul1 ring bitstream)
# ---------------------------------------------------------------------------

def _ring_pack(vals: np.ndarray, bits: int, scale: float) -> np.ndarray:
    """Packed row from 160 K-bit ring values: value p occupies stream bits
    [p K, p K + K), LSB-first in the int16 words after the fp16 scale word."""
    n_words = O.ngram_words_per_row(bits)
    stream = np.zeros(16 * (n_words - 1), np.uint8)
    for p, v in enumerate(vals):
        for b in range(bits):
            stream[p * bits + b] = (int(v) >> b) & 1
    words = (stream.reshape(-1, 16).astype(np.uint32) << np.arange(16)).sum(-1)
    row = np.zeros(n_words, np.uint16)
    row[0] = np.float16(scale).view(np.uint16)
    row[1:] = words
    return row.view(np.int16)


def test_ngram_words_per_row_reference_vectors():
    # tests/test_native_pack_unit.py:27-29 of the reference
    assert O.ngram_words_per_row(5) == 51 and O.ngram_words_per_row(3) == 31


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 8])
def test_ngram_state_is_the_ring_of_k_bit_values(bits):
    g = np.random.default_rng(bits)
    vals = g.integers(0, 1 << bits, 160)
    row = _ring_pack(vals, bits, 1.0)
    out = O.ngram_dequant_rows(row[None], bits, np.zeros(1, np.int64), np.zeros((1, 160), np.float16))
    # state of element i: K-bit group j holds ring value (i - j) mod 160
    groups = (16 + bits - 1) // bits
    for i in (0, 1, 7, 80, 159):
        st = 0
        for j in range(groups):
            st |= int(vals[(i - j) % 160]) << (j * bits)
        st &= 0xFFFF
        assert out[0, i].view(np.uint16) == O.decode_codebook(st, 2)


def test_ngram_scale_and_bias():
    g = np.random.default_rng(11)
    bits = 4
    rows = np.stack([_ring_pack(g.integers(0, 16, 160), bits, s) for s in (0.5, -4.0, 0.0078125)])
    hb = g.standard_normal((3, 160)).astype(np.float16)
    heads = np.array([2, 0, 1])
    got = O.ngram_dequant_rows(rows, bits, heads, hb).astype(np.float64)
    base = O.ngram_dequant_rows(rows, bits, np.zeros(3, np.int64), np.zeros((1, 160), np.float16))
    scales = np.array([0.5, -4.0, 0.0078125])[:, None]
    # base = fp16(cb * scale): exact in fp16 for power-of-two scales
    cb = base.astype(np.float64) / scales
    want = cb * scales + hb[heads].astype(np.float64)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -10 + 2.0 ** -24)
