"""Pins of the NVFP4 KV oracle (oracle/nvfp4.py) on the CPU.

* the reference's own vectors and properties (tests/test_minimax_q4kv.py:
  113-239 and :1665-1710 of the reference): pool arithmetic, scale offsets,
  e2m1 ladder, RZ product properties, round-trip bound, byte-exact repack;
* the e4m3 encoder against torch's float8_e4m3fn cast (a library routine);
* byte fixtures written by the reference's own packer
  (tests/golden/make_nvfp4_vectors.py) incl. ties, RZ boundaries,
  saturation, clamped and zero groups.
"""

import pathlib

import numpy as np
import torch

import nvfp4 as N

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "nvfp4_pack_vectors.npz"


def test_pool_arithmetic_and_scale_offsets():
    assert N.ROW_BYTES == 72 and N.SLOT_REGION == 9216 and N.DATA_REGION == 8192
    assert 2 * 4 * N.PAGE_TOKENS * N.ROW_BYTES == 73728      # one page of 4 KV heads
    assert 2 * 4 * N.ROW_BYTES == 576                        # bytes per token of 4 KV heads
    for t in (0, 5, 127):
        for g in (0, 3, 7):
            assert N.scale_offset(0, t, g) == t * 8 + g
    assert N.scale_offset(1, 0, 0) == 0
    assert N.scale_offset(1, 1, 0) == 1
    assert N.scale_offset(1, 0, 1) == 4
    assert N.scale_offset(1, 7, 3) == (4 + 1) * 8 + 1 * 4 + 3
    t, g = np.meshgrid(np.arange(128), np.arange(8), indexing="ij")
    for side in (0, 1):
        off = N.scale_offset(side, t, g).reshape(-1)
        assert np.array_equal(np.sort(off), np.arange(1024))


def test_e4m3_encoder_matches_torch_cast():
    vals = np.concatenate([
        np.linspace(-500, 500, 2001, dtype=np.float32),
        np.array([0.0, 1e-12, 2 ** -9, 2 ** -9 * 1.5, 2 ** -6, 0.5, 447.9, 448.0, 448.5, 450.0,
                  1e30, np.inf, -np.inf, -0.0], np.float32),
        np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 50,
        (np.random.default_rng(1).random(100000).astype(np.float32) * 2.0 ** -6),
    ])
    # torch's cast is the RNE conversion inside the finite range; on overflow
    # this torch build returns NaN where the reference's encoder (the
    # hardware cvt.rn.satfinite) saturates, so the two are compared below
    # the RNE overflow boundary 464 and saturation is checked on its own.
    fin = vals[np.abs(vals) < 464]
    ours = N.e4m3_encode(fin)
    cast = torch.from_numpy(fin).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, cast)
    over = np.array([464.0, 500.0, 1e30, np.inf, -470.0, -np.inf], np.float32)
    assert N.e4m3_encode(over).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert N.e4m3_encode(np.array([447.9, 463.9], np.float32)).tolist() == [0x7E, 0x7E]
    assert N.e4m3_encode(np.array([np.nan], np.float32))[0] == 0x7F
    # decode inverts encode on every finite code
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    assert np.array_equal(N.e4m3_encode(N.e4m3_decode(codes)), codes)
    assert np.array_equal(N.e4m3_decode(codes),
                          torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy())


def test_e2m1_ladder():
    vals = np.array(N.E2M1_VALUES, np.float32)
    assert N.e2m1_code(vals).tolist() == list(range(8))
    for n in range(16):
        mag = N.E2M1_VALUES[n & 7]
        assert float(N.e2m1_decode(n)) == (-mag if n & 8 else mag)
    assert int(N.e2m1_code(0.26)) == 1 and int(N.e2m1_code(0.24)) == 0
    # the tie rules: lower midpoints stay down, upper midpoints move up
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    assert N.e2m1_code(mids).tolist() == [0, 2, 2, 4, 4, 6, 6]
    assert int(N.e2m1_code(np.float32(100))) == 7 and int(N.e2m1_code(np.float32(np.nan))) == 7


def test_rz_product_is_true_rz():
    g = np.random.default_rng(0)
    x = (g.standard_normal((4096, 16)) * 3).astype(np.float32)
    c = (g.random((4096, 16)) * 4 + 0.5).astype(np.float32)
    rz = N.rz_product(x, c)
    rn = (x * c).astype(np.float32)
    exact = x.astype(np.float64) * c.astype(np.float64)
    assert ((rz.astype(np.float64) - exact) * np.sign(exact) <= 0).all()
    away = np.abs(rn.astype(np.float64)) > np.abs(exact)
    assert np.array_equal(rz == rn, ~away)
    assert (rz != rn).sum() > 0 and ((rz != rn) & (exact < 0)).sum() > 0
    # |rz| is the largest fp32 magnitude not above |exact|
    nxt = np.nextafter(np.abs(rz), np.float32(np.inf)).astype(np.float64)
    assert (nxt > np.abs(exact)).all()


def test_pack_matches_reference_bytes():
    d = np.load(GOLDEN)
    rows = (d["rows_bf16"].astype(np.int32) << 16).astype(np.uint32).view(np.float32)
    data, scales = N.pack_row(rows)
    assert np.array_equal(data, d["data"]) and np.array_equal(scales, d["scales"])
    assert np.array_equal(N.pack_slot(rows[:128], 0), d["k_region"])
    assert np.array_equal(N.pack_slot(rows[:128], 1), d["v_region"])


def test_roundtrip_bound_and_byte_exact_repack():
    x = N.bf16_round(np.random.default_rng(1).standard_normal((256, 128)).astype(np.float32))
    data, sc = N.pack_row(x)
    back = N.unpack_row(data, sc)
    scale = np.repeat(N.e4m3_decode(sc), 16, axis=-1)
    assert (np.abs(back - x) <= scale * 1.0 + 1e-9).all()
    data2, sc2 = N.pack_row(back)
    assert np.array_equal(data, data2) and np.array_equal(sc, sc2)
    for side in (0, 1):
        flat = N.pack_slot(x[:128], side)
        assert np.array_equal(N.pack_slot(N.unpack_slot(flat, side), side), flat)


def test_pack_pages_places_tokens_and_sparse_attention_closed_form():
    g = np.random.default_rng(2)
    B, H, L = 2, 2, 300
    k = N.bf16_round(g.standard_normal((B, H, L, 128)).astype(np.float32))
    v = N.bf16_round(g.standard_normal((B, H, L, 128)).astype(np.float32))
    seq = np.array([300, 129], np.int32)
    bt = np.array([[4, 0, 2], [1, 3, 5]], np.int32)
    pool = N.pack_pages(k, v, seq, bt, 6)
    vals = N.dequant_pool(pool)
    # token 200 of sequence 0, head 1 = slot 72 of page bt[0, 1] = 0
    d, s = N.pack_row(k[0, 1, 200])
    assert np.array_equal(pool[0, 2][72 * 64:73 * 64], d)
    assert np.allclose(vals[0, 3, 72], N.unpack_row(*N.pack_row(v[0, 1, 200])))
    # slots past a sequence's end stay zero
    assert not pool[3, :, 1 * 64:128 * 64].any()
    # identical keys -> output is the mean of the visible values
    q = g.standard_normal((2, 4, 128))
    kv = vals.copy()
    kv[:, 0::2] = kv[0, 0, 0]
    topk = np.array([[[0, 2, -1], [1, -1, 7]], [[2, 0, 1], [0, 1, -1]]])  # [Hkv, total_q, topk]
    out = N.sparse_decode(q, kv, topk, bt, seq, 1, 0.1)
    # query 0 (seq 300, pos 299), head 0: blocks {0, 2}: tokens 0..127 and 256..299
    want = np.concatenate([kv[4, 1, :128], kv[2, 1, :44]]).mean(axis=0)
    assert np.allclose(out[0, 0], want) and np.allclose(out[0, 1], want)
    # query 1 (seq 129, pos 128), head 1: blocks {0, 1}; block 1 holds one token
    want = np.concatenate([kv[1, 3, :128], kv[3, 3, :1]]).mean(axis=0)
    assert np.allclose(out[1, 2], want)
