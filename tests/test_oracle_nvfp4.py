"""Pins of the NVFP4 KV oracle (oracle/nvfp4.py) on the CPU.

* the reference's own vectors and properties (tests/test_minimax_q4kv.py:
  113-239 and :1665-1710 of the reference): pool arithmetic, scale offsets,
  e2m1 ladder, RZ product properties, round-trip bound, byte-exact repack;
* the e4m3 encoder against torch's float8_e4m3fn cast (a library routine);
* byte fixtures written by the reference's own packer
  (tests/golden/make_nvfp4_vectors.py) incl. ties, RZ boundaries,
  saturation, clamped and zero groups;
* the prefill staging rows: exactness of every e2m1 x e4m3 product in bf16
  (all 16 x 256 codes), the identity on rows the format holds exactly
  (pack -> stage gives the rows back, K and V halves), the zero row and the
  reference test's layout (tests/test_minimax_q4kv.py:560-581 of the
  reference).
"""

import pathlib

import numpy as np
import pytest
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


# ---------------------------------------------------------------------------
# W1 write side (Gemma norm + partial NeoX RoPE + q4 pack-insert)
# ---------------------------------------------------------------------------

W1_NQ, W1_NKV, W1_NIQ, W1_ROT = 8, 4, 4, 64  # the reference test's branch layout


def w1_batch(num_tokens=5, seed=4):
    """Inputs shaped like the reference's _w1_batch (tests/test_minimax_q4kv.py:
    246-265): bf16 rows N(0, 0.25), N(0,1) norm weights and cos/sin rows,
    positions 3.., slots [0, 1, 130, -1, 257]."""
    g = np.random.default_rng(seed)
    width = (W1_NQ + 2 * W1_NKV + W1_NIQ + 1) * 128
    qkv = N.bf16_round((g.standard_normal((num_tokens, width)) * 0.5).astype(np.float32))
    ws = [g.standard_normal(128).astype(np.float32) for _ in range(4)]
    cos_sin = g.standard_normal((64, W1_ROT)).astype(np.float32)
    positions = np.arange(num_tokens, dtype=np.int64) + 3
    sm = np.array([0, 1, 130, -1, 257], dtype=np.int64)[:num_tokens]
    ism = np.array([0, 1, 2, -1, 4], dtype=np.int64)[:num_tokens]
    return qkv, ws, cos_sin, positions, 1e-4, sm, ism


def test_w1_sumsq_tree_matches_float64():
    x = np.random.default_rng(1).standard_normal((64, 128)).astype(np.float32)
    want = (x.astype(np.float64) ** 2).sum(-1)
    got = N.sumsq_tree(x).astype(np.float64)
    assert np.all(np.abs(got - want) <= 8 * np.finfo(np.float32).eps * want)
    # a dropped or doubled term would be far outside that bound
    assert N.sumsq_tree(np.ones((1, 128), np.float32))[0] == 128.0


def test_w1_gemma_rmsnorm_closed_form():
    g = np.random.default_rng(2)
    x = g.standard_normal((32, 128)).astype(np.float32)
    w = g.standard_normal(128).astype(np.float32)
    eps = 1e-4
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps) * (1 + w.astype(np.float64))
    got = N.gemma_rmsnorm(x, w, eps).astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-7)
    # w = 0 gives unit RMS (up to eps)
    u = N.gemma_rmsnorm(x, np.zeros(128, np.float32), 0.0)
    assert np.allclose(np.sqrt((u.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-6)


@pytest.mark.parametrize("rot", [8, 64, 128])
def test_w1_rope_is_complex_rotation(rot):
    g = np.random.default_rng(3 + rot)
    x = g.standard_normal((16, 128)).astype(np.float32)
    th = g.uniform(-3, 3, (16, rot // 2))
    cs = np.concatenate([np.cos(th), np.sin(th)], -1).astype(np.float32)
    y = N.rope_partial_neox(x, cs, rot).astype(np.float64)
    h = rot // 2
    z = (x[:, :h] + 1j * x[:, h:rot]).astype(np.complex128) * (cs[:, :h] + 1j * cs[:, h:]).astype(np.complex128)
    assert np.allclose(y[:, :h], z.real, rtol=0, atol=2e-6 * np.abs(x).max())
    assert np.allclose(y[:, h:rot], z.imag, rtol=0, atol=2e-6 * np.abs(x).max())
    assert np.array_equal(y[:, rot:], x[:, rot:].astype(np.float64))  # pass-through dims
    # identity angle leaves the row unchanged bit for bit
    ident = np.concatenate([np.ones((16, h)), np.zeros((16, h))], -1).astype(np.float32)
    assert np.array_equal(N.rope_partial_neox(x, ident, rot), x)


def test_w1_e4m3_clamped():
    got = N.e4m3_clamped(np.array([np.nan, 1e9, -1e9, 448.0, 0.5, -0.0], np.float32))
    assert got.tolist() == [0xFE, 0x7E, 0xFE, 0x7E, 0x30, 0x80]


def test_w1_write_layout():
    # Mirrors test_reference_w1_write_layout (tests/test_minimax_q4kv.py:268-330).
    qkv, ws, cs, pos, eps, sm, ism = w1_batch()
    pool = np.zeros((3, 2 * W1_NKV, N.SLOT_REGION), np.uint8)  # sm max 257 -> page 2
    icache = np.zeros((5, 128), np.uint8)
    out = N.w1_write(qkv, *ws, cs, pos, eps, W1_ROT, W1_NQ, W1_NKV, W1_NIQ, sm, ism, pool, icache)
    assert out["q"].shape == (5, W1_NQ, 128) and out["index_q"].shape == (5, W1_NIQ, 128)
    x = qkv.reshape(5, -1, 128)
    csr = cs[pos]
    kn = N.rope_partial_neox(N.gemma_rmsnorm(x[:, W1_NQ:W1_NQ + W1_NKV], ws[1], eps), csr, W1_ROT)
    for i, s in enumerate(sm.tolist()):
        if s < 0:
            continue
        page, tok = s // 128, s % 128
        for h in range(W1_NKV):
            got_k = N.unpack_slot(pool[page, 2 * h], 0)[tok]
            got_v = N.unpack_slot(pool[page, 2 * h + 1], 1)[tok]
            assert np.array_equal(got_k, N.unpack_row(*N.pack_row(kn[i, h])))
            assert np.array_equal(got_v, N.unpack_row(*N.pack_row(x[i, W1_NQ + W1_NKV + h])))
    # unmapped tokens leave the pool zero at their data positions
    assert not pool[0, 0, 3 * 64:3 * 64 + 8].any()
    assert not icache[3].any()
    ikn = N.rope_partial_neox(N.gemma_rmsnorm(x[:, -1], ws[3], eps), csr, W1_ROT)
    assert np.array_equal(icache[[0, 1, 2, 4]], N.e4m3_clamped(ikn)[[0, 1, 2, 4]])


def test_stage_products_exact_in_bf16():
    """Every e2m1 x e4m3 product is a bf16 value: staging is a lossless cast."""
    e2 = N.e2m1_decode(np.arange(16))
    e4 = N.e4m3_decode(np.arange(256))
    prod = (e2[:, None] * e4[None, :]).astype(np.float32)
    bits = N.bf16_bits(prod)
    finite = np.isfinite(prod)
    back = (bits.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(back[finite].view(np.uint32), prod[finite].view(np.uint32))
    assert (bits[~finite] == 0x7FC0).all() and (~finite).sum() == 2 * 16


def _representable_rows(rng, n):
    """Rows the q4 format holds exactly: per 16-group a power-of-two scale s
    and e2m1 multiples of s with one +-6 s (so amax / 6 == s)."""
    s = np.exp2(rng.integers(-6, 4, size=(n, 8))).astype(np.float32)
    codes = rng.integers(0, 16, size=(n, 8, 16))
    codes[:, :, 0] = np.where(rng.random((n, 8)) < 0.5, 7, 15)  # +-6
    vals = N.e2m1_decode(codes) * s[:, :, None]
    return vals.reshape(n, 128).astype(np.float32)


def test_stage_pages_identity_on_representable_rows():
    rng = np.random.default_rng(5)
    H, nb = 3, 4
    rows = _representable_rows(rng, nb * 2 * H * 128).reshape(nb, 2 * H, 128, 128)
    pool = np.stack([np.stack([N.pack_slot(rows[p, sl], sl % 2) for sl in range(2 * H)])
                     for p in range(nb)])
    pages = np.array([2, 0, 3, 2])
    st = N.stage_pages(pool, pages)
    assert st.shape == (5, H, 128, 256) and not st[4].any()
    as_f = (st.astype(np.uint32) << 16).view(np.float32)
    for r, pg in enumerate(pages):
        assert np.array_equal(as_f[r, :, :, :128], rows[pg, 0::2])   # K slots 2h
        assert np.array_equal(as_f[r, :, :, 128:], rows[pg, 1::2])   # V slots 2h+1


def test_stage_pages_layout_matches_reference_test():
    """Reference tests/test_minimax_q4kv.py:560-581: staged[row, :, :, :128]
    is the K page and [..., 128:] the V page, in bf16; the last row is zero;
    capacity rows beyond n + 1 stay zero; an id outside the pool stages
    zeros."""
    rng = np.random.default_rng(6)
    H, nb = 2, 3
    x = N.bf16_round(rng.standard_normal((nb, 2 * H, 128, 128)).astype(np.float32))
    pool = np.stack([np.stack([N.pack_slot(x[p, sl], sl % 2) for sl in range(2 * H)])
                     for p in range(nb)])
    vals = N.dequant_pool(pool)
    st = N.stage_pages(pool.reshape(nb, 2 * H, 128, 72), [1, 7, 0], capacity=6)
    assert st.shape == (6, H, 128, 256)
    as_f = (st.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(as_f[0, :, :, :128], vals[1, 0::2])
    assert np.array_equal(as_f[0, :, :, 128:], vals[1, 1::2])
    assert np.array_equal(as_f[2, :, :, 128:], vals[0, 1::2])
    assert not st[1].any() and not st[3:].any()


def test_stage_pages_planted_side_swap_is_caught():
    """A staging that puts the V slot first fails the identity check."""
    rng = np.random.default_rng(7)
    rows = _representable_rows(rng, 2 * 128).reshape(1, 2, 128, 128)
    pool = np.stack([np.stack([N.pack_slot(rows[0, sl], sl % 2) for sl in range(2)])])
    st = N.stage_pages(pool, [0])
    swapped = np.concatenate([st[..., 128:], st[..., :128]], axis=-1)
    as_f = (swapped.astype(np.uint32) << 16).view(np.float32)
    assert not np.array_equal(as_f[0, 0, :, :128], rows[0, 0])
