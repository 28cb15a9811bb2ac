"""CPU checks of the int4 paged KV oracle (format defined in this build).

Pins: the page layout is a bijection onto its byte regions; quantisation
matches an element-by-element restatement of the rule and the closed-form
error bound; pack -> unpack equals quantise -> dequantise on ragged batches
with random block tables; the float64 attention reduces to closed forms."""

import numpy as np
import pytest

import oracle as O
from vllm_exl3_amd import synthetic as S


def test_page_layout_is_a_bijection():
    t, d = np.meshgrid(np.arange(16), np.arange(128), indexing="ij")
    kb = O.kv_k_nibble_bit(t, d).ravel()
    vb = O.kv_v_nibble_bit(t, d).ravel()
    assert np.array_equal(np.sort(kb), np.arange(0, 1024 * 8, 4))
    assert np.array_equal(np.sort(vb), np.arange(1024 * 8, 2048 * 8, 4))
    assert O.KV_PAGE_BYTES == 2560 and O.KV_PAGE_BYTES // 16 == 160  # bytes per token


def test_k_layout_lane_words():
    # lane l = t + 16 j holds dims 32 g + 8 j + p of token t in word g, nibble p
    for t, d in [(0, 0), (15, 127), (3, 40), (9, 77)]:
        g, r = divmod(d, 32)
        j, p = divmod(r, 8)
        assert O.kv_k_nibble_bit(t, d) == (16 * (t + 16 * j) + 4 * g) * 8 + 4 * p


def _quantise_scalar(row):
    """Element-by-element restatement of the quantisation rule."""
    row = [np.float32(x) for x in row]
    mn, mx = min(row), max(row)
    z = np.float16(mn)
    s = np.float16(np.float32(np.float32(mx - mn) / np.float32(15.0)))
    q = []
    for x in row:
        if np.float32(s) > 0:
            c = np.rint(np.float32(np.float32(x - np.float32(z)) / np.float32(s)))
        else:
            c = 0.0
        q.append(int(min(max(c, 0), 15)))
    return q, s, z


def test_quantise_matches_scalar_rule_and_error_bound():
    g = np.random.default_rng(5)
    rows = g.standard_normal((40, 128)).astype(np.float32)
    rows[3] = 1.25          # constant groups: scale 0, code 0, exact
    rows[4, :32] = 0.0
    rows[5] *= 100.0
    q, s, z = O.kv_quantize_rows(rows)
    for r in range(rows.shape[0]):
        for gi in range(4):
            qq, ss, zz = _quantise_scalar(rows[r, 32 * gi:32 * gi + 32])
            assert list(q[r, 32 * gi:32 * gi + 32]) == qq
            assert s[r, gi] == ss and z[r, gi] == zz
    x = O.kv_dequantize_rows(q, s, z)
    sf = np.repeat(s.astype(np.float32), 32, axis=-1)
    zf = np.repeat(z.astype(np.float32), 32, axis=-1)
    # |x - deq| <= s/2 + the fp16 rounding of zero and scale (|z| 2^-11, 15 s 2^-11)
    bound = sf / 2 + np.abs(zf) * 2.0 ** -10 + 15 * sf * 2.0 ** -10 + 1e-6
    assert np.all(np.abs(rows - x) <= bound)
    assert np.array_equal(x[3], rows[3]) and np.all(x[4, :32] == 0)


def test_pack_unpack_round_trip_ragged():
    B, H, L = 3, 2, 53
    k, v = S.kv_inputs(7, B, H, L)
    seq = np.array([53, 16, 1], dtype=np.int32)
    bt = S.block_table(8, B, 4, 20)
    pool = O.kv_pack_pages(k, v, seq, bt, 20)
    kk, vv = O.kv_unpack_pages(pool, seq, bt, L)
    for b in range(B):
        n = seq[b]
        for src, got in ((k, kk), (v, vv)):
            q, s, z = O.kv_quantize_rows(src[b, :, :n])
            assert np.array_equal(got[b, :, :n], O.kv_dequantize_rows(q, s, z))
            assert np.all(got[b, :, n:] == 0)
    # pages nobody uses stay zero; past-the-end slots of a last page are zero
    used = {int(bt[b, p]) for b in range(B) for p in range((seq[b] + 15) // 16)}
    for pg in range(20):
        if pg not in used:
            assert not pool[pg].any()
    q, s, z = O.kv_unpack_page(pool[bt[2, 0], 1], 1)
    assert not q[1:].any() and not s[1:].any() and not z[1:].any()


def test_attention_closed_forms():
    g = np.random.default_rng(3)
    B, Hq, Hkv, L, D = 2, 4, 2, 9, 128
    q = g.standard_normal((B, Hq, D))
    v = g.standard_normal((B, Hkv, L, D))
    k = np.repeat(g.standard_normal((B, Hkv, 1, D)), L, axis=2)  # identical keys
    o = O.attention_decode(q, k, v, 0.1)
    want = np.repeat(v.mean(axis=2), Hq // Hkv, axis=1)
    assert np.allclose(o, want, atol=1e-12)
    o1 = O.attention_decode_lens(q, g.standard_normal((B, Hkv, L, D)), v, np.array([1, 0]), 0.1)
    assert np.allclose(o1[0], np.repeat(v[0, :, 0], Hq // Hkv, axis=0)) and not o1[1].any()
