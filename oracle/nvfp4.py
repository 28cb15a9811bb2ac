"""CPU oracle of the reference's NVFP4 ("q4") paged KV cache -- TEST
INFRASTRUCTURE ONLY (imported by ``tests/`` as the checker; the product
package never imports it).

A numpy restatement of ``src/vllm_exl3/minimax_q4kv_reference.py`` (paths
relative to the vllm-exl3 repository root):

* pool geometry: 128-token pages, container ``[pages, 2*Hkv, 128, 72]``;
  slot ``2h + side`` (K side 0, V side 1) is a flat 9216-byte region: data
  ``[128 tokens][64 B]`` then scales ``[1024 B]`` (``:7-24, 51-75``);
* scale offsets: K linear ``t*8+g``, V 4x4 token-quad swizzle (``:77-90``);
* e4m3 satfinite RNE encoder (``:179-220``) and decoder (``:157-170``);
* e2m1 RNE code ladder with its tie rules (``:226-244``) and decoder
  (``:140-154``);
* RZ of the exact product at fp32 precision (``:256-294``);
* row pack / unpack (``:297-349``), slot-region pack (``:352-366``), pool
  dequant (``:735-776``) and the bf16 prefill staging rows built from it
  (``q4_stage_pages``, ``minimax_q4kv_kernels.py:509-566, 880-951``);
* block-sparse decode attention over top-k pages with the causal rule of
  the decode kernel (``minimax_q4kv_kernels.py:416-506``), in float64, with
  the union-of-blocks semantics of ``reference_sparse_attention``
  (``minimax_q4kv_reference.py:1566-1612``).

Pins: ``tests/test_oracle_nvfp4.py`` (the reference's own vectors and
properties, torch's float8_e4m3fn cast, and byte fixtures the reference
module wrote, ``tests/golden/``).
"""

from __future__ import annotations

import numpy as np

HEAD_DIM = 128
GROUP = 16
NUM_GROUPS = 8
DATA_BYTES = 64
SCALE_BYTES = 8
ROW_BYTES = 72
PAGE_TOKENS = 128
SLOT_REGION = PAGE_TOKENS * ROW_BYTES      # 9216
DATA_REGION = PAGE_TOKENS * DATA_BYTES     # 8192
E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def scale_offset(side: int, t, g):
    """Offset inside a slot's 1024-byte scale block (``:77-90``)."""
    t = np.asarray(t)
    g = np.asarray(g)
    if side == 0:
        return t * SCALE_BYTES + g
    return ((t // 4) * 4 + g // 2) * SCALE_BYTES + (g % 2) * 4 + t % 4


def e4m3_decode(b) -> np.ndarray:
    """e4m3fn bytes -> float32; 0x7F / 0xFF are NaN (``:157-170``)."""
    b = np.asarray(b).astype(np.int64) & 0xFF
    e = (b >> 3) & 0xF
    m = b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (m + 8.0) * np.exp2(e - 10.0))
    v = np.where((b & 0x7F) == 0x7F, np.nan, v)
    return np.where(b & 0x80, -v, v).astype(np.float32)


def e4m3_encode(x) -> np.ndarray:
    """float32 -> e4m3fn byte, saturating round-to-nearest-even; NaN -> 0x7F
    with its sign (``:179-220``)."""
    v = np.asarray(x, dtype=np.float32)
    sign = np.signbit(v)
    ax = np.where(np.isnan(v), np.float32(0), np.abs(v)).astype(np.float32)
    bits = ax.view(np.uint32).astype(np.int64)
    e8 = ((bits >> 23) & 0xFF) - 120
    man = bits & 0x7FFFFF
    m3 = man >> 20
    rest = man & 0xFFFFF
    up = (rest > 0x80000) | ((rest == 0x80000) & ((m3 & 1) == 1))
    m3 = m3 + up
    carry = m3 == 8
    m3 = np.where(carry, 0, m3)
    e8 = e8 + carry
    normal = (e8 << 3) | m3
    normal_ok = (e8 >= 1) & (e8 <= 15) & ~((e8 == 15) & (m3 == 7))
    # subnormal candidate (only used where e8 <= 0, i.e. ax < 2^-6)
    t = np.where(ax < 1.0, ax.astype(np.float64) * 512.0, 0.0)  # exact scaling
    fl = np.floor(t)
    frac = t - fl
    inc = (frac > 0.5) | ((frac == 0.5) & ((fl.astype(np.int64) & 1) == 1))
    sub = (fl + inc).astype(np.int64)        # 8 carries into the smallest normal, code 0x08
    is_sub = e8 <= 0
    code = np.where(is_sub, sub, normal)
    ok = np.where(is_sub, True, normal_ok)
    code = np.where(ok, code, 0x7E)
    code = np.where(np.isnan(v), 0x7F, code)
    return ((code | (sign.astype(np.int64) << 7)) & 0xFF).astype(np.uint8)


def e2m1_code(mag) -> np.ndarray:
    """Saturating RNE e2m1 code 0..7 of |q| with the reference's tie rules;
    NaN -> 7 (``:226-244``)."""
    a = np.asarray(mag, dtype=np.float32)
    c = ((a > 0.25).astype(np.uint8) + (a >= 0.75) + (a > 1.25) + (a >= 1.75)
         + (a > 2.5) + (a >= 3.5) + (a > 5.0)).astype(np.uint8)
    return np.where(np.isnan(a), np.uint8(7), c).astype(np.uint8)


def e2m1_decode(n) -> np.ndarray:
    n = np.asarray(n).astype(np.int64) & 0xF
    v = np.asarray(E2M1_VALUES, dtype=np.float32)[n & 7]
    return np.where(n & 8, -v, v).astype(np.float32)


def rz_product(x, r) -> np.ndarray:
    """Round-toward-zero at fp32 of the exact product x*r (``:256-294``):
    the fp32 RN product, stepped one fp32 value toward zero when it landed
    farther from zero than the exact (float64) product."""
    x = np.asarray(x, dtype=np.float32)
    r = np.asarray(r, dtype=np.float32)
    p = (x * r).astype(np.float32)
    exact = x.astype(np.float64) * r.astype(np.float64)
    away = (p.astype(np.float64) - exact) * np.sign(exact) > 0
    step = np.nextafter(p, np.float32(0)).astype(np.float32)
    return np.where(away & np.isfinite(p), step, p).astype(np.float32)


def bf16_round(x) -> np.ndarray:
    """float32 values rounded to bfloat16 (RNE), returned as float32."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    b = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = b.view(np.float32)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def pack_row(x) -> tuple[np.ndarray, np.ndarray]:
    """[..., 128] -> ([..., 64] data bytes, [..., 8] e4m3 scale bytes)
    (``pack_q4_row``, ``:297-326``)."""
    x = np.asarray(x, dtype=np.float32)
    xb = bf16_round(x)
    g = xb.reshape(*x.shape[:-1], NUM_GROUPS, GROUP)
    absx = np.where(np.isnan(g), np.float32(0), np.abs(g)).astype(np.float32)
    amax = absx.max(axis=-1)
    s = np.maximum((amax / np.float32(6.0)).astype(np.float32), np.float32(2.0 ** -9))
    sb = e4m3_encode(s)
    sv = e4m3_decode(sb)
    recip = (np.float32(1.0) / sv).astype(np.float32)
    q = rz_product(g, recip[..., None])
    codes = e2m1_code(np.abs(q))
    signed = np.where(np.signbit(q), codes | 8, codes).astype(np.uint8)
    nib = np.where(codes == 0, 0, signed).astype(np.uint8).reshape(*x.shape[:-1], HEAD_DIM)
    data = (nib[..., 0::2] | (nib[..., 1::2] << 4)).astype(np.uint8)
    return data, sb


def unpack_row(data, scales) -> np.ndarray:
    """(``unpack_q4_row``, ``:329-349``)."""
    data = np.asarray(data, dtype=np.uint8)
    lo = e2m1_decode(data & 0xF)
    hi = e2m1_decode(data >> 4)
    vals = np.stack((lo, hi), axis=-1).reshape(*data.shape[:-1], HEAD_DIM)
    sc = np.repeat(e4m3_decode(scales), GROUP, axis=-1)
    return (vals * sc).astype(np.float32)


def pack_slot(rows, side: int) -> np.ndarray:
    """[128, 128] values of one slot -> flat uint8 [9216] (``:352-366``)."""
    data, sc = pack_row(rows)
    flat = np.zeros(SLOT_REGION, np.uint8)
    flat[:DATA_REGION] = data.reshape(-1)
    t, g = np.meshgrid(np.arange(PAGE_TOKENS), np.arange(NUM_GROUPS), indexing="ij")
    flat[DATA_REGION + scale_offset(side, t, g).reshape(-1)] = sc.reshape(-1)
    return flat


def unpack_slot(flat, side: int) -> np.ndarray:
    """flat uint8 [9216] -> [128, 128] float32 (``:369-382``)."""
    flat = np.asarray(flat, dtype=np.uint8)
    data = flat[:DATA_REGION].reshape(PAGE_TOKENS, DATA_BYTES)
    t, g = np.meshgrid(np.arange(PAGE_TOKENS), np.arange(NUM_GROUPS), indexing="ij")
    sc = flat[DATA_REGION + scale_offset(side, t, g)]
    return unpack_row(data, sc)


def pack_pages(k, v, seq_lens, block_table, num_pages: int) -> np.ndarray:
    """Pack K, V [B, Hkv, L, 128] into a pool uint8 [num_pages, 2*Hkv, 9216]:
    token p of sequence b lands in slot p % 128 of page block_table[b, p//128];
    positions past seq_lens[b] stay zero bytes."""
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    B, H, L, _ = k.shape
    pool = np.zeros((num_pages, 2 * H, SLOT_REGION), np.uint8)
    t_all, g_all = np.arange(PAGE_TOKENS), np.arange(NUM_GROUPS)
    for b in range(B):
        n = int(seq_lens[b])
        for blk in range((n + PAGE_TOKENS - 1) // PAGE_TOKENS):
            page = int(block_table[b, blk])
            t0, t1 = blk * PAGE_TOKENS, min(n, (blk + 1) * PAGE_TOKENS)
            for h in range(H):
                for side, x in ((0, k), (1, v)):
                    data, sc = pack_row(x[b, h, t0:t1])
                    reg = pool[page, 2 * h + side]
                    tt = np.arange(t1 - t0)
                    reg[:DATA_REGION].reshape(PAGE_TOKENS, DATA_BYTES)[tt] = data
                    off = scale_offset(side, tt[:, None], g_all[None, :])
                    reg[DATA_REGION + off.reshape(-1)] = sc.reshape(-1)
    del t_all
    return pool


def dequant_pool(pool) -> np.ndarray:
    """uint8 [pages, 2*Hkv, 9216] -> float32 [pages, 2*Hkv, 128, 128]
    (``dequant_pool_pages``, ``:735-776``)."""
    pool = np.asarray(pool, dtype=np.uint8)
    P, S, _ = pool.shape
    out = np.empty((P, S, PAGE_TOKENS, HEAD_DIM), np.float32)
    for p in range(P):
        for s in range(S):
            out[p, s] = unpack_slot(pool[p, s], s % 2)
    return out


def bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, RNE; NaN -> 0x7FC0 (torch's scalar
    float -> bfloat16 cast)."""
    x = np.asarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r).astype(np.uint16)


def stage_pages(pool, pages, capacity: int | None = None) -> np.ndarray:
    """Prefill staging (``q4_stage_pages``, ``minimax_q4kv_kernels.py:880-951``,
    kernel ``:509-566``): bf16 bits [capacity or n+1, Hkv, 128, 256]; row r
    < n holds page pages[r] -- the bf16 cast of ``dequant_pool`` with the K
    slot (2h) in columns 0..127 and the V slot (2h+1) in 128..255 -- and every
    other row is zero, as is a row whose page id is outside [0, nb) (this
    build's definition; the reference kernel does not bound the id)."""
    pool = np.asarray(pool, dtype=np.uint8)
    nb, slots = pool.shape[:2]
    pool = pool.reshape(nb, slots, SLOT_REGION)
    H = slots // 2
    pages = np.asarray(pages, dtype=np.int64).reshape(-1)
    n = pages.size
    rows = n + 1 if capacity is None else capacity
    out = np.zeros((rows, H, PAGE_TOKENS, 2 * HEAD_DIM), np.uint16)
    for r, pg in enumerate(pages):
        if 0 <= pg < nb:
            vals = dequant_pool(pool[pg:pg + 1])[0]          # [2H, 128, 128]
            out[r, :, :, :HEAD_DIM] = bf16_bits(vals[0::2])
            out[r, :, :, HEAD_DIM:] = bf16_bits(vals[1::2])
    return out


def sparse_decode(q, kv_vals, topk_idx, block_table, seq_lens, decode_query_len: int,
                  sm_scale: float) -> np.ndarray:
    """Block-sparse decode attention in float64.

    q [total_q, H, 128]; kv_vals [pages, 2*Hkv, 128, 128] (dequantised
    pool); topk_idx [Hkv, total_q, topk] logical block ids (entries outside
    [0, n_blocks) are skipped); query token i belongs to request
    i // decode_query_len at position seq_len - decode_query_len + offset and
    attends to the union of its KV head's listed blocks, causally
    (``minimax_q4kv_kernels.py:416-506``; union semantics of
    ``reference_sparse_attention``, ``minimax_q4kv_reference.py:1566-1612``).
    A query with no visible token yields zeros."""
    q = np.asarray(q, dtype=np.float64)
    total_q, Hq, D = q.shape
    Hkv = topk_idx.shape[0]
    G = Hq // Hkv
    out = np.zeros((total_q, Hq, D), np.float64)
    for i in range(total_q):
        req, off = divmod(i, decode_query_len)
        pos = int(seq_lens[req]) - decode_query_len + off
        kv_len = max(pos + 1, 0)
        n_blocks = (kv_len + PAGE_TOKENS - 1) // PAGE_TOKENS
        for h in range(Hkv):
            blocks = sorted({int(b) for b in topk_idx[h, i] if 0 <= int(b) < n_blocks})
            ks, vs = [], []
            for blk in blocks:
                page = int(block_table[req, blk])
                n = min(PAGE_TOKENS, kv_len - blk * PAGE_TOKENS)
                ks.append(kv_vals[page, 2 * h, :n])
                vs.append(kv_vals[page, 2 * h + 1, :n])
            if not ks:
                continue
            K = np.concatenate(ks).astype(np.float64)
            V = np.concatenate(vs).astype(np.float64)
            s = q[i, h * G:(h + 1) * G] @ K.T * sm_scale
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[i, h * G:(h + 1) * G] = p @ V
    return out


# ---------------------------------------------------------------------------
# W1 write side: Gemma QK-norm + partial NeoX RoPE + q4 pack-insert
# (``reference_w1_write``, ``minimax_q4kv_reference.py:422-612``)
# ---------------------------------------------------------------------------

def sumsq_tree(x) -> np.ndarray:
    """Sum of squares over the last axis (128) in one fixed fp32 order:
    adjacent pairs (2i, 2i+1) first, then a balanced tree over the 64 pair
    sums in index order.  The reference reduces with ``torch.sum``, whose
    order is unspecified; this order is the one the GPU kernel uses (a
    butterfly over lanes that hold dims 2l, 2l+1), so the oracle pins the
    kernel bit for bit and the reference within fp32 reduction rounding."""
    x = np.asarray(x, dtype=np.float32)
    sq = (x * x).astype(np.float32)
    p = (sq[..., 0::2] + sq[..., 1::2]).astype(np.float32)
    while p.shape[-1] > 1:
        p = (p[..., 0::2] + p[..., 1::2]).astype(np.float32)
    return p[..., 0]


def gemma_rmsnorm(x, w, eps: float, sumsq=sumsq_tree) -> np.ndarray:
    """``x * (1 / sqrt(mean(x^2) + eps)) * (1 + w)`` in fp32, each operation
    rounded once, left to right (``gemma_rmsnorm``, ``:422-432``)."""
    x = np.asarray(x, dtype=np.float32)
    ss = sumsq(x).astype(np.float32)
    d = (ss / np.float32(HEAD_DIM) + np.float32(eps)).astype(np.float32)
    r = (np.float32(1.0) / np.sqrt(d).astype(np.float32)).astype(np.float32)
    w1 = (np.float32(1.0) + np.asarray(w, dtype=np.float32)).astype(np.float32)
    return ((x * r[..., None]).astype(np.float32) * w1).astype(np.float32)


def rope_partial_neox(x, cos_sin_rows, rotary_dim: int) -> np.ndarray:
    """Rotate the first ``rotary_dim`` dims of each 128-row: pairs (i, i+half)
    as y[i] = x[i] c[i] - x[i+half] s[i], y[i+half] = x[i+half] c[i] +
    x[i] s[i], the rest unchanged (``rope_partial_neox``, ``:435-464``).
    ``cos_sin_rows`` [..., rotary_dim] = [cos | sin], broadcast over heads."""
    x = np.asarray(x, dtype=np.float32)
    half = rotary_dim // 2
    d = np.arange(HEAD_DIM)
    in_rope = d < rotary_dim
    ci = np.where(d < half, d, d - half).clip(0, max(half - 1, 0))
    partner = np.where(in_rope, np.where(d < half, d + half, d - half), d)
    cs = np.asarray(cos_sin_rows, dtype=np.float32)
    c = cs[..., ci]
    s = cs[..., (ci + half).clip(0, rotary_dim - 1)]
    while c.ndim < x.ndim:
        c, s = c[..., None, :], s[..., None, :]
    px = x[..., partner]
    t1 = (x * c).astype(np.float32)
    t2 = (px * s).astype(np.float32)
    rot = np.where(d < half, t1 - t2, t1 + t2).astype(np.float32)
    return np.where(in_rope, rot, x).astype(np.float32)


def e4m3_clamped(x) -> np.ndarray:
    """e4m3 bytes of clamp(x, +-448), NaN -> -448 (``_e4m3_clamped``,
    ``:613-617``)."""
    v = np.asarray(x, dtype=np.float32)
    v = np.where(np.isnan(v), np.float32(-448.0), v)
    return e4m3_encode(np.clip(v, -448.0, 448.0).astype(np.float32))


def w1_write(qkv, q_norm_w, k_norm_w, iq_norm_w, ik_norm_w, cos_sin, positions, eps: float,
             rotary_dim: int, nq: int, nkv: int, niq: int, slot_mapping, index_slot_mapping,
             pool, index_cache, sumsq=sumsq_tree) -> dict:
    """``reference_w1_write`` (``:467-578``) writing into existing buffers:
    ``pool`` uint8 [pages, 2*nkv, 9216] and ``index_cache`` uint8 [rows, 128]
    are updated in place at the mapped slots (-1 skips); returns q (bf16
    values as float32), index_q bytes and the processed K / index-K rows
    (bf16 values, the rows the reference kernel writes back into qkv)."""
    x = np.asarray(qkv, dtype=np.float32).reshape(len(qkv), -1, HEAD_DIM)
    T = x.shape[0]
    cs = np.asarray(cos_sin, dtype=np.float32)[np.asarray(positions, dtype=np.int64)][:, :rotary_dim]

    def proc(sl, w):
        return rope_partial_neox(gemma_rmsnorm(sl, w, eps, sumsq), cs, rotary_dim)

    q = bf16_round(proc(x[:, :nq], q_norm_w))
    kn = bf16_round(proc(x[:, nq:nq + nkv], k_norm_w))
    vb = bf16_round(x[:, nq + nkv:nq + 2 * nkv])
    sm = np.asarray(slot_mapping, dtype=np.int64)
    for i in range(T):
        if sm[i] < 0:
            continue
        page, t = int(sm[i] // PAGE_TOKENS), int(sm[i] % PAGE_TOKENS)
        for h in range(nkv):
            for side, rows in ((0, kn), (1, vb)):
                data, sc = pack_row(rows[i, h])
                region = pool[page, 2 * h + side]
                region[t * DATA_BYTES:(t + 1) * DATA_BYTES] = data
                for g in range(NUM_GROUPS):
                    region[DATA_REGION + scale_offset(side, t, g)] = sc[g]
    out = {"q": q, "k_rows": kn}
    if niq:
        lo = nq + 2 * nkv
        iq = proc(x[:, lo:lo + niq], iq_norm_w)
        out["index_q"] = e4m3_encode(bf16_round(iq))
        ik = proc(x[:, lo + niq], ik_norm_w)
        out["ik_rows"] = bf16_round(ik)
        kb = e4m3_clamped(ik)
        ism = np.asarray(index_slot_mapping, dtype=np.int64)
        for i in range(T):
            if ism[i] >= 0:
                index_cache[ism[i]] = kb[i]
    return out
