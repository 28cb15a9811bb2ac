"""GPU parity of the reference's NVFP4 q4 KV cache (pack, pool dequant,
block-sparse decode attention).

Pack and dequant are checked bit-exact against the CPU oracle (itself pinned
to bytes the reference packer wrote); decode against the oracle's float64
block-sparse attention over the oracle-dequantised pool, relative L2 <= 2e-3."""

import math

import numpy as np
import pytest
import torch

import nvfp4 as N
from moe_util import rel_l2
from vllm_exl3_amd import nvfp4_kv as Q
from vllm_exl3_amd import synthetic as S

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _pool_bytes(pool):
    return pool.cpu().numpy().reshape(pool.size(0), pool.size(1), -1)


def _setup(gpu, seed, B, H, L, seq, n_pages, dtype=torch.bfloat16):
    k, v = S.kv_inputs(seed, B, H, L)
    max_blocks = (L + 127) // 128
    bt = S.block_table(seed + 1, B, max_blocks, n_pages)
    pool = Q.new_pool(n_pages, H, gpu)
    Q.pack_pages(torch.from_numpy(k).to(gpu).to(dtype), torch.from_numpy(v).to(gpu).to(dtype),
                 torch.tensor(seq, dtype=torch.int32, device=gpu), torch.from_numpy(bt).to(gpu), pool)
    return k, v, np.asarray(seq), bt, pool


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_pack_and_dequant_bit_exact(gpu, dtype):
    B, H, L = 2, 2, 300
    seq = [300, 129]
    k, v, seq, bt, pool = _setup(gpu, 7, B, H, L, seq, 8, dtype)
    # the oracle sees the same values the kernel read
    kd = torch.from_numpy(k).to(dtype).float().numpy()
    vd = torch.from_numpy(v).to(dtype).float().numpy()
    want = N.pack_pages(kd, vd, seq, bt, 8)
    assert np.array_equal(_pool_bytes(pool), want)
    vals = Q.dequant_pool_pages(pool).cpu().numpy()
    assert np.array_equal(vals, N.dequant_pool(want))


def test_pack_special_values(gpu):
    # saturation, the 2^-9 scale clamp, exact e2m1 ties, signed zeros, a NaN
    x = np.zeros((1, 1, 128, 128), np.float32)
    g = np.random.default_rng(3)
    x[0, 0, 0] = g.standard_normal(128) * 5000.0
    x[0, 0, 1] = g.standard_normal(128) * 1e-5
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
    for grp in range(8):
        x[0, 0, 2, 16 * grp] = 6.0
        x[0, 0, 2, 16 * grp + 1:16 * grp + 8] = mids
        x[0, 0, 2, 16 * grp + 8:16 * grp + 15] = -mids
    x[0, 0, 3] = -0.0
    x[0, 0, 4, 5] = np.nan
    x[0, 0, 4, 6:20] = 1.0
    x[0, 0, 5:] = g.standard_normal((123, 128))
    v = -x
    pool = Q.new_pool(1, 1, gpu)
    seq = np.array([128], np.int32)
    bt = np.zeros((1, 1), np.int32)
    Q.pack_pages(torch.from_numpy(x).to(gpu), torch.from_numpy(v).to(gpu),
                 torch.from_numpy(seq).to(gpu), torch.from_numpy(bt).to(gpu), pool)
    got, want = _pool_bytes(pool), N.pack_pages(x, v, seq, bt, 1)
    bad = np.argwhere(got != want)
    assert len(bad) == 0, [(tuple(b), int(got[tuple(b)]), int(want[tuple(b)])) for b in bad[:8]]


def _decode_case(gpu, seed, seqs, dql, Hq, Hkv, topk, q_dtype=torch.bfloat16):
    B = len(seqs)
    L = max(seqs)
    k, v, seq, bt, pool = _setup(gpu, seed, B, Hkv, L, seqs, B * ((L + 127) // 128) + 3)
    total_q = B * dql
    g = np.random.default_rng(seed + 5)
    tk = np.full((Hkv, total_q, topk), -1, np.int32)
    for i in range(total_q):
        req, off = divmod(i, dql)
        pos = seqs[req] - dql + off
        nb = (max(pos + 1, 0) + 127) // 128
        for h in range(Hkv):
            pick = g.permutation(nb)[:min(topk, nb)]
            if nb > 1 and h == 0:
                pick = pick[: max(1, len(pick) - 1)]  # leave a -1 slot
            tk[h, i, :len(pick)] = pick
    q = S.activations(seed + 9, total_q * Hq, 128).reshape(total_q, Hq, 128)
    return k, v, seq, bt, pool, tk, q


@pytest.mark.parametrize("seqs,dql,Hq,Hkv,topk", [
    ([300, 129, 700], 1, 16, 2, 4),
    ([513, 260], 2, 8, 1, 3),
    ([1000], 1, 64, 8, 8),
    ([130, 5], 1, 4, 4, 2),
])
def test_sparse_decode_vs_oracle(gpu, seqs, dql, Hq, Hkv, topk):
    k, v, seq, bt, pool, tk, q = _decode_case(gpu, 60 + topk + Hkv, seqs, dql, Hq, Hkv, topk)
    vals = N.dequant_pool(_pool_bytes(pool))
    scale = 1.0 / math.sqrt(128)
    want = N.sparse_decode(q, vals, tk, bt, seq, dql, scale)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu)
    Q.q4_sparse_decode(torch.from_numpy(q).to(gpu).bfloat16(), pool, torch.from_numpy(tk).to(gpu),
                       torch.from_numpy(bt).to(gpu), torch.tensor(seqs, dtype=torch.int32, device=gpu),
                       Hkv, scale, out, dql)
    assert rel_l2(out, want) <= TOL


def test_sparse_decode_graph_replay_and_errors(gpu):
    k, v, seq, bt, pool, tk, q = _decode_case(gpu, 90, [400, 300], 1, 16, 2, 4)
    qt = torch.from_numpy(q).to(gpu).bfloat16()
    tkt, btt = torch.from_numpy(tk).to(gpu), torch.from_numpy(bt).to(gpu)
    st = torch.tensor([400, 300], dtype=torch.int32, device=gpu)
    out = torch.empty(qt.shape, dtype=torch.bfloat16, device=gpu)
    Q.q4_sparse_decode(qt, pool, tkt, btt, st, 2, 0.1, out, 1)
    ref = out.clone()
    Q.q4_sparse_decode(qt, pool, tkt, btt, st, 2, 0.1, out, 1)
    assert torch.equal(out, ref)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        Q.q4_sparse_decode(qt, pool, tkt, btt, st, 2, 0.1, out, 1)
    for seed in (91, 92):
        qt.copy_(torch.from_numpy(S.activations(seed, 2 * 16, 128).reshape(2, 16, 128)))
        g.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(out)
        Q.q4_sparse_decode(qt, pool, tkt, btt, st, 2, 0.1, eager, 1)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    with pytest.raises(ValueError):
        Q.q4_sparse_decode(qt, pool, tkt, btt, st, 4, 0.1, out, 1)   # pool holds 2 KV heads
    with pytest.raises(ValueError):
        Q.q4_sparse_decode(qt[:, :, :64], pool, tkt, btt, st, 2, 0.1, out, 1)
    with pytest.raises(ValueError):
        Q.q4_sparse_decode(qt, pool.view(torch.int8), tkt, btt, st, 2, 0.1, out, 1)


# ---------------------------------------------------------------------------
# W1 write side: bit-exact against the oracle's norm/RoPE/pack restatement
# (the oracle uses the kernel's fixed fp32 reduction order; it is pinned to
# the closed forms and to the reference test's layout in test_oracle_nvfp4.py)
# ---------------------------------------------------------------------------

def _w1_case(gpu, seed, T, nq, nkv, niq, rot, n_pages, max_pos=4096, w_dtype=torch.float32):
    g = np.random.default_rng(seed)
    per = nq + 2 * nkv + (niq + 1 if niq else 0)
    qkv = N.bf16_round((g.standard_normal((T, per * 128)) * 0.5).astype(np.float32))
    ws = [N.bf16_round(g.standard_normal(128).astype(np.float32) * 0.5) for _ in range(4)]
    inv = 1.0 / (5e6 ** (np.arange(0, rot, 2) / rot))
    ang = np.outer(np.arange(max_pos), inv)
    cs = np.concatenate([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    pos = g.integers(0, max_pos, T).astype(np.int64)
    sm = g.permutation(n_pages * 128)[:T].astype(np.int64)
    sm[g.random(T) < 0.2] = -1
    ism = g.permutation(2 * T)[:T].astype(np.int64)
    ism[g.random(T) < 0.2] = -1
    return qkv, ws, cs, pos, sm, ism


@pytest.mark.parametrize("T, nq, nkv, niq, rot", [(5, 8, 4, 4, 64), (37, 6, 2, 0, 128),
                                                  (300, 48, 8, 2, 64), (64, 4, 1, 1, 8)])
def test_w1_insert_bit_exact(gpu, T, nq, nkv, niq, rot):
    n_pages, eps = 4, 1e-6
    qkv, ws, cs, pos, sm, ism = _w1_case(gpu, 100 + T, T, nq, nkv, niq, rot, n_pages)
    pool = np.zeros((n_pages, 2 * nkv, N.SLOT_REGION), np.uint8)
    icache = np.zeros((2 * T, 128), np.uint8)
    want = N.w1_write(qkv, *ws, cs, pos, eps, rot, nq, nkv, niq, sm, ism, pool, icache)

    d_qkv = torch.from_numpy(qkv).to(gpu).bfloat16()
    d_w = [torch.from_numpy(w).to(gpu) for w in ws]
    d_pool = Q.new_pool(n_pages, nkv, gpu)
    d_ic = torch.zeros((2 * T, 128), dtype=torch.uint8, device=gpu)
    q_out = torch.empty((T, nq * 128), dtype=torch.bfloat16, device=gpu)
    iq_out = torch.empty((T, max(niq, 1) * 128), dtype=torch.uint8, device=gpu)[:, :niq * 128]
    Q.q4_w1_insert(d_qkv, d_w[0], d_w[1], torch.from_numpy(cs).to(gpu), torch.from_numpy(pos).to(gpu),
                   nq, nkv, rot, eps, d_w[2] if niq else None, d_w[3] if niq else None, niq,
                   torch.from_numpy(sm).to(gpu), torch.from_numpy(ism).to(gpu), d_pool,
                   d_ic if niq else None, 128, q_out, iq_out.contiguous() if niq else None)
    torch.cuda.synchronize()
    bits = lambda t: t.cpu().view(torch.int16).numpy()
    wq = torch.from_numpy(want["q"].reshape(T, -1)).bfloat16()
    assert np.array_equal(bits(q_out), bits(wq)), "q"
    assert np.array_equal(_pool_bytes(d_pool), pool), "pool"
    # processed K (and index-K) rows written back into qkv; other rows unchanged
    back = torch.from_numpy(qkv).bfloat16().view(T, -1, 128).clone()
    back[:, nq:nq + nkv] = torch.from_numpy(want["k_rows"]).bfloat16()
    if niq:
        back[:, -1] = torch.from_numpy(want["ik_rows"]).bfloat16()
        assert np.array_equal(d_ic.cpu().numpy(), icache), "index_k"
    assert np.array_equal(bits(d_qkv.view(T, -1, 128)), bits(back)), "qkv write-back"


def test_w1_insert_index_q_bytes(gpu):
    # index_q bytes: e4m3(bf16(v)) of the processed index_q rows
    T, nq, nkv, niq, rot = 9, 2, 1, 3, 64
    qkv, ws, cs, pos, sm, ism = _w1_case(gpu, 7, T, nq, nkv, niq, rot, 1)
    pool = np.zeros((1, 2, N.SLOT_REGION), np.uint8)
    icache = np.zeros((2 * T, 128), np.uint8)
    want = N.w1_write(qkv, *ws, cs, pos, 1e-6, rot, nq, nkv, niq, sm, ism, pool, icache)
    d_w = [torch.from_numpy(w).to(gpu) for w in ws]
    iq_out = torch.zeros((T, niq * 128), dtype=torch.uint8, device=gpu)
    Q.q4_w1_insert(torch.from_numpy(qkv).to(gpu).bfloat16(), d_w[0], d_w[1],
                   torch.from_numpy(cs).to(gpu), torch.from_numpy(pos).to(gpu), nq, nkv, rot, 1e-6,
                   d_w[2], d_w[3], niq, torch.from_numpy(sm).to(gpu), torch.from_numpy(ism).to(gpu),
                   Q.new_pool(1, nkv, gpu), torch.zeros((2 * T, 128), dtype=torch.uint8, device=gpu),
                   128, torch.empty((T, nq * 128), dtype=torch.bfloat16, device=gpu), iq_out)
    assert np.array_equal(iq_out.cpu().numpy().reshape(T, niq, 128), want["index_q"])
